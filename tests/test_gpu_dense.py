"""The two-pass path on the GPU: the weight dequantized into the workspace, then hipBLASLt.

This is the reference's own computation (``QuantLinear._dequantized_weight`` then ``F.linear``,
src/llmopt/quantization/quant_linear.py:93-113), with the dense weight rebuilt in the workspace
by every call. ``llmopt_q_linear`` takes it from 1024 tokens (65 with fp32 activations);
``LLMOPT_ALGO_DENSE`` takes it at any size.

* Small shapes, every storage format, each compute dtype, with and without bias: against the
  reference's sequence on the host (oracle dequantization, rounding to the compute dtype,
  ``F.linear``), within 1e-2 (16-bit) / 2e-3 (fp32) of max|y_ref|.
* The automatic choice from 1024 tokens returns exactly what ``LLMOPT_ALGO_DENSE`` returns
  (the same two launches), and stays within the bound of the fused GEMM's result.
* fp32 activations against the product in float64: within 2e-5, the fp32 bound (the dense fp32
  weight is exact, hipBLASLt accumulates in fp32).
* Strided rows and leading dimensions; the SwiGLU product from the two-pass path through the
  combining kernel; correct results after the plan cache has been emptied and refilled.
"""

from __future__ import annotations

import pytest
import torch

from llmopt.kernels import _lib, ops
from llmopt.kernels._lib import ALGO_AUTO, ALGO_DENSE, ALGO_PREFILL
from llmopt.quantization import QuantizedTensor, RoundToNearestQuantizer, dequantize, interleave_gate_up
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu
DEV = "cuda"
NP_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}
TOL = {torch.float32: 2e-3, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _host_qt(rows, cols, bits, group, symmetric, seed):
    w = torch.randn(rows, cols, generator=torch.Generator().manual_seed(seed)) * 0.02
    return RoundToNearestQuantizer(bits, group, symmetric).quantize(w)


def _to_device(qt):
    return QuantizedTensor(qt.qweight.to(DEV), qt.scales.to(DEV), qt.zeros.to(DEV), qt.bits, qt.group_size,
                           qt.symmetric, qt.shape)


def _oracle_dense(qt):
    return qo.dequantize(qt.qweight.cpu().numpy(), qt.scales.cpu().numpy(), qt.zeros.cpu().numpy(), qt.bits,
                         qt.group_size, qt.symmetric, qt.shape)


def _reference(x, qt, bias, dtype):
    w = torch.from_numpy(qo.round_to_dtype(_oracle_dense(qt), NP_NAMES[dtype])).to(dtype)
    return qo.reference_linear(x, w, bias)


def _rel(y, ref):
    y, ref = y.detach().double().cpu(), ref.detach().double().cpu()
    d = float(ref.abs().max())
    return float((y - ref).abs().max()) / (d if d > 0 else 1.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bits,symmetric", [(4, False), (4, True), (8, False), (8, True), (2, False)])
@pytest.mark.parametrize("n,k,group", [(48, 256, 128), (200, 512, 64), (64, 176, 16), (96, 1024, 32),
                                       (80, 1024, 256)])
@pytest.mark.parametrize("m", [1, 7, 200])
@pytest.mark.parametrize("with_bias", [False, True])
def test_dense_small_shapes(dtype, bits, symmetric, n, k, group, m, with_bias):
    qt = _host_qt(n, k, bits, group, symmetric, seed=n + k + bits + group)
    gen = torch.Generator().manual_seed(m + n)
    x = torch.randn(m, k, generator=gen).to(dtype)
    bias = torch.randn(n, generator=gen).to(dtype) if with_bias else None
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None if bias is None else bias.to(DEV), dtype, algo=ALGO_DENSE)
    assert y.dtype == dtype and y.shape == (m, n)
    assert _rel(y, _reference(x, qt, bias, dtype)) <= TOL[dtype], (dtype, bits, n, k, m)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1024, 1500])
def test_auto_takes_the_two_pass_path_from_1024_tokens(dtype, m):
    n, k = 1536, 2048
    qt = _host_qt(n, k, 4, 128, False, seed=m)
    dqt = _to_device(qt)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(1)).to(dtype).to(DEV)
    auto = ops.quant_linear(x, dqt, None, dtype, algo=ALGO_AUTO)
    dense = ops.quant_linear(x, dqt, None, dtype, algo=ALGO_DENSE)
    fused = ops.quant_linear(x, dqt, None, dtype, algo=ALGO_PREFILL)
    assert torch.equal(auto.view(torch.int16), dense.view(torch.int16))
    assert _rel(auto, fused) <= TOL[dtype]
    rows = torch.arange(0, m, 97)
    assert _rel(auto[rows.to(DEV)], _reference(x[rows.to(DEV)].cpu(), qt, None, dtype)) <= TOL[dtype]


@pytest.mark.parametrize("m", [65, 300])
def test_fp32_two_pass_against_float64(m):
    n, k = 1024, 4096
    qt = _host_qt(n, k, 4, 64, True, seed=m)
    dqt = _to_device(qt)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(2)).to(DEV)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(3)).to(DEV)
    y = ops.quant_linear(x, dqt, bias, torch.float32)
    ref = x.double() @ dequantize(dqt, torch.float32).double().t() + bias.double()
    assert _rel(y, ref) <= 2e-5
    assert torch.equal(y, ops.quant_linear(x, dqt, bias, torch.float32, algo=ALGO_DENSE))


def test_strided_rows_and_leading_dims():
    n, k = 640, 2048
    qt = _host_qt(n, k, 4, 128, False, seed=5)
    dqt = _to_device(qt)
    base = torch.randn(2, 600, 2 * k, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(DEV)
    x = base[..., :k]  # rows with stride 2k, 1200 tokens
    y = ops.quant_linear(x, dqt, None, torch.bfloat16)
    assert y.shape == (2, 600, n)
    ref = _reference(x.reshape(-1, k).cpu(), qt, None, torch.bfloat16)
    assert _rel(y.reshape(-1, n), ref) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("m", [1024, 2000])
def test_swiglu_from_the_two_pass_product(m):
    inter, k = 768, 2048
    gate = _host_qt(inter, k, 4, 128, False, seed=9)
    up = _host_qt(inter, k, 4, 128, False, seed=10)
    fused = _to_device(interleave_gate_up(gate, up))
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16).to(DEV)
    y = ops.quant_linear_swiglu(x, fused, None, torch.bfloat16)
    g = ops.quant_linear(x, _to_device(gate), None, torch.bfloat16, algo=ALGO_DENSE).float()
    u = ops.quant_linear(x, _to_device(up), None, torch.bfloat16, algo=ALGO_DENSE).float()
    ref = torch.nn.functional.silu(g) * u
    assert y.shape == (m, inter)
    assert _rel(y, ref) <= 1e-2


def test_plan_cache_refill_keeps_results():
    # More distinct shapes than the plan cache holds (256): it is emptied and refilled, and a
    # shape seen before the refill still gives the same result.
    n, k = 128, 256
    qt = _host_qt(n, k, 4, 128, False, seed=11)
    dqt = _to_device(qt)
    x = torch.randn(300, k, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16).to(DEV)
    first = ops.quant_linear(x[:37], dqt, None, torch.bfloat16, algo=ALGO_DENSE)
    for m in range(1, 300):
        ops.quant_linear(x[:m], dqt, None, torch.bfloat16, algo=ALGO_DENSE)
    again = ops.quant_linear(x[:37], dqt, None, torch.bfloat16, algo=ALGO_DENSE)
    assert torch.equal(first.view(torch.int16), again.view(torch.int16))
    assert _rel(again, _reference(x[:37].cpu(), qt, None, torch.bfloat16)) <= TOL[torch.bfloat16]


def test_dense_without_its_workspace_is_refused():
    lib = _lib.load_library()
    n, k, m = 256, 512, 8
    qt = _to_device(_host_qt(n, k, 4, 128, False, seed=13))
    x = torch.randn(m, k).to(torch.bfloat16).to(DEV)
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    need = lib.llmopt_q_linear_dense_workspace(n, k, _lib.DTYPE_CODES[torch.bfloat16])
    assert need == n * k * 2 + (32 << 20)
    rc = lib.llmopt_q_linear_ex(x.data_ptr(), m, k, k, qt.qweight.data_ptr(), k // 2, qt.scales.data_ptr(),
                                qt.zeros.data_ptr(), None, y.data_ptr(), n, n, _lib.DTYPE_CODES[torch.bfloat16], 4,
                                128, 0, 0, None, 0, torch.cuda.current_stream().cuda_stream, ALGO_DENSE)
    assert rc == -4 and b"dense path" in lib.llmopt_q_last_error()
    torch.cuda.synchronize()
    assert bool(torch.isnan(y.float()).all())

"""fp32 activations on the GPU: the reference engine's own quantized configuration.

``LLMEngine.from_pretrained(quantize=True)`` quantizes a float32 model with
``quantize_model_(model, bits=4, group_size=64)`` (symmetric by default), and each
``QuantLinear`` computes in its layer's dtype (src/llmopt/engine/llm_engine.py:258-264,
quantization/quant_linear.py:199-201, model/modeling.py:57-58). Through the C ABI, fp32
activations are split exactly into three bf16 pieces that the decode kernels multiply, and the
pieces' fp32 sums are added with the bias.

* Against the reference's sequence on the host (oracle dequantization in fp32, ``F.linear`` in
  fp32): max|y - y_ref| / max|y_ref| <= 2e-3, the fp32 bound.
* Against the same product in float64 on the GPU: <= 2e-5. An fp32 result keeps fp32
  accuracy; rounding the activations or the weights to bf16 anywhere would put the error near
  2^-9 (about 2e-3) and fail this bound.
* The projections of the Llama-3-8B shapes at 1, 32 and 2048 tokens in that configuration;
  small shapes across widths, groups, symmetry and bias; the chunking of batches of more than
  21 tokens; the generic kernel when the workspace is missing; the fused SwiGLU in fp32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from llmopt.kernels import _lib, ops
from llmopt.quantization import QuantizedTensor, RoundToNearestQuantizer, dequantize, interleave_gate_up
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32_TOL = 2e-3
F64_TOL = 2e-5
PROJECTIONS = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (28672, 4096), "down": (4096, 14336)}


def _host_qt(rows, cols, bits, group, symmetric, seed):
    w = torch.randn(rows, cols, generator=torch.Generator().manual_seed(seed)) * 0.02
    return RoundToNearestQuantizer(bits, group, symmetric).quantize(w)


def _to_device(qt):
    return QuantizedTensor(qt.qweight.to(DEV), qt.scales.to(DEV), qt.zeros.to(DEV), qt.bits, qt.group_size,
                           qt.symmetric, qt.shape)


def _oracle_dense(qt):
    return qo.dequantize(qt.qweight.cpu().numpy(), qt.scales.cpu().numpy(), qt.zeros.cpu().numpy(), qt.bits,
                         qt.group_size, qt.symmetric, qt.shape)


def _rel(y, ref):
    y, ref = y.detach().double(), ref.detach().double().to(y.device)
    d = float(ref.abs().max())
    return float((y - ref).abs().max()) / (d if d > 0 else 1.0)


def _f64_reference(x_dev, dqt, bias=None):
    """The product in float64 on the GPU, over the fp32 dense weight (bit-exact dequantization)."""
    w = dequantize(dqt, torch.float32).double()
    y = x_dev.double() @ w.t()
    return y if bias is None else y + bias.double()


@pytest.fixture(scope="module")
def engine_projections():
    out = {}
    for i, (name, (n, k)) in enumerate(PROJECTIONS.items()):
        qt = _host_qt(n, k, 4, 64, True, seed=20 + i)
        out[name] = (qt, _to_device(qt))
    return out


@pytest.mark.parametrize("name", list(PROJECTIONS))
@pytest.mark.parametrize("m", [1, 2, 16, 32, 2048])
def test_engine_configuration_projections(engine_projections, name, m):
    # 4-bit symmetric groups of 64, fp32 compute: sampled columns (and, at 2048 tokens, rows)
    # against the reference's fp32 sequence on the host; every output against float64.
    qt, dqt = engine_projections[name]
    n, k = qt.shape
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m + n))
    xd = x.to(DEV)
    y = ops.quant_linear(xd, dqt, None, torch.float32)
    assert y.dtype == torch.float32 and y.shape == (m, n)
    assert _rel(y, _f64_reference(xd, dqt)) <= F64_TOL
    rng = np.random.default_rng(m + k)
    cols = np.sort(rng.choice(n, size=128, replace=False))
    rows = np.arange(m) if m <= 64 else np.sort(rng.choice(m, size=64, replace=False))
    w = torch.from_numpy(np.ascontiguousarray(_oracle_dense(qt)[cols]))
    ref = qo.reference_linear(x[torch.from_numpy(rows)], w, None)
    got = y[torch.from_numpy(rows).to(DEV)][:, torch.from_numpy(cols).to(DEV)].cpu()
    assert _rel(got, ref) <= F32_TOL


@pytest.mark.parametrize("bits,symmetric,group", [(4, True, 64), (4, False, 128), (4, True, 128), (2, False, 128),
                                                   (8, False, 128), (8, True, 64), (4, False, 32)])
@pytest.mark.parametrize("m", [1, 2, 5, 21, 22, 47, 100])
@pytest.mark.parametrize("with_bias", [False, True])
def test_small_shapes_every_format(bits, symmetric, group, m, with_bias):
    # Batches of 1-21 tokens are one chunk of piece rows; 22, 47 and 100 tokens run in chunks.
    n, k = 320, 1024
    qt = _host_qt(n, k, bits, group, symmetric, seed=bits * 100 + group + m)
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, k, generator=gen)
    bias = torch.randn(n, generator=gen) if with_bias else None
    dqt = _to_device(qt)
    y = ops.quant_linear(x.to(DEV), dqt, None if bias is None else bias.to(DEV), torch.float32)
    ref = qo.reference_linear(x, torch.from_numpy(_oracle_dense(qt)), bias)
    assert _rel(y.cpu(), ref) <= F32_TOL
    assert _rel(y, _f64_reference(x.to(DEV), dqt, None if bias is None else bias.to(DEV))) <= F64_TOL


def test_magnitudes_and_pieces():
    # Activations over many binades (tiny, huge, mixed in one row): the three pieces carry each
    # fp32 value exactly, so the relative accuracy does not depend on the scale of x.
    n, k = 256, 2048
    qt = _host_qt(n, k, 4, 128, False, seed=3)
    dqt = _to_device(qt)
    gen = torch.Generator().manual_seed(4)
    base = torch.randn(6, k, generator=gen)
    expo = torch.randint(-60, 60, (6, k), generator=gen).float()
    x = torch.cat([base * 1e-30, base * 1e30, base * torch.exp2(expo)], dim=0)
    xd = x.to(DEV)
    y = ops.quant_linear(xd, dqt, None, torch.float32)
    ref = _f64_reference(xd, dqt)
    for r in range(x.shape[0]):
        assert _rel(y[r], ref[r]) <= F64_TOL, r


def test_strided_and_leading_dims():
    n, k = 512, 2048
    qt = _host_qt(n, k, 4, 64, True, seed=5)
    dqt = _to_device(qt)
    base = torch.randn(2, 3, 2 * k, generator=torch.Generator().manual_seed(6)).to(DEV)
    x = base[..., :k]  # rows with stride 2k
    y = ops.quant_linear(x, dqt, None, torch.float32)
    assert y.shape == (2, 3, n)
    assert _rel(y.reshape(-1, n), _f64_reference(x.reshape(-1, k), dqt)) <= F64_TOL


def test_without_a_workspace_the_generic_kernel_runs():
    # Through the C ABI with no workspace: the generic kernel on the fp32 inputs, same bound.
    lib = _lib.load_library()
    n, k, m = 384, 1024, 4
    qt = _host_qt(n, k, 4, 64, True, seed=7)
    dqt = _to_device(qt)
    assert lib.llmopt_q_linear_workspace_ex(m, n, k, 4, 64, _lib.DTYPE_CODES[torch.float32]) >= 3 * m * k * 2
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(8)).to(DEV)
    y = torch.full((m, n), float("nan"), device=DEV)
    rc = lib.llmopt_q_linear(x.data_ptr(), m, k, k, dqt.qweight.data_ptr(), k // 2, dqt.scales.data_ptr(),
                             dqt.zeros.data_ptr(), None, y.data_ptr(), n, n, _lib.DTYPE_CODES[torch.float32], 4, 64,
                             1, 0, None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.llmopt_q_last_error()
    assert _rel(y, _f64_reference(x, dqt)) <= 1e-5
    assert _rel(y, ops.quant_linear(x, dqt, None, torch.float32)) <= 1e-5


@pytest.mark.parametrize("m", [1, 8, 40])
def test_swiglu_in_fp32(m):
    # The fused gate/up product in fp32: the product, then the combining kernel's SiLU * up.
    inter, k = 512, 1024
    gate = _host_qt(inter, k, 4, 64, True, seed=9)
    up = _host_qt(inter, k, 4, 64, True, seed=10)
    fused = _to_device(interleave_gate_up(gate, up))
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(DEV)
    y = ops.quant_linear_swiglu(x, fused, None, torch.float32)
    g = _f64_reference(x, _to_device(gate))
    u = _f64_reference(x, _to_device(up))
    ref = torch.nn.functional.silu(g) * u
    assert y.dtype == torch.float32 and y.shape == (m, inter)
    assert _rel(y, ref) <= 1e-4


@pytest.mark.parametrize("n,k", [(4096, 14336), (2048, 4096)])
@pytest.mark.parametrize("group,symmetric", [(64, True), (128, False)])
@pytest.mark.parametrize("m", [1, 2, 3, 6, 10])
@pytest.mark.parametrize("with_bias", [False, True])
def test_k_sliced_pieces(n, k, group, symmetric, m, with_bias):
    # One to ten fp32 tokens whose piece rows the K-sliced kernel splits over K (long rows from
    # one token, K = 4096 from 3 tokens in groups of 64 or 6 in groups of 128): the pieces, the
    # K-sliced kernel with its reduction into fp32 sums, then the combining kernel. One token on
    # the long rows in groups of 128 takes the one-shot kernel's eight-step chunks instead, the
    # split and the pieces' sum inside it.
    qt = _host_qt(n, k, 4, group, symmetric, seed=m + n + group)
    dqt = _to_device(qt)
    gen = torch.Generator().manual_seed(m + 100)
    x = torch.randn(m, k, generator=gen)
    bias = torch.randn(n, generator=gen) if with_bias else None
    xd = x.to(DEV)
    y = ops.quant_linear(xd, dqt, None if bias is None else bias.to(DEV), torch.float32)
    assert y.dtype == torch.float32 and y.shape == (m, n)
    assert _rel(y, _f64_reference(xd, dqt, None if bias is None else bias.to(DEV))) <= F64_TOL
    cols = np.sort(np.random.default_rng(m).choice(n, size=64, replace=False))
    w = torch.from_numpy(np.ascontiguousarray(_oracle_dense(qt)[cols]))
    ref = qo.reference_linear(x, w, None if bias is None else bias[torch.from_numpy(cols)])
    assert _rel(y[:, torch.from_numpy(cols).to(DEV)].cpu(), ref) <= F32_TOL

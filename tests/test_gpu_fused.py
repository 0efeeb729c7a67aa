"""Parity of the fused projections on the GPU, through the C ABI.

* ``llmopt_q_linear_swiglu`` (gate and up rows interleaved in blocks of four), two bounds:
  - against ``silu(gate) * up`` computed in float64 from the same rounded operands (oracle
    dequantization cast to the compute dtype, the activations in the compute dtype):
    max|y - y64| / max|y64| <= 1e-2, the bf16 bound of a single linear -- or, where the
    reference's own sequence is itself further from the exact value, no further than it plus one
    bf16 rounding step (2^-8). Both round gate, up, silu(gate) and the product to the compute
    dtype (src/llmopt/model/layers.py:44), four roundings of up to 2^-9 each, so both sit up to
    about 1e-2 from the exact value, and a gate or up value on the other side of a rounding
    boundary moves an output by a step;
  - against that reference sequence (``F.linear`` for gate and for up, then
    ``silu(gate) * up``, each step rounded to the compute dtype): <= 2e-2, since each side's
    distance from the exact value adds (seen together: 1.2e-2).
  The shapes cover the kernels with the activation in their epilogue (one-shot and multi-tile
  decode, the prefill GEMM unsplit and split), the two-pass path from 1024 tokens (product, then
  the combining kernel), and the workspace path for the others (8-bit codes, groups of 64).
* ``FusedQuantLinear``: each part of one launch equals the separate ``QuantLinear``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from llmopt.kernels import _lib, ops
from llmopt.quantization import (
    FusedQuantLinear,
    QuantLinear,
    QuantSwiGLU,
    QuantizedTensor,
    RoundToNearestQuantizer,
    dequantize,
    interleave_gate_up,
)
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu

DEV = "cuda"
NP_NAMES = {torch.float16: "float16", torch.bfloat16: "bfloat16"}
SWIGLU_TOL = 2e-2  # against the reference's sequence of four bf16 roundings
EXACT_TOL = 1e-2  # against the exact product of the rounded operands
STEP = 2.0**-8    # one bf16 rounding step, beyond the reference sequence's own distance


def _host_qt(rows, cols, bits, group, symmetric, seed):
    gen = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, cols, generator=gen) * 0.02
    return RoundToNearestQuantizer(bits, group, symmetric).quantize(w)


def _to_device(qt):
    return QuantizedTensor(qt.qweight.to(DEV), qt.scales.to(DEV), qt.zeros.to(DEV), qt.bits,
                           qt.group_size, qt.symmetric, qt.shape)


def _oracle_dense(qt):
    return qo.dequantize(qt.qweight.numpy(), qt.scales.numpy(), qt.zeros.numpy(), qt.bits,
                         qt.group_size, qt.symmetric, qt.shape)


def _rel_err(y, ref):
    y, ref = y.detach().float().cpu(), ref.detach().float().cpu()
    d = float(ref.abs().max())
    return float((y - ref).abs().max()) / (d if d > 0 else 1.0)


def _ref_linear(x, dense32, dtype, bias=None):
    w = torch.from_numpy(qo.round_to_dtype(dense32, NP_NAMES[dtype])).to(dtype)
    return qo.reference_linear(x, w, bias)


def _no_worse_than_reference(y, ref, exact):
    """The kernel is within EXACT_TOL of the exact product, or within the reference sequence's
    own distance plus one rounding step where that is larger."""
    e_hip, e_ref = _rel_err(y, exact), _rel_err(ref, exact)
    return e_hip <= max(EXACT_TOL, e_ref + STEP), (e_hip, e_ref)


def _fp32_swiglu(x, gate32, up32, dtype):
    """silu(x W_g^T) * (x W_u^T) in float64 on the host from the compute-dtype activations and
    the oracle's dense weights rounded to the compute dtype (the operands both sides use)."""
    xd = x.double()
    g = xd @ torch.from_numpy(qo.round_to_dtype(gate32, NP_NAMES[dtype])).double().t()
    u = xd @ torch.from_numpy(qo.round_to_dtype(up32, NP_NAMES[dtype])).double().t()
    return torch.nn.functional.silu(g) * u


def _gpu_fp32_swiglu(x, gate, up, dtype):
    """The same on the GPU in fp32 (float64 would take the slow path there), over the bit-exact
    device dequantization."""
    g = x.float() @ dequantize(gate, dtype).float().t().contiguous()
    u = x.float() @ dequantize(up, dtype).float().t().contiguous()
    return torch.nn.functional.silu(g) * u


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits,symmetric,group", [(4, False, 128), (4, True, 128), (2, False, 256),
                                                   (4, False, 64), (8, False, 128)])
@pytest.mark.parametrize("inter,k", [(64, 1024), (96, 512)])
@pytest.mark.parametrize("m", [1, 3, 8, 33, 64, 200, 300])
def test_swiglu_small_shapes(dtype, bits, symmetric, group, inter, k, m):
    gate = _host_qt(inter, k, bits, group, symmetric, seed=inter + k + bits)
    up = _host_qt(inter, k, bits, group, symmetric, seed=inter + k + bits + 1)
    fused = _to_device(interleave_gate_up(gate, up))
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(dtype)
    y = ops.quant_linear_swiglu(x.to(DEV), fused, None, dtype)
    g = _ref_linear(x, _oracle_dense(gate), dtype)
    u = _ref_linear(x, _oracle_dense(up), dtype)
    ref = torch.nn.functional.silu(g) * u
    assert y.shape == (m, inter) and y.dtype == dtype
    assert _rel_err(y, ref) <= SWIGLU_TOL, (dtype, bits, symmetric, group, inter, k, m)
    ok, errs = _no_worse_than_reference(y, ref, _fp32_swiglu(x, _oracle_dense(gate), _oracle_dense(up), dtype))
    assert ok, (errs, dtype, bits, symmetric, group, inter, k, m)


def test_swiglu_bias_and_leading_dims():
    dtype = torch.bfloat16
    gen = torch.Generator().manual_seed(7)
    lin_g, lin_u = nn.Linear(512, 64), nn.Linear(512, 64)
    with torch.no_grad():
        for lin in (lin_g, lin_u):
            lin.weight.copy_(torch.randn(64, 512, generator=gen) * 0.02)
            lin.bias.copy_(torch.randn(64, generator=gen) * 0.1)
    qg = RoundToNearestQuantizer(4, 128, False).quantize(lin_g.weight.detach())
    qu = RoundToNearestQuantizer(4, 128, False).quantize(lin_u.weight.detach())
    gate = QuantLinear.from_float(lin_g.to(dtype), qg, compute_dtype=dtype)
    up = QuantLinear.from_float(lin_u.to(dtype), qu, compute_dtype=dtype)
    fused_host = QuantSwiGLU(gate, up)
    fused_dev = QuantSwiGLU(gate, up).to(DEV)
    wg, wu = dequantize(qg, dtype).double(), dequantize(qu, dtype).double()
    for m in (1, 40, 300, 1100):
        x = torch.randn(2, m, 512, generator=gen).to(dtype)
        ref = fused_host(x)
        y = fused_dev(x.to(DEV))
        assert y.shape == (2, m, 64)
        assert _rel_err(y, ref) <= SWIGLU_TOL, m
        xd = x.double()
        exact = (torch.nn.functional.silu(xd @ wg.t() + gate.bias.double()) * (xd @ wu.t() + up.bias.double()))
        ok, errs = _no_worse_than_reference(y, ref, exact)
        assert ok, (errs, m)


@pytest.mark.parametrize("m", [2, 9, 24, 32])
def test_swiglu_k_sliced_single_slice(m):
    # K = 2048 over 128 fused tiles: the K-sliced kernel with one slice applies the activation
    # in its own epilogue.
    dtype = torch.bfloat16
    gate = _host_qt(1024, 2048, 4, 128, False, seed=m + 11)
    up = _host_qt(1024, 2048, 4, 128, False, seed=m + 12)
    fused = _to_device(interleave_gate_up(gate, up))
    x = torch.randn(m, 2048, generator=torch.Generator().manual_seed(m)).to(dtype)
    y = ops.quant_linear_swiglu(x.to(DEV), fused, None, dtype)
    ref = torch.nn.functional.silu(_ref_linear(x, _oracle_dense(gate), dtype)) * _ref_linear(x, _oracle_dense(up), dtype)
    assert y.shape == (m, 1024)
    assert _rel_err(y, ref) <= SWIGLU_TOL, m
    ok, errs = _no_worse_than_reference(y, ref, _fp32_swiglu(x, _oracle_dense(gate), _oracle_dense(up), dtype))
    assert ok, (errs, m)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("m", [1, 8, 16, 32, 40, 64, 2048, 16384])
def test_swiglu_llama_gate_up(m):
    dtype = torch.bfloat16
    inter, k = 14336, 4096
    gate = _to_device(_host_qt(inter, k, 4, 128, False, seed=1))
    up = _to_device(_host_qt(inter, k, 4, 128, False, seed=2))
    fused = interleave_gate_up(gate, up)
    x = torch.randn(m, k, device=DEV).to(dtype)
    y = ops.quant_linear_swiglu(x, fused, None, dtype)
    # GPU fp32 reference over the bit-exact dequantized weights (dequantize is checked
    # bit-exact against the oracle elsewhere), rounded like the reference's sequence.
    g = (x.float() @ dequantize(gate, dtype).float().t().contiguous()).to(dtype)
    u = (x.float() @ dequantize(up, dtype).float().t().contiguous()).to(dtype)
    ref = torch.nn.functional.silu(g.float()).to(dtype).float() * u.float()
    assert _rel_err(y, ref) <= SWIGLU_TOL
    ok, errs = _no_worse_than_reference(y, ref, _gpu_fp32_swiglu(x, gate, up, dtype))
    assert ok, errs


@pytest.mark.parametrize("m", [1, 5, 64, 300])
def test_fused_qkv_matches_separate(m):
    dtype = torch.bfloat16
    gen = torch.Generator().manual_seed(m)
    parts = []
    for i, n in enumerate((128, 32, 32)):
        lin = nn.Linear(1024, n, bias=False)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(n, 1024, generator=gen) * 0.02)
        qt = RoundToNearestQuantizer(4, 128, False).quantize(lin.weight.detach())
        parts.append(QuantLinear.from_float(lin.to(dtype), qt, compute_dtype=dtype).to(DEV))
    fused = FusedQuantLinear(parts)
    x = torch.randn(m, 1024, generator=gen).to(dtype).to(DEV)
    outs = fused(x)
    for o, p in zip(outs, parts):
        assert o.shape == (m, p.out_features)
        assert _rel_err(o, p(x)) <= 1e-2


def test_swiglu_rejects_bad_row_count():
    qt = _to_device(_host_qt(12, 256, 4, 128, False, seed=3))
    with pytest.raises(ValueError):
        ops.quant_linear_swiglu(torch.randn(2, 256, device=DEV).to(torch.bfloat16), qt, None, torch.bfloat16)


@pytest.mark.parametrize("m", [12, 32])
def test_swiglu_long_rows_over_k_slices(m):
    # Long rows on a small grid with the workspace the swiglu entry point asks for: the decode
    # kernel over K slices, whose reduction applies SiLU(gate) * up.
    dtype = torch.bfloat16
    inter, k = 2048, 14336  # 256 tiles of fused rows: 14 slices of K
    assert _lib.load_library().llmopt_q_linear_workspace(m, 2 * inter, k, 4, 128) > 0
    gate = _to_device(_host_qt(inter, k, 4, 128, False, seed=11))
    up = _to_device(_host_qt(inter, k, 4, 128, False, seed=12))
    fused = interleave_gate_up(gate, up)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(dtype).to(DEV)
    y = ops.quant_linear_swiglu(x, fused, None, dtype)
    g = (x.float() @ dequantize(gate, dtype).float().t().contiguous()).to(dtype)
    u = (x.float() @ dequantize(up, dtype).float().t().contiguous()).to(dtype)
    ref = torch.nn.functional.silu(g.float()).to(dtype).float() * u.float()
    assert _rel_err(y, ref) <= SWIGLU_TOL
    ok, errs = _no_worse_than_reference(y, ref, _gpu_fp32_swiglu(x, gate, up, dtype))
    assert ok, errs


def _swiglu_of_product(t: torch.Tensor, dtype) -> torch.Tensor:
    """The reference's SwiGLU (layers.py:44) on a fused [M, 2I] product in the compute dtype:
    gate row 4p + r is fused column 8p + r, up row 4p + r is fused column 8p + 4 + r."""
    m, n = t.shape
    blocks = t.view(m, n // 8, 2, 4)
    g, u = blocks[:, :, 0, :].reshape(m, n // 2), blocks[:, :, 1, :].reshape(m, n // 2)
    return (torch.nn.functional.silu(g.float()).to(dtype).float() * u.float()).to(dtype)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("m", [1, 8, 32, 64, 256, 2048, 16384])
def test_swiglu_epilogue_is_the_reference_activation_of_the_product(m):
    # The fused output splits into a GEMM output held to the 1e-2 bound of a single quantized
    # linear and an epilogue that applies the reference's activation to it: the product
    # without the epilogue (same weight, same kernel family, same summation order) is checked
    # against the oracle on sampled columns, and the fused output against silu(gate) * up of
    # that product in the compute dtype, to within one bf16 rounding step (silu's exp in the
    # kernel and in torch may differ in the last fp32 bits, which can move a rounding).
    dtype = torch.bfloat16
    inter, k = 14336, 4096
    gate = _host_qt(inter, k, 4, 128, False, seed=1)
    up = _host_qt(inter, k, 4, 128, False, seed=2)
    fused_host = interleave_gate_up(gate, up)
    fused = _to_device(fused_host)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(dtype)
    xd = x.to(DEV)
    t = ops.quant_linear(xd, fused, None, dtype)
    y = ops.quant_linear_swiglu(xd, fused, None, dtype)
    cols = np.sort(np.random.default_rng(m).choice(2 * inter, size=256, replace=False))
    rows = np.arange(m) if m <= 2048 else np.sort(np.random.default_rng(m + 1).choice(m, size=256, replace=False))
    ref = _ref_linear(x[torch.from_numpy(rows)], _oracle_dense(fused_host)[cols], dtype)
    got = t[torch.from_numpy(rows).to(DEV)][:, torch.from_numpy(cols).to(DEV)]
    assert _rel_err(got, ref) <= 1e-2
    want = _swiglu_of_product(t, dtype).float()
    diff = (y.float() - want).abs()
    step = want.abs() * 2.0 ** -7 + 2.0 ** -133  # one bf16 rounding step at each value
    assert bool((diff <= step).all()), float((diff / step).max())
    assert float((diff == 0).float().mean()) >= 0.99

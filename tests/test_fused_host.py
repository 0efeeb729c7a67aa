"""Host-side behaviour of the fused projections (``llmopt.quantization.fused``).

* The interleaved and concatenated packed weights dequantize, bit for bit, to the rows of the
  parts in the documented order (the order the kernels' epilogues rely on).
* ``QuantSwiGLU`` and ``FusedQuantLinear`` on the host give what the separate ``QuantLinear``s
  give followed by ``silu(gate) * up`` (``src/llmopt/model/layers.py:44``) or nothing.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from llmopt.quantization import (
    FusedQuantLinear,
    QuantLinear,
    QuantSwiGLU,
    RoundToNearestQuantizer,
    concat_rows,
    dequantize,
    interleave_gate_up,
)


def _qlinear(out_f, in_f, seed, dtype=torch.float32, bias=False, bits=4, group=128, symmetric=False):
    gen = torch.Generator().manual_seed(seed)
    lin = nn.Linear(in_f, out_f, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(out_f, in_f, generator=gen) * 0.02)
        if bias:
            lin.bias.copy_(torch.randn(out_f, generator=gen) * 0.1)
    qt = RoundToNearestQuantizer(bits, group, symmetric).quantize(lin.weight.detach())
    return QuantLinear.from_float(lin.to(dtype), qt, compute_dtype=dtype)


def test_interleave_order_is_bit_exact():
    gate, up = _qlinear(24, 256, 1).quantized_tensor(), _qlinear(24, 256, 2).quantized_tensor()
    fused = dequantize(interleave_gate_up(gate, up), torch.float32)
    g, u = dequantize(gate, torch.float32), dequantize(up, torch.float32)
    for p in range(6):
        for r in range(4):
            assert torch.equal(fused[8 * p + r], g[4 * p + r])
            assert torch.equal(fused[8 * p + 4 + r], u[4 * p + r])


def test_concat_rows_is_bit_exact():
    parts = [_qlinear(n, 128, 10 + n).quantized_tensor() for n in (16, 8, 8)]
    fused = dequantize(concat_rows(parts), torch.float32)
    assert torch.equal(fused, torch.cat([dequantize(p, torch.float32) for p in parts]))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bias", [False, True])
def test_swiglu_host_matches_separate_linears(dtype, bias):
    gate, up = _qlinear(32, 256, 3, dtype, bias=bias), _qlinear(32, 256, 4, dtype, bias=False)
    fused = QuantSwiGLU(gate, up)
    x = torch.randn(5, 256, generator=torch.Generator().manual_seed(5)).to(dtype)
    ref = torch.nn.functional.silu(gate(x)) * up(x)
    got = fused(x)
    assert got.shape == ref.shape and got.dtype == dtype
    torch.testing.assert_close(got, ref, rtol=1e-5 if dtype == torch.float32 else 1e-2, atol=1e-6)


def test_fused_qkv_host_matches_separate_linears():
    parts = [_qlinear(n, 128, 20 + i, bias=(i == 1)) for i, n in enumerate((64, 16, 16))]
    fused = FusedQuantLinear(parts)
    x = torch.randn(3, 7, 128, generator=torch.Generator().manual_seed(6))
    outs = fused(x)
    assert [o.shape for o in outs] == [(3, 7, 64), (3, 7, 16), (3, 7, 16)]
    for o, p in zip(outs, parts):
        torch.testing.assert_close(o, p(x), rtol=1e-5, atol=1e-6)


def test_fused_modules_reject_mismatched_parts():
    with pytest.raises(ValueError):
        FusedQuantLinear([_qlinear(16, 128, 1), _qlinear(16, 256, 2)])
    with pytest.raises(ValueError):
        FusedQuantLinear([_qlinear(16, 128, 1), _qlinear(16, 128, 2, group=64)])
    with pytest.raises(ValueError):
        QuantSwiGLU(_qlinear(16, 128, 1), _qlinear(8, 128, 2))
    with pytest.raises(ValueError):
        QuantSwiGLU(_qlinear(6, 128, 1), _qlinear(6, 128, 2))  # rows not a multiple of 4
    with pytest.raises(ValueError):
        QuantSwiGLU(_qlinear(8, 128, 1, torch.float32), _qlinear(8, 128, 2, torch.bfloat16))
    with pytest.raises(ValueError):
        FusedQuantLinear([])

"""Seeded random shapes through every route of llmopt_q_linear, against the oracle.

The hand-picked parity tests name the shapes that select each kernel. This sweep draws 160
shapes from a fixed seed over the space the routing spans -- output rows N (multiples of 16 and
ragged), input width K (multiples of 128, including multiples of 2048 and rows of 8192 codes or
more), tokens M (1-64, a few above), 2/4/8-bit codes, groups of 64, 128, 256 and whole rows,
symmetric and asymmetric, with and without bias, bf16 and fp16 -- and checks each call, once
through ``ops.quant_linear`` (which passes the workspace that ``llmopt_q_linear_workspace``
asks for) and once through the C ABI with no workspace (the kernels that need none), against
the reference's sequence on the host: the oracle's dequantized weight cast to the compute
dtype, then ``F.linear`` (max|y - y_ref| / max|y_ref| <= 1e-2).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from llmopt.kernels import _lib, ops
from llmopt.quantization import QuantizedTensor, RoundToNearestQuantizer
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu

DEV = "cuda"
NP_NAMES = {torch.float16: "float16", torch.bfloat16: "bfloat16"}
TOL = 1e-2


def _cases(count: int = 160, seed: int = 20261202):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        k = int(128 * rng.choice([1, 2, 4, 8, 12, 16, 24, 32, 48, 64, 72, 112]))
        n = int(rng.choice([16 * int(rng.integers(1, 200)), int(rng.integers(1, 3200))]))
        if n * k > 8 * 2**20:
            continue
        m = int(rng.choice([int(rng.integers(1, 65)), int(rng.integers(1, 9)), int(rng.integers(65, 300))],
                           p=[0.7, 0.2, 0.1]))
        bits = int(rng.choice([2, 4, 4, 8]))
        group = int(rng.choice([64, 128, 128, 256, -1]))
        if group > 0 and k % group:
            continue
        out.append((n, k, m, bits, group, bool(rng.integers(0, 2)), bool(rng.integers(0, 2)),
                    torch.bfloat16 if rng.integers(0, 3) else torch.float16))
    return out


CASES = _cases()


def _id(case):
    n, k, m, bits, group, sym, bias, dtype = case
    return f"N{n}-K{k}-M{m}-b{bits}-g{group}-{'sym' if sym else 'asym'}-{'bias' if bias else 'nobias'}-{NP_NAMES[dtype]}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_random_shape_against_oracle(case):
    n, k, m, bits, group, symmetric, with_bias, dtype = case
    seed = n * 7 + k * 3 + m
    gen = torch.Generator().manual_seed(seed)
    qt = RoundToNearestQuantizer(bits, group if group > 0 else k, symmetric).quantize(
        torch.randn(n, k, generator=gen) * 0.02)
    dense = qo.dequantize(qt.qweight.numpy(), qt.scales.numpy(), qt.zeros.numpy(), qt.bits, qt.group_size,
                          qt.symmetric, qt.shape)
    x = torch.randn(m, k, generator=gen).to(dtype)
    bias = torch.randn(n, generator=gen).to(dtype) if with_bias else None
    w = torch.from_numpy(qo.round_to_dtype(dense, NP_NAMES[dtype])).to(dtype)
    ref = qo.reference_linear(x, w, bias)
    dq = QuantizedTensor(qt.qweight.to(DEV), qt.scales.to(DEV), qt.zeros.to(DEV), qt.bits, qt.group_size,
                         qt.symmetric, qt.shape)
    xd = x.to(DEV)
    bd = None if bias is None else bias.to(DEV)
    y = ops.quant_linear(xd, dq, bd, dtype)

    def rel(got):
        got, want = got.float().cpu(), ref.float()
        d = float(want.abs().max())
        return float((got - want).abs().max()) / (d if d > 0 else 1.0)

    assert rel(y) <= TOL, _id(case)
    # The same call through the C ABI without a workspace: the kernels that need none.
    lib = _lib.load_library()
    y2 = torch.empty(m, n, dtype=dtype, device=DEV)
    qw, ldq, sc, zr, _, _, grp, signed = ops._weight_args(dq, xd.device)
    rc = lib.llmopt_q_linear(xd.data_ptr(), m, k, k, qw.data_ptr(), ldq, sc.data_ptr(),
                             zr.data_ptr() if zr is not None else None, None if bd is None else bd.data_ptr(),
                             y2.data_ptr(), n, n, _lib.DTYPE_CODES[dtype], bits, grp, int(symmetric), int(signed),
                             None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.llmopt_q_last_error()
    assert rel(y2) <= TOL, _id(case)

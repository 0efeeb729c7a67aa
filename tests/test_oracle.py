"""Pins the CPU oracle (oracle/quant_oracle.py) before anything is compared against it.

Every check here is independent of the oracle's own formulas: closed forms over all
byte values, hand-computed cases with exactly representable numbers, invariants, and
float64 re-derivations of each float32 operation.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import quant_oracle as qo

F32 = np.float32


# ---- pack / unpack (quantizers.py:83-97) ------------------------------------------------------

def test_unpack_every_byte_value():
    packed = np.arange(256, dtype=np.uint8).reshape(1, 256)
    codes = qo.unpack_nibbles(packed, 512)
    for b in range(256):
        assert codes[0, 2 * b] == b % 16
        assert codes[0, 2 * b + 1] == b // 16


def test_pack_every_code_pair_round_trips():
    lo, hi = np.meshgrid(np.arange(16), np.arange(16), indexing="ij")
    codes = np.stack([lo.ravel(), hi.ravel()], axis=1).reshape(1, -1).astype(np.uint8)
    packed = qo.pack_nibbles(codes)
    assert packed.shape == (1, 256)
    assert sorted(packed.ravel().tolist()) == list(range(256))
    np.testing.assert_array_equal(qo.unpack_nibbles(packed, 512), codes)


def test_unpack_truncates_and_pack_rejects_odd():
    packed = np.array([[0x21, 0x43]], dtype=np.uint8)
    np.testing.assert_array_equal(qo.unpack_nibbles(packed, 3), [[1, 2, 3]])
    with pytest.raises(ValueError):
        qo.pack_nibbles(np.zeros((2, 3), dtype=np.uint8))


# ---- choose_qparams (quantizers.py:100-142) ---------------------------------------------------

def test_qparams_asymmetric_closed_forms():
    w = np.array(
        [
            [-3.75, 0.0, 1.0, -1.0],  # min -3.75, max 1 -> s = 4.75/15, z = rne(3.75 / s)
            [0.0, 0.0, 0.0, 0.0],  # constant zero -> s = 1e-8, z = 0
            [0.5, 1.5, 3.75, 2.0],  # all positive -> min widened to 0, z = 0
            [-0.5, -1.5, -3.75, -2.0],  # all negative -> max widened to 0, z = 15
        ],
        dtype=F32,
    )
    s, z = qo.choose_qparams(w, bits=4, group_size=4, symmetric=False)
    assert s[0, 0] == F32(4.75) / F32(15)
    assert z[0, 0] == np.rint(F32(3.75) / s[0, 0])
    assert s[1, 0] == F32(1e-8) and z[1, 0] == 0
    assert s[2, 0] == F32(0.25) and z[2, 0] == 0  # 3.75 / 15 is exact
    assert s[3, 0] == F32(0.25) and z[3, 0] == 15


def test_qparams_symmetric_closed_forms():
    w = np.array([[-3.5, 1.0, 0.0, 2.0], [0.0, 0.0, 0.0, 0.0]], dtype=F32)
    s, z = qo.choose_qparams(w, bits=4, group_size=4, symmetric=True)
    assert s[0, 0] == F32(0.5)  # 3.5 / 7
    assert s[1, 0] == F32(1e-8) / F32(7)
    assert not z.any()
    s8, _ = qo.choose_qparams(w, bits=8, group_size=2, symmetric=True)
    np.testing.assert_array_equal(s8[0], [F32(3.5) / F32(127), F32(2.0) / F32(127)])


def test_qparams_groups_and_errors():
    w = np.arange(24, dtype=F32).reshape(2, 12) - 5
    s, _ = qo.choose_qparams(w, 4, 4, False)
    assert s.shape == (2, 3)
    s_row, _ = qo.choose_qparams(w, 4, 0, False)  # group <= 0: one group per row
    assert s_row.shape == (2, 1)
    with pytest.raises(ValueError):
        qo.choose_qparams(w, 4, 5, False)
    with pytest.raises(ValueError):
        qo.choose_qparams(w[0], 4, 4, False)


# ---- quantize / dequantize (quantizers.py:167-239) --------------------------------------------

def test_codes_hand_example():
    # s = 0.25, z = 15 (all-negative group); w / s is exact, rne(-0.5/0.25) = -2.
    w = np.array([[-0.5, -1.5, -3.75, -2.0]], dtype=F32)
    s, z = qo.choose_qparams(w, 4, 4, False)
    q = qo.quantize_codes(w, s, z, 4, 4, False)
    np.testing.assert_array_equal(q, [[13, 9, 0, 7]])
    np.testing.assert_array_equal(qo.dequantize_codes(q, s, z, 4, 4, False), w)


def test_round_half_even_ties():
    w = np.array([[0.5, 1.5, 2.5, -0.5, -2.5, 7.0]], dtype=F32)
    s = np.ones((1, 1), dtype=F32)
    q = qo.quantize_codes(w, s, np.zeros((1, 1), F32), 4, 6, True)
    # rne: 0, 2, 2, -0, -2, 7 ; stored biased by 8
    np.testing.assert_array_equal(q.astype(int) - 8, [[0, 2, 2, 0, -2, 7]])


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("symmetric", [False, True])
def test_invariants_random(bits, symmetric):
    rng = np.random.default_rng(bits * 10 + symmetric)
    w = (rng.standard_normal((16, 256)) * 0.02).astype(F32)
    w[0, :64] = 0.0
    s, z = qo.choose_qparams(w, bits, 64, symmetric)
    q = qo.quantize_codes(w, s, z, bits, 64, symmetric)
    if symmetric and bits == 8:
        assert q.dtype == np.int8
    else:
        assert q.dtype == np.uint8 and int(q.max()) <= 2**bits - 1
    deq = qo.dequantize_codes(q, s, z, bits, 64, symmetric)
    step = np.repeat(s, 64, axis=1)
    if not symmetric:
        # The grid spans [min, max] widened to 0, so every weight is in range.
        assert np.all(np.abs(deq - w) <= step / 2 * (1 + 1e-6) + 1e-12)
        assert np.all(deq[0, :64] == 0.0)
    else:
        # Symmetric grids clip only at the positive end of a group whose min is -amax.
        inside = np.abs(w) <= step * (2 ** (bits - 1) - 1)
        assert np.all(np.abs(deq - w)[inside] <= step[inside] / 2 * (1 + 1e-6) + 1e-12)


def test_float32_ops_match_float64_rederivation():
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((32, 512)) * 0.03).astype(F32)
    for bits, symmetric in [(4, False), (4, True), (2, False), (8, True), (8, False)]:
        s, z = qo.choose_qparams(w, bits, 128, symmetric)
        grouped = w.reshape(32, 4, 128).astype(np.float64)
        lo = np.minimum(grouped.min(-1), 0.0) if not symmetric else grouped.min(-1)
        hi = np.maximum(grouped.max(-1), 0.0) if not symmetric else grouped.max(-1)
        if symmetric:
            expect_s = np.maximum(np.maximum(np.abs(lo), np.abs(hi)), float(F32(1e-8))) / (2 ** (bits - 1) - 1)
        else:
            diff = (hi - lo).astype(F32).astype(np.float64)  # the fp32 subtraction, re-derived
            expect_s = np.maximum(diff / (2**bits - 1), float(F32(1e-8)))
        np.testing.assert_array_equal(s, expect_s.astype(F32))
        q = qo.quantize_codes(w, s, z, bits, 128, symmetric)
        deq = qo.dequantize_codes(q, s, z, bits, 128, symmetric)
        q64 = q.astype(np.float64).reshape(32, 4, 128)
        off = 0.0 if not symmetric else (float(1 << (bits - 1)) if bits < 8 else 0.0)
        zz = z.astype(np.float64)[..., None] if not symmetric else off
        exact = (q64 - zz) * s.astype(np.float64)[..., None]  # exact in float64
        np.testing.assert_array_equal(deq, exact.astype(F32).reshape(32, 512))


def test_dequantize_packed_matches_codes_path():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((8, 96)) * 0.1).astype(F32)
    for bits in (2, 4, 8):
        qw, s, z = qo.rtn_quantize(w, bits, 32, False)
        codes = qo.quantize_codes(w, s, z, bits, 32, False)
        np.testing.assert_array_equal(
            qo.dequantize(qw, s, z, bits, 32, False, w.shape),
            qo.dequantize_codes(codes, s, z, bits, 32, False),
        )
        assert qw.shape == ((8, 96) if bits == 8 else (8, 48))


# ---- dtype rounding ---------------------------------------------------------------------------

def test_bf16_round_to_nearest_even():
    cases = {
        0x3F800000: 0x3F80,  # 1.0
        0x3F808000: 0x3F80,  # tie, even stays
        0x3F818000: 0x3F82,  # tie, odd rounds up
        0x3F808001: 0x3F81,  # above tie
        0x3F807FFF: 0x3F80,  # below tie
        0x7F7FFFFF: 0x7F80,  # max float rounds to inf
        0xFF800000: 0xFF80,  # -inf
        0x00000001: 0x0000,  # smallest denormal rounds to zero
        0x80000000: 0x8000,  # -0
    }
    u = np.array(list(cases), dtype=np.uint32)
    np.testing.assert_array_equal(qo.bf16_bits(u.view(F32)), np.array(list(cases.values()), np.uint16))
    assert qo.bf16_bits(np.array([np.nan], F32))[0] == 0x7FC0


def test_bf16_matches_torch_on_finite_values():
    import torch

    rng = np.random.default_rng(11)
    v = np.concatenate([rng.standard_normal(100000).astype(F32), (rng.standard_normal(1000) * 1e-38).astype(F32)])
    ours = qo.bf16_bits(v)
    theirs = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


def test_reference_linear_matches_float64():
    import torch

    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 64)).astype(F32)
    w = rng.standard_normal((5, 64)).astype(F32)
    b = rng.standard_normal(5).astype(F32)
    y = qo.reference_linear(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b)).numpy()
    exact = x.astype(np.float64) @ w.astype(np.float64).T + b
    np.testing.assert_allclose(y, exact, rtol=1e-5, atol=1e-5)

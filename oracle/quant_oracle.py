"""CPU oracle for the quantized-linear hot path. TEST INFRASTRUCTURE ONLY.

Only tests, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may
import this module, and only to check or time against it. The product (the
``llmopt`` package and ``libllmopt_qlinear.so``) never calls it.

It restates the reference's arithmetic (``src/llmopt/quantization/quantizers.py``
and ``quant_linear.py``) in numpy float32/integer operations, independent of torch,
plus the reference's own final step (``torch.nn.functional.linear`` on the
dequantized weight) where a GEMM result is needed.

How each function is pinned (tests/test_oracle.py):

* ``pack_nibbles`` / ``unpack_nibbles``: exhaustively over all 256 byte values
  against the closed form ``(b & 15, b >> 4)``, and by the round trip.
* ``choose_qparams``, ``quantize_codes``, ``dequantize_codes``: hand-computed cases
  with exactly representable values (constant-zero, all-positive, all-negative and
  mixed groups, symmetric and asymmetric, 2/4/8 bits); invariants (codes in range,
  reconstruction error <= s/2, w = 0 reconstructs to 0 for asymmetric grids); and each
  float32 operation re-derived through float64, which is exact for the product and,
  by the double-rounding theorem for p' >= 2p + 2, equal for sums and quotients.
* ``bf16_bits``: the round-to-nearest-even rule checked on ties, carries into the
  exponent, overflow to infinity and NaN.
* ``reference_linear``: calls ``torch.nn.functional.linear``, the library routine
  the reference calls (``quant_linear.py:113``); checked against a float64 matmul.
* GPTQ with a non-diagonal Hessian is not restated here; it is pinned by the golden
  vectors in ``tests/golden/gptq_small.npz`` written from the reference itself.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "bf16_bits",
    "bf16_to_f32",
    "choose_qparams",
    "dequantize",
    "dequantize_codes",
    "pack_nibbles",
    "quantize_codes",
    "reference_linear",
    "rtn_quantize",
    "round_to_dtype",
    "unpack_nibbles",
]

F32 = np.float32


def _group(cols: int, group_size: int | None) -> int:
    return cols if group_size is None or group_size <= 0 else group_size


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """quantizers.py:83-89 -- byte j = code[2j] | code[2j+1] << 4 (uint8 arithmetic)."""
    if codes.shape[-1] % 2:
        raise ValueError("4-bit packing requires an even number of columns")
    c = codes.astype(np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << np.uint8(4))).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray, columns: int) -> np.ndarray:
    """quantizers.py:92-97 -- low nibble first, truncated to ``columns``."""
    p = packed.astype(np.uint8)
    out = np.empty(p.shape[:-1] + (2 * p.shape[-1],), dtype=np.uint8)
    out[..., 0::2] = p & np.uint8(0x0F)
    out[..., 1::2] = p >> np.uint8(4)
    return out[..., :columns].copy()


def choose_qparams(weight: np.ndarray, bits: int, group_size: int, symmetric: bool):
    """quantizers.py:100-142 -- per-group min/max scale and zero, float32."""
    if weight.ndim != 2:
        raise ValueError(f"expected a 2D weight, got shape {weight.shape}")
    rows, cols = weight.shape
    g = _group(cols, group_size)
    if cols % g:
        raise ValueError(f"in_features={cols} not divisible by group_size={g}")
    grouped = weight.reshape(rows, cols // g, g)
    lo = grouped.min(axis=-1).astype(F32)
    hi = grouped.max(axis=-1).astype(F32)
    tiny = F32(1e-8)
    if symmetric:
        amax = np.maximum(np.maximum(np.abs(lo), np.abs(hi)), tiny)
        scales = (amax / F32(2 ** (bits - 1) - 1)).astype(F32)
        zeros = np.zeros_like(scales)
    else:
        lo = np.minimum(lo, F32(0))
        hi = np.maximum(hi, F32(0))
        scales = np.maximum((hi - lo) / F32(2**bits - 1), tiny).astype(F32)
        zeros = np.rint(-lo / scales).astype(F32)
    return scales, zeros


def quantize_codes(weight, scales, zeros, bits: int, group_size: int, symmetric: bool):
    """quantizers.py:167-201 -- clamp(rne(w/s) [+ z]); int8 for symmetric 8-bit."""
    rows, cols = weight.shape
    g = _group(cols, group_size)
    w = weight.astype(F32).reshape(rows, cols // g, g)
    ratio = np.rint(w / scales[..., None]).astype(F32)
    if symmetric:
        top = 2 ** (bits - 1) - 1
        q = np.clip(ratio, F32(-top - 1), F32(top))
        if bits == 8:
            return q.astype(np.int8).reshape(rows, cols)
        q = q + F32(1 << (bits - 1))
    else:
        q = np.clip(ratio + zeros[..., None], F32(0), F32(2**bits - 1))
    return q.astype(np.uint8).reshape(rows, cols)


def dequantize_codes(codes, scales, zeros, bits: int, group_size: int, symmetric: bool):
    """quantizers.py:204-228 -- float32 (q - z) * s (symmetric: storage bias or none)."""
    rows, cols = codes.shape
    g = _group(cols, group_size)
    q = codes.astype(F32).reshape(rows, cols // g, g)
    s = scales.astype(F32)[..., None]
    if symmetric:
        if bits < 8:
            q = q - F32(1 << (bits - 1))
        w = q * s
    else:
        w = (q - zeros.astype(F32)[..., None]) * s
    return w.astype(F32).reshape(rows, cols)


def dequantize(qweight, scales, zeros, bits: int, group_size: int, symmetric: bool, shape):
    """quantizers.py:231-239 -- float32 dense weight from the packed form."""
    if bits == 8:
        codes = qweight
    else:
        codes = unpack_nibbles(qweight, shape[1])
    return dequantize_codes(codes, scales, zeros, bits, group_size, symmetric)


def rtn_quantize(weight: np.ndarray, bits: int, group_size: int, symmetric: bool):
    """quantizers.py:285-305 -- (qweight, scales, zeros) in the packed layout."""
    scales, zeros = choose_qparams(weight, bits, group_size, symmetric)
    codes = quantize_codes(weight, scales, zeros, bits, group_size, symmetric)
    qweight = codes if bits == 8 else pack_nibbles(codes)
    return qweight, scales, zeros


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even; NaN -> 0x7FC0."""
    u = np.ascontiguousarray(values, dtype=F32).view(np.uint32).astype(np.uint64)
    rounded = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16))
    out = rounded.astype(np.uint16)
    nan = np.isnan(np.asarray(values, dtype=F32))
    out[nan] = np.uint16(0x7FC0)
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(F32)


def round_to_dtype(values: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values as the reference's ``.to(dtype)`` leaves them, returned as float32."""
    if dtype == "float32":
        return values.astype(F32)
    if dtype == "float16":
        return values.astype(F32).astype(np.float16).astype(F32)
    if dtype == "bfloat16":
        return bf16_to_f32(bf16_bits(values))
    raise ValueError(dtype)


def reference_linear(x, dense_weight, bias=None):
    """The reference's final step, ``F.linear(x, W, bias)`` (quant_linear.py:113), on CPU.

    ``x``, ``dense_weight`` and ``bias`` are torch tensors already in the compute dtype.
    """
    import torch

    with torch.no_grad():
        return torch.nn.functional.linear(x, dense_weight, bias)

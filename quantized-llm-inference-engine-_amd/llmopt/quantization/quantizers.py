"""Packed weight storage and the quantize / dequantize arithmetic.

This module keeps the reference's public names, storage layout and error
behaviour (``src/llmopt/quantization/quantizers.py``) so existing callers and
checkpoints work unchanged:

* ``qweight`` for 2- and 4-bit widths is ``uint8 [out, in/2]``: column ``k`` lives
  in byte ``k >> 1``, even columns in the low nibble, odd columns in the high
  nibble (``quantizers.py:83-97``). 8-bit codes are ``uint8`` (asymmetric) or
  ``int8`` (symmetric) ``[out, in]``.
* ``scales`` and ``zeros`` are fp32 ``[out, in/group]``; group ``j`` covers
  columns ``[j*g, (j+1)*g)``. Symmetric sub-byte codes are stored biased by
  ``2**(bits-1)``.

The offline producers (min/max parameters, rounding, RTN, GPTQ) run in torch
on whatever device the weight lives on. The consumers that sit on the hot path
(:func:`unpack_int4`, :func:`dequantize`) dispatch on device: tensors on a HIP
device go to the gfx950 kernels in ``libllmopt_qlinear.so`` and never to a
host fallback; host tensors use the torch arithmetic below.
"""

from __future__ import annotations

import abc
from dataclasses import dataclass

import torch

__all__ = [
    "GPTQQuantizer",
    "QuantizedTensor",
    "Quantizer",
    "RoundToNearestQuantizer",
    "build_quantizer",
    "choose_qparams",
    "dequantize",
    "dequantize_codes",
    "expand_group_metadata",
    "pack_int4",
    "quantize_to_codes",
    "unpack_int4",
]


def _resolve_group(in_features: int, group_size: int | None) -> int:
    """Columns per group; a non-positive or missing size means one group per row."""
    if group_size is None or group_size <= 0:
        return in_features
    return group_size


@dataclass(frozen=True, slots=True)
class QuantizedTensor:
    """Packed integer codes plus the group metadata that reconstructs them.

    Same fields and helpers as the reference (``quantizers.py:25-80``).

    Attributes:
        qweight: ``uint8 [out, in/2]`` for 2/4-bit widths (two codes per byte),
            ``uint8``/``int8 [out, in]`` for 8-bit.
        scales: fp32 ``[out, num_groups]``.
        zeros: fp32 ``[out, num_groups]``; unused (zero) for symmetric grids.
        bits: Code width (2, 4 or 8).
        group_size: Input columns that share one scale/zero.
        symmetric: Whether the grid is centred on zero.
        shape: The dense ``(out_features, in_features)`` shape.
    """

    qweight: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    bits: int
    group_size: int
    symmetric: bool
    shape: tuple[int, int]

    @property
    def code_offset(self) -> int:
        """Bias that keeps symmetric codes non-negative in unsigned storage."""
        return 1 << (self.bits - 1) if self.symmetric else 0

    @property
    def pack_factor(self) -> int:
        # Kept with the reference's value (quantizers.py:59-61) for API parity;
        # the storage itself always holds two sub-byte codes per byte.
        return 32 // self.bits if self.bits < 8 else 1

    def dequantize(self) -> torch.Tensor:
        """Dense fp32 weight ``[out, in]``."""
        return dequantize(self)

    def nbytes(self) -> int:
        """Bytes held by codes, scales and zeros together."""
        total = 0
        for tensor in (self.qweight, self.scales, self.zeros):
            if tensor is not None:
                total += tensor.numel() * tensor.element_size()
        return total

    def dense_nbytes(self) -> int:
        """Bytes of the same weight held as fp16."""
        rows, cols = self.shape
        return rows * cols * 2

    def compression_ratio(self) -> float:
        return self.dense_nbytes() / max(1, self.nbytes())


def _on_hip(tensor: torch.Tensor) -> bool:
    return tensor.device.type == "cuda"


def pack_int4(codes: torch.Tensor) -> torch.Tensor:
    """Two codes per byte along the last dimension (``quantizers.py:83-89``).

    Byte ``j`` holds column ``2j`` in bits 0-3 and column ``2j+1`` in bits 4-7.

    Raises:
        ValueError: The last dimension is odd.
    """
    if codes.shape[-1] % 2:
        raise ValueError("4-bit packing requires an even number of columns")
    as_bytes = codes.to(torch.uint8)
    even = as_bytes[..., 0::2]
    odd = as_bytes[..., 1::2]
    return torch.bitwise_or(even, torch.bitwise_left_shift(odd, 4)).contiguous()


def unpack_int4(packed: torch.Tensor, columns: int) -> torch.Tensor:
    """Split every byte into its low and high nibble (``quantizers.py:92-97``).

    Returns ``[..., columns]`` codes with the dtype of ``packed``. On a HIP
    device the split runs in the gfx950 unpack kernel.
    """
    if _on_hip(packed):
        from llmopt.kernels import ops

        return ops.unpack_nibbles(packed, columns)
    low = torch.bitwise_and(packed, 0x0F)
    high = torch.bitwise_right_shift(packed, 4)
    interleaved = torch.stack((low, high), dim=-1).flatten(-2)
    return interleaved[..., :columns].contiguous()


def choose_qparams(
    weight: torch.Tensor,
    bits: int,
    group_size: int,
    symmetric: bool,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-group min/max scale and zero point (``quantizers.py:100-142``).

    Asymmetric grids widen ``[min, max]`` to include 0, then
    ``s = max((max-min)/(2**b-1), 1e-8)`` and ``z = round_half_even(-min/s)``.
    Symmetric grids use ``s = max(|min|, |max|, 1e-8) / (2**(b-1)-1)`` and ``z = 0``.

    Returns:
        ``(scales, zeros)``, fp32 ``[out, in/group]``.

    Raises:
        ValueError: ``weight`` is not 2D, or the group size does not divide the
            number of columns.
    """
    if weight.dim() != 2:
        raise ValueError(f"expected a 2D weight, got shape {tuple(weight.shape)}")
    rows, cols = weight.shape
    gsize = _resolve_group(cols, group_size)
    if cols % gsize:
        raise ValueError(f"in_features={cols} not divisible by group_size={gsize}")

    groups = weight.reshape(rows, cols // gsize, gsize)
    lo = groups.amin(dim=-1).to(torch.float32)
    hi = groups.amax(dim=-1).to(torch.float32)

    if symmetric:
        magnitude = torch.maximum(lo.abs(), hi.abs()).clamp(min=1e-8)
        scales = magnitude / (2 ** (bits - 1) - 1)
        zeros = torch.zeros_like(scales)
    else:
        lo = lo.clamp(max=0.0)
        hi = hi.clamp(min=0.0)
        scales = ((hi - lo) / (2**bits - 1)).clamp(min=1e-8)
        zeros = torch.round(torch.neg(lo) / scales)
    return scales.contiguous(), zeros.contiguous()


def expand_group_metadata(
    scales: torch.Tensor,
    zeros: torch.Tensor,
    group_size: int,
    in_features: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-column copies of the group tables (``quantizers.py:145-164``)."""
    per_col_scale = torch.repeat_interleave(scales, group_size, dim=1)[:, :in_features]
    per_col_zero = torch.repeat_interleave(zeros, group_size, dim=1)[:, :in_features]
    return per_col_scale, per_col_zero


def quantize_to_codes(
    weight: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    bits: int,
    group_size: int,
    symmetric: bool = True,
) -> torch.Tensor:
    """Round onto the integer grid (``quantizers.py:167-201``).

    Asymmetric: ``clamp(rne(w/s) + z, 0, 2**b-1)``. Symmetric:
    ``clamp(rne(w/s), -2**(b-1), 2**(b-1)-1)``, stored as ``int8`` for 8-bit
    and biased by ``2**(b-1)`` into ``uint8`` otherwise.
    """
    rows, cols = weight.shape
    gsize = _resolve_group(cols, group_size)
    grid = weight.to(torch.float32).reshape(rows, cols // gsize, gsize)
    ratio = torch.round(grid / scales.unsqueeze(-1))
    if symmetric:
        top = 2 ** (bits - 1) - 1
        codes = ratio.clamp(-top - 1, top)
        if bits == 8:
            return codes.to(torch.int8).reshape(rows, cols).contiguous()
        codes = codes + (1 << (bits - 1))
    else:
        codes = (ratio + zeros.unsqueeze(-1)).clamp(0, 2**bits - 1)
    return codes.to(torch.uint8).reshape(rows, cols).contiguous()


def dequantize_codes(
    codes: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    bits: int,
    group_size: int,
    dtype: torch.dtype = torch.float32,
    symmetric: bool = True,
) -> torch.Tensor:
    """``(q - z) * s`` in fp32, then cast to ``dtype`` (``quantizers.py:204-228``).

    Symmetric sub-byte grids subtract the storage bias ``2**(b-1)`` instead of a
    zero point; symmetric 8-bit codes are signed and use ``q * s``.
    """
    rows, cols = codes.shape
    gsize = _resolve_group(cols, group_size)
    q = codes.reshape(rows, cols // gsize, gsize).to(torch.float32)
    s = scales.unsqueeze(-1)
    if symmetric:
        if bits < 8:
            q = q - (1 << (bits - 1))
        dense = q * s
    else:
        dense = (q - zeros.unsqueeze(-1)) * s
    return dense.reshape(rows, cols).to(dtype)


def dequantize(qt: QuantizedTensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Dense ``[out, in]`` weight in ``dtype`` (``quantizers.py:231-239``).

    On a HIP device the unpack and the fp32 ``(q - z) * s`` run fused in one
    gfx950 kernel whose output is bit-identical to the host arithmetic.
    """
    if _on_hip(qt.qweight):
        from llmopt.kernels import ops

        return ops.dequantize(qt, dtype)
    if qt.bits == 8:
        codes = qt.qweight.to(torch.float32)
    else:
        codes = unpack_int4(qt.qweight, qt.shape[1]).to(torch.float32)
    return dequantize_codes(
        codes, qt.scales, qt.zeros, qt.bits, qt.group_size, dtype, qt.symmetric
    )


class Quantizer(abc.ABC):
    """Common validation and packing for weight quantizers (``quantizers.py:242-282``)."""

    name: str = "base"

    def __init__(self, bits: int, group_size: int = 128, symmetric: bool = True) -> None:
        if bits not in (2, 4, 8):
            raise ValueError(f"unsupported bit width: {bits}")
        if group_size <= 0 or group_size % 2:
            raise ValueError("group_size must be a positive even number")
        self.bits = bits
        self.group_size = group_size
        self.symmetric = symmetric

    @abc.abstractmethod
    def quantize(
        self, weight: torch.Tensor, hessian: torch.Tensor | None = None
    ) -> QuantizedTensor:
        """Quantize ``weight [out, in]``; ``hessian`` is ``[in, in]`` when known."""

    def _finalize(
        self,
        codes: torch.Tensor,
        scales: torch.Tensor,
        zeros: torch.Tensor,
        shape: tuple[int, int],
    ) -> QuantizedTensor:
        storage = codes if self.bits == 8 else pack_int4(codes)
        return QuantizedTensor(
            qweight=storage,
            scales=scales,
            zeros=zeros,
            bits=self.bits,
            group_size=self.group_size,
            symmetric=self.symmetric,
            shape=shape,
        )


class RoundToNearestQuantizer(Quantizer):
    """Min/max round-to-nearest (``quantizers.py:285-305``)."""

    name = "rtn"

    def quantize(
        self, weight: torch.Tensor, hessian: torch.Tensor | None = None
    ) -> QuantizedTensor:
        del hessian
        weight = weight.detach()
        if weight.dim() != 2:
            raise ValueError(f"expected a 2D weight, got {tuple(weight.shape)}")
        if _on_hip(weight):
            # One fused pass on the GPU, bit-exact with the sequence below.
            from llmopt.kernels import ops

            qweight, scales, zeros = ops.quantize_rtn(weight, self.bits, self.group_size, self.symmetric)
            return QuantizedTensor(
                qweight=qweight,
                scales=scales,
                zeros=zeros,
                bits=self.bits,
                group_size=self.group_size,
                symmetric=self.symmetric,
                shape=tuple(weight.shape),
            )
        scales, zeros = choose_qparams(weight, self.bits, self.group_size, self.symmetric)
        codes = quantize_to_codes(weight, scales, zeros, self.bits, self.group_size, self.symmetric)
        return self._finalize(codes, scales, zeros, tuple(weight.shape))


class GPTQQuantizer(Quantizer):
    """Hessian-driven error-compensated rounding (``quantizers.py:308-457``).

    Scales and zeros come from the unmodified weight (min/max per group). The
    columns are then visited in descending ``diag(H)`` order (``act_order``),
    block by block; each column's rounding error, divided by the pivot of the
    upper Cholesky factor of ``H^-1``, is pushed onto the columns not yet
    visited. Codes are returned in the original column order, so the layout is
    the same as round-to-nearest (no column index table).
    """

    name = "gptq"

    def __init__(
        self,
        bits: int = 4,
        group_size: int = 128,
        symmetric: bool = True,
        damping: float = 0.01,
        act_order: bool = True,
        block_size: int | None = None,
    ) -> None:
        super().__init__(bits, group_size, symmetric)
        self.damping = damping
        self.act_order = act_order
        self.block_size = block_size or group_size

    @torch.no_grad()
    def quantize(
        self, weight: torch.Tensor, hessian: torch.Tensor | None = None
    ) -> QuantizedTensor:
        """Quantize ``weight [out, in]`` given ``hessian = 2/n * X^T X`` (or RTN if None)."""
        weight = weight.detach().to(torch.float32)
        if weight.dim() != 2:
            raise ValueError(f"expected a 2D weight, got {tuple(weight.shape)}")
        rows, cols = weight.shape
        if hessian is None:
            return RoundToNearestQuantizer(self.bits, self.group_size, self.symmetric).quantize(
                weight
            )

        hinv_upper = self._prepare_hessian(hessian, cols, weight.device)
        scales, zeros = choose_qparams(weight, self.bits, self.group_size, self.symmetric)
        col_scale, col_zero = expand_group_metadata(scales, zeros, self.group_size, cols)

        order = self._activation_order(hinv_upper, cols) if self.act_order else None
        if order is None:
            work = weight.clone()
            h = hinv_upper
        else:
            work = weight[:, order]
            h = hinv_upper[order][:, order]
            col_scale = col_scale[:, order]
            col_zero = col_zero[:, order]

        signed_codes = torch.empty(rows, cols, dtype=torch.float32, device=weight.device)
        for start in range(0, cols, self.block_size):
            stop = min(start + self.block_size, cols)
            signed_codes[:, start:stop], residual = self._quantize_block(
                work[:, start:stop].clone(),
                col_scale[:, start:stop],
                col_zero[:, start:stop],
                h[start:stop, start:stop],
            )
            if stop < cols:
                work[:, stop:] -= residual @ h[start:stop, stop:]

        if order is not None:
            signed_codes = signed_codes[:, torch.argsort(order)]
        if self.symmetric and self.bits == 8:
            stored = signed_codes.to(torch.int8)
        else:
            if self.symmetric:
                signed_codes = signed_codes + (1 << (self.bits - 1))
            stored = signed_codes.to(torch.uint8)
        return QuantizedTensor(
            qweight=stored if self.bits == 8 else pack_int4(stored),
            scales=scales,
            zeros=zeros,
            bits=self.bits,
            group_size=self.group_size,
            symmetric=self.symmetric,
            shape=(rows, cols),
        )

    def _quantize_block(
        self,
        block: torch.Tensor,
        scale: torch.Tensor,
        zero: torch.Tensor,
        h_block: torch.Tensor,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Round one block column by column, feeding each error forward in the block."""
        rows, width = block.shape
        codes = torch.zeros(rows, width, dtype=torch.float32, device=block.device)
        residual = torch.zeros_like(block)
        for j in range(width):
            pivot = h_block[j, j].clamp(min=1e-8)
            col = block[:, j]
            q = _quantize_vector(col, scale[:, j], zero[:, j], self.bits, self.symmetric)
            codes[:, j] = q
            residual[:, j] = (col - _dequantize_vector(q, scale[:, j], zero[:, j], self.symmetric)) / pivot
            if j + 1 < width:
                block[:, j + 1 :] -= residual[:, j : j + 1] * h_block[j, j + 1 :].unsqueeze(0)
        return codes, residual

    def _prepare_hessian(
        self, hessian: torch.Tensor, in_features: int, device: torch.device
    ) -> torch.Tensor:
        """Symmetrize, revive dead channels, damp, and return chol(H^-1) (upper)."""
        h = hessian.detach().to(device=device, dtype=torch.float32)
        h = 0.5 * (h + h.T)
        dead = torch.diag(h) == 0
        h[dead, dead] = 1.0
        mean_diag = torch.diag(h).mean().clamp(min=1e-8)
        diag_index = range(in_features)
        h[diag_index, diag_index] += mean_diag * self.damping

        ridge = mean_diag * self.damping
        factor = None
        for _ in range(8):
            try:
                factor = torch.linalg.cholesky(h)
                break
            except Exception:  # noqa: BLE001 - widen the ridge and retry
                h[diag_index, diag_index] += ridge
                ridge = ridge * 10
        if factor is None:
            factor = torch.eye(in_features, device=device)
        upper = torch.linalg.cholesky(torch.cholesky_inverse(factor), upper=True)
        return torch.nan_to_num(upper, nan=0.0, posinf=0.0, neginf=0.0)

    @staticmethod
    def _activation_order(h: torch.Tensor, in_features: int) -> torch.Tensor:
        """Visit the highest-energy input channels first (descending diagonal)."""
        diagonal = torch.diag(h)
        if not bool(torch.isfinite(diagonal).all()) or bool((diagonal <= 0).all()):
            return torch.arange(in_features, device=h.device)
        return torch.argsort(diagonal, descending=True)


def _quantize_vector(
    w: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, bits: int, symmetric: bool
) -> torch.Tensor:
    """Signed grid rounding of one column (``quantizers.py:460-467``)."""
    if symmetric:
        top = 2 ** (bits - 1) - 1
        return torch.round(w / scale).clamp(-top - 1, top)
    return (torch.round(w / scale) + zero).clamp(0, 2**bits - 1)


def _dequantize_vector(
    q: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, symmetric: bool = True
) -> torch.Tensor:
    """Inverse of :func:`_quantize_vector` on signed codes (``quantizers.py:470-477``)."""
    if symmetric:
        return q * scale
    return (q - zero) * scale


_STRATEGY_KWARGS = {
    "gptq": (GPTQQuantizer, {"bits", "group_size", "symmetric", "damping", "act_order"}),
    "rtn": (RoundToNearestQuantizer, {"bits", "group_size", "symmetric"}),
}


def build_quantizer(strategy: str, **kwargs: object) -> Quantizer:
    """``"gptq"`` or ``"rtn"`` factory that drops unknown kwargs (``quantizers.py:480-493``).

    Raises:
        ValueError: Any other strategy name.
    """
    if strategy not in _STRATEGY_KWARGS:
        raise ValueError(f"unknown quantization strategy: {strategy!r}")
    cls, accepted = _STRATEGY_KWARGS[strategy]
    return cls(**{key: value for key, value in kwargs.items() if key in accepted})

"""The reference's host sequence in multi-threaded torch, for the CPU baseline. TEST
INFRASTRUCTURE ONLY: imported by tests and by the ``cpu_baseline`` leg of ``bench.py``.

``QuantLinear.forward`` in the reference (``src/llmopt/quantization/quant_linear.py:93-113``)
dequantizes the packed weight once -- ``unpack_int4`` (``quantizers.py:92-97``), ``.to(fp32)``,
``(q - z) * s`` (``quantizers.py:204-228``), ``.to(compute_dtype)`` -- caches that dense
weight, and calls ``F.linear``. :class:`ReferenceLinear` restates that sequence with
torch host tensors so it can be timed with every host core. Pinned in
tests/test_cpu_reference.py against the numpy oracle (dense weight bit for bit).
"""

from __future__ import annotations

import torch

__all__ = ["ReferenceLinear", "dense_weight"]


def dense_weight(qweight, scales, zeros, bits, group_size, symmetric, shape, dtype):
    """Dense ``[N, K]`` weight in ``dtype``, computed exactly as the reference does."""
    rows, cols = shape
    if bits == 8:
        q = qweight.to(torch.float32)
    else:
        lo = qweight & 0x0F
        hi = qweight >> 4
        q = torch.stack((lo, hi), dim=-1).reshape(rows, -1)[:, :cols].to(torch.float32)
    g = cols if group_size <= 0 else group_size
    q = q.reshape(rows, cols // g, g)
    if symmetric:
        if bits < 8:
            q = q - (1 << (bits - 1))
        w = q * scales.unsqueeze(-1)
    else:
        w = (q - zeros.unsqueeze(-1)) * scales.unsqueeze(-1)
    return w.reshape(rows, cols).to(dtype)


class ReferenceLinear:
    """Host ``QuantLinear``: the dense weight is built on first call and cached (warm)."""

    def __init__(self, qweight, scales, zeros, bits, group_size, symmetric, shape, dtype):
        self.args = (qweight, scales, zeros, bits, group_size, symmetric, shape, dtype)
        self.cached: torch.Tensor | None = None

    def invalidate(self) -> None:
        self.cached = None

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if self.cached is None:
            self.cached = dense_weight(*self.args)
        return torch.nn.functional.linear(x, self.cached)

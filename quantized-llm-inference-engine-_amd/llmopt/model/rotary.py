"""Rotary position embeddings, half-split (non-interleaved) layout (``src/llmopt/model/rotary.py``).

Dimension ``i < d/2`` of a head rotates with dimension ``i + d/2`` by the angle
``position * base^(-2i/d)``: ``x -> x * cos + rotate_half(x) * sin`` with
``rotate_half([a, b]) = [-b, a]`` and the angle table repeated over both halves.
"""

from __future__ import annotations

import torch
from torch import nn

__all__ = ["RotaryEmbedding", "apply_rotary_pos_emb", "rotate_half"]


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """``[a, b] -> [-b, a]`` over the last dimension."""
    a, b = x.chunk(2, dim=-1)
    return torch.cat((-b, a), dim=-1)


def apply_rotary_pos_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate ``q`` and ``k``; ``cos``/``sin`` broadcast against both (one row per token)."""
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


class RotaryEmbedding(nn.Module):
    """cos/sin tables for positions ``0 .. max_position_embeddings - 1``, built once in fp32."""

    def __init__(self, head_dim: int, max_position_embeddings: int = 4096, base: float = 10000.0,
                 dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        if head_dim % 2:
            raise ValueError("head_dim must be even for rotary embeddings")
        self.head_dim = head_dim
        self.max_position_embeddings = max_position_embeddings
        self.base = base
        exponents = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
        inv_freq = 1.0 / (base ** exponents)
        angles = torch.arange(max_position_embeddings, dtype=torch.float32)[:, None] * inv_freq[None, :]
        angles = torch.cat((angles, angles), dim=-1)
        self.register_buffer("cos_cached", angles.cos().to(dtype), persistent=False)
        self.register_buffer("sin_cached", angles.sin().to(dtype), persistent=False)

    def check(self, positions: torch.Tensor) -> None:
        """Raise ``ValueError`` for a position past the table. The check reads the positions on
        the host, so it is skipped while a HIP graph is being captured (a replayed step must not
        synchronize)."""
        capturing = positions.is_cuda and torch.cuda.is_current_stream_capturing()
        if not capturing and positions.numel() and int(positions.max()) >= self.max_position_embeddings:
            raise ValueError(f"position {int(positions.max())} exceeds table length {self.max_position_embeddings}")

    def forward(self, positions: torch.Tensor, dtype: torch.dtype | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """``(cos, sin)``, each ``[len(positions), head_dim]`` (see :meth:`check`)."""
        self.check(positions)
        cos = self.cos_cached[positions]
        sin = self.sin_cached[positions]
        if dtype is not None:
            cos, sin = cos.to(dtype), sin.to(dtype)
        return cos, sin

"""Paged attention (``src/llmopt/attention/paged_attention.py``) with gfx950 kernels.

The reference gathers every sequence's K/V into one padded tensor, repeats each KV head for
its query heads, and runs matmul, softmax and matmul (split into context chunks merged by
log-sum-exp when the context is long). Here, on a HIP device, :meth:`PagedAttention.forward`
calls ``llmopt_paged_attention_decode`` for one query token per sequence (the decode step) and
``llmopt_paged_attention_prefill`` for more (a prefill chunk, with the causal mask): both read
K/V from the cache blocks in place, once per KV head for all the query heads that share it, with
an online softmax. Other calls (host tensors, shapes the kernels do not take) run the
reference's sequence in torch.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from llmopt.utils.logging import get_logger

__all__ = ["AttentionBackend", "PagedAttention", "PagedAttentionConfig", "merge_states"]

logger = get_logger("attention.paged")


def merge_states(
    output: torch.Tensor,
    partial: torch.Tensor,
    prefix_lse: torch.Tensor,
    suffix_lse: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Merge two attention results over disjoint key sets by their log-sum-exp weights
    (``paged_attention.py:30-56``); returns ``(output, lse)``."""
    total = torch.logaddexp(prefix_lse, suffix_lse)
    w_prefix = torch.exp(prefix_lse - total).unsqueeze(-1)
    w_suffix = torch.exp(suffix_lse - total).unsqueeze(-1)
    return output * w_prefix + partial * w_suffix, total


@dataclass(slots=True)
class PagedAttentionConfig:
    """Settings of the attention (``paged_attention.py:59-73``)."""

    block_size: int = 16
    split_kv: bool = True
    split_size: int = 512
    causal: bool = True
    softcap: float = 0.0

    def __post_init__(self) -> None:
        if self.block_size < 1:
            raise ValueError("block_size must be >= 1")
        if self.split_size < 1:
            raise ValueError("split_size must be >= 1")


class AttentionBackend:
    """Backend names (``paged_attention.py:76-110``). ``"auto"`` (and ``"hip"``) select the gfx950
    decode kernel; ``"sdpa"``/``"math"``/``"eager"`` force the torch sequence. flash-attn and
    Triton are not part of this package: asking for them gives the torch sequence, with a log line,
    as the reference does when they are missing."""

    @classmethod
    def detect(cls, requested: str = "auto") -> str:
        if requested in ("auto", "hip"):
            return "hip"
        if requested in ("sdpa", "math", "eager"):
            return "sdpa"
        if requested in ("flash", "flash_attn", "triton"):
            logger.info("%s unavailable, falling back to sdpa", requested)
            return "sdpa"
        raise ValueError(f"unknown attention backend: {requested!r}")


class PagedAttention:
    """Attention that reads K/V from a paged KV cache (``paged_attention.py:113-300``).

    Args:
        num_heads: Query heads.
        num_kv_heads: Key/value heads (GQA: query head ``h`` reads KV head ``h // group``).
        head_dim: Per-head dimension.
        scale: Softmax scale, ``head_dim ** -0.5`` by default.
        config: :class:`PagedAttentionConfig`.
        backend: ``"auto"``, ``"hip"`` or ``"sdpa"`` (see :class:`AttentionBackend`).
    """

    def __init__(
        self,
        num_heads: int,
        num_kv_heads: int,
        head_dim: int,
        scale: float | None = None,
        config: PagedAttentionConfig | None = None,
        backend: str = "auto",
    ) -> None:
        if num_heads % num_kv_heads != 0:
            raise ValueError("num_heads must be divisible by num_kv_heads")
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.group_size = num_heads // num_kv_heads
        self.scale = scale if scale is not None else head_dim**-0.5
        self.config = config or PagedAttentionConfig()
        self.backend = AttentionBackend.detect(backend)

    def forward(
        self,
        query: torch.Tensor,
        cache: object,
        layer_idx: int,
        block_ids: torch.Tensor,
        context_lens: torch.Tensor,
        query_lens: int | None = None,
    ) -> torch.Tensor:
        """Attention of ``query [seq, heads, q_len, head_dim]`` over the cached context.

        ``block_ids`` is ``[seq, max_blocks]`` (``-1`` padded); ``context_lens`` is ``[seq]``, the
        context length after this step's K/V were written. Returns ``[seq, heads, q_len, head_dim]``
        in the query's dtype. Query position ``i`` of a sequence sits at ``ctx - q_len + i`` and
        sees keys up to and including its own position.
        """
        seqs = int(query.shape[0])
        q_len = query_lens if query_lens is not None else int(query.shape[2])
        if q_len == 0:
            return torch.zeros((seqs, self.num_heads, 0, self.head_dim), dtype=query.dtype, device=query.device)
        if self.backend == "hip" and query.device.type == "cuda":
            from llmopt.kernels import ops

            try:
                if q_len == 1:
                    out = ops.paged_decode_attention(
                        query[:, :, 0, :], cache.key_cache[layer_idx], cache.value_cache[layer_idx], block_ids,
                        context_lens, self.scale, self.config.softcap,
                    )
                    return out.unsqueeze(2)
                return ops.paged_prefill_attention(
                    query[:, :, :q_len], cache.key_cache[layer_idx], cache.value_cache[layer_idx], block_ids,
                    context_lens, self.scale, self.config.softcap,
                )
            except NotImplementedError:
                pass  # a shape outside the kernels: the torch sequence below
        keys, values, valid = cache.gather(layer_idx, block_ids, context_lens)
        k = keys.permute(0, 2, 1, 3)
        v = values.permute(0, 2, 1, 3)
        if self.config.split_kv and self.config.split_size < k.shape[2]:
            return self._split(query, k, v, valid, context_lens, q_len)
        return self._dense(query, k, v, valid, context_lens, q_len)

    # ---- the torch sequence ----------------------------------------------------------------------

    def _per_query_head(self, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """``[seq, kv_heads, ctx, d]`` -> ``[seq, heads, ctx, d]``, KV head g serving heads
        ``g * group .. g * group + group - 1`` (``paged_attention.py:184-205``)."""
        if self.group_size == 1:
            return k.contiguous(), v.contiguous()
        return (k.repeat_interleave(self.group_size, dim=1).contiguous(),
                v.repeat_interleave(self.group_size, dim=1).contiguous())

    def _mask(self, valid: torch.Tensor, context_lens: torch.Tensor, q_len: int) -> torch.Tensor:
        """``[seq, 1, q_len, ctx]``: valid keys, and causal when several queries
        (``paged_attention.py:207-216``)."""
        mask = valid[:, None, None, :].expand(-1, 1, q_len, -1)
        if q_len > 1:
            q_pos = context_lens.to(valid.device)[:, None] - q_len + torch.arange(q_len, device=valid.device)
            k_pos = torch.arange(valid.shape[1], device=valid.device)
            mask = mask & (k_pos[None, None, :] <= q_pos[:, :, None])[:, None]
        return mask

    def _scores(self, q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
        # The transposed operand is made contiguous: batched products with a transposed right
        # operand are avoided on the GPU.
        scores = torch.matmul(q.to(k.dtype), k.transpose(-1, -2).contiguous()) * self.scale
        if self.config.softcap > 0:
            scores = torch.tanh(scores / self.config.softcap) * self.config.softcap
        return scores

    def _dense(self, q, k, v, valid, context_lens, q_len):  # noqa: ANN001, ANN202
        k, v = self._per_query_head(k, v)
        scores = self._scores(q, k).masked_fill(~self._mask(valid, context_lens, q_len), float("-inf"))
        probs = torch.nan_to_num(torch.softmax(scores, dim=-1), nan=0.0)
        return torch.matmul(probs, v).to(q.dtype)

    def _split(self, q, k, v, valid, context_lens, q_len):  # noqa: ANN001, ANN202
        """Context chunks of ``split_size`` keys merged by log-sum-exp (``paged_attention.py:237-290``)."""
        k, v = self._per_query_head(k, v)
        out = lse = None
        for lo in range(0, k.shape[2], self.config.split_size):
            hi = min(lo + self.config.split_size, k.shape[2])
            scores = self._scores(q, k[:, :, lo:hi])
            scores = scores.masked_fill(~self._mask(valid[:, lo:hi], context_lens - lo, q_len), float("-inf"))
            part_lse = torch.logsumexp(scores, dim=-1)
            probs = torch.nan_to_num(torch.softmax(scores, dim=-1), nan=0.0)
            part = torch.matmul(probs, v[:, :, lo:hi].contiguous())
            if out is None:
                out, lse = part, part_lse
            else:
                out, lse = merge_states(out, part, lse, part_lse)
        return torch.nan_to_num(out, nan=0.0).to(q.dtype)

    def __repr__(self) -> str:
        return (
            f"PagedAttention(heads={self.num_heads}, kv_heads={self.num_kv_heads}, head_dim={self.head_dim}, "
            f"backend={self.backend}, split_kv={self.config.split_kv})"
        )

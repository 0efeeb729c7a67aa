"""Attention over the paged KV cache (``src/llmopt/attention``)."""

from __future__ import annotations

from llmopt.attention.paged_attention import (
    AttentionBackend,
    PagedAttention,
    PagedAttentionConfig,
    merge_states,
)

__all__ = ["AttentionBackend", "PagedAttention", "PagedAttentionConfig", "merge_states"]

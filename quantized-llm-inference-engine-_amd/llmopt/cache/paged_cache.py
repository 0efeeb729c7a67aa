"""Paged key/value cache with GPU writes (``src/llmopt/cache/paged_cache.py:137-331``).

Storage is the reference's: per layer ``[num_blocks, block_size, kv_heads, head_dim]`` for keys
and for values, preallocated and zero-filled, so a block table row maps a sequence's token ``t``
to block ``row[t // block_size]``, slot ``t % block_size``.

On HIP devices :meth:`PagedKVCache.write_decode` and :meth:`PagedKVCache.write` run one gfx950
kernel each (``llmopt_kv_write_decode`` / ``llmopt_kv_write``) instead of indexed assignment or
a Python loop over sequences and blocks; on the host they follow the same rules in torch.
"""

from __future__ import annotations

import torch

__all__ = ["PagedKVCache"]


def _on_hip(t: torch.Tensor) -> bool:
    return t.device.type == "cuda"


class PagedKVCache:
    """Fixed-capacity paged K/V store shared by all layers.

    Args:
        num_layers: Decoder layers sharing the store.
        num_blocks: Physical blocks per layer.
        block_size: Tokens per block.
        num_kv_heads: Key/value heads.
        head_dim: Per-head dimension.
        dtype: Storage dtype.
        device: Device to allocate on.
    """

    def __init__(
        self,
        num_layers: int,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype = torch.float16,
        device: torch.device | str = "cpu",
    ) -> None:
        if num_layers < 1:
            raise ValueError("num_layers must be >= 1")
        if num_blocks < 1 or block_size < 1:
            raise ValueError("num_blocks and block_size must be >= 1")
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        shape = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        self.key_cache = torch.zeros(shape, dtype=dtype, device=self.device)
        self.value_cache = torch.zeros(shape, dtype=dtype, device=self.device)

    # ---- writes ---------------------------------------------------------------------------------

    def write(
        self,
        layer_idx: int,
        block_ids: torch.Tensor,
        token_offsets: torch.Tensor,
        keys: torch.Tensor,
        values: torch.Tensor,
    ) -> None:
        """Store ``keys``/``values`` ``[seq, q_len, kv_heads, head_dim]`` from ``token_offsets[s]``.

        A sequence's tokens go block by block through its row of ``block_ids`` (``-1`` padded);
        writing stops at the first ``-1`` block or at the end of the row (``paged_cache.py:187-244``).
        """
        seqs, q_len = int(keys.shape[0]), int(keys.shape[1])
        if seqs == 0 or q_len == 0:
            return
        if _on_hip(self.key_cache):
            from llmopt.kernels import ops

            ops.kv_write(self.key_cache[layer_idx], self.value_cache[layer_idx], block_ids, token_offsets,
                         keys, values)
            return
        table = block_ids.to("cpu", torch.long)
        starts = token_offsets.to("cpu", torch.long)
        for s in range(seqs):
            pos = int(starts[s])
            for j in range(q_len):
                index = (pos + j) // self.block_size
                if index >= table.shape[1] or int(table[s, index]) < 0:
                    break
                block, slot = int(table[s, index]), (pos + j) % self.block_size
                self.key_cache[layer_idx, block, slot] = keys[s, j].to(self.dtype)
                self.value_cache[layer_idx, block, slot] = values[s, j].to(self.dtype)

    def write_decode(
        self,
        layer_idx: int,
        block_ids: torch.Tensor,
        token_offsets: torch.Tensor,
        keys: torch.Tensor,
        values: torch.Tensor,
    ) -> None:
        """Store one token per sequence, ``keys``/``values`` ``[seq, kv_heads, head_dim]``.

        Token ``token_offsets[s]`` lands in block ``block_ids[s, off // block_size]`` at slot
        ``off % block_size``; a block id outside ``[0, num_blocks)`` is replaced by block 0, as the
        reference does (``paged_cache.py:246-277``). On HIP devices an offset past the end of the
        table row writes nothing (the reference raises an IndexError there).
        """
        seqs = int(keys.shape[0])
        if seqs == 0:
            return
        if _on_hip(self.key_cache):
            from llmopt.kernels import ops

            ops.kv_write_decode(self.key_cache[layer_idx], self.value_cache[layer_idx], block_ids,
                                token_offsets, keys, values)
            return
        offsets = token_offsets.to(torch.long)
        index = torch.div(offsets, self.block_size, rounding_mode="floor")
        slot = offsets - index * self.block_size
        blocks = block_ids.to(torch.long)[torch.arange(seqs, device=block_ids.device), index]
        blocks = torch.where((blocks >= 0) & (blocks < self.num_blocks), blocks, torch.zeros_like(blocks))
        self.key_cache[layer_idx, blocks, slot] = keys.to(self.dtype)
        self.value_cache[layer_idx, blocks, slot] = values.to(self.dtype)

    # ---- reads ----------------------------------------------------------------------------------

    def gather(
        self,
        layer_idx: int,
        block_ids: torch.Tensor,
        context_lens: torch.Tensor,
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Dense ``(keys, values, valid)`` for a ragged batch (``paged_cache.py:279-324``).

        keys/values are ``[seq, max_len, kv_heads, head_dim]`` padded with zeros to the longest
        context; ``valid[s, t]`` is true when ``t < context_lens[s]`` and the token's block id is
        not ``-1``.
        """
        seqs = int(block_ids.shape[0])
        dev = self.key_cache.device
        longest = int(context_lens.max().item()) if seqs else 0
        if longest == 0:
            empty = torch.zeros((seqs, 0, self.num_kv_heads, self.head_dim), dtype=self.dtype, device=dev)
            return empty, empty.clone(), torch.zeros((seqs, 0), dtype=torch.bool, device=dev)
        pos = torch.arange(longest, device=dev)
        ids = block_ids.to(dev, torch.long)[:, pos // self.block_size]
        valid = (ids >= 0) & (pos[None, :] < context_lens.to(dev)[:, None])
        rows = torch.where(ids >= 0, ids, torch.zeros_like(ids)) * self.block_size + pos % self.block_size
        flat_k = self.key_cache[layer_idx].reshape(-1, self.num_kv_heads, self.head_dim)
        flat_v = self.value_cache[layer_idx].reshape(-1, self.num_kv_heads, self.head_dim)
        keys = flat_k[rows]
        values = flat_v[rows]
        keep = valid[:, :, None, None]
        zero = torch.zeros((), dtype=self.dtype, device=dev)
        return torch.where(keep, keys, zero), torch.where(keep, values, zero), valid

    # ---- housekeeping ---------------------------------------------------------------------------

    def memory_bytes(self) -> int:
        return 2 * self.key_cache.numel() * self.key_cache.element_size()

    def reset(self) -> None:
        self.key_cache.zero_()
        self.value_cache.zero_()

    def __repr__(self) -> str:
        return (
            f"PagedKVCache(layers={self.num_layers}, blocks={self.num_blocks}, "
            f"block_size={self.block_size}, kv_heads={self.num_kv_heads}, head_dim={self.head_dim}, "
            f"dtype={self.dtype}, bytes={self.memory_bytes()})"
        )

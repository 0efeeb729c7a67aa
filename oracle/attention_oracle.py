"""CPU oracle for the paged KV cache and decode attention. TEST INFRASTRUCTURE ONLY.

Only tests (and ``__graft_entry__.smoke()``/``bench.py``'s CPU leg, should they need it) may
import this module, and only to check against it; the ``llmopt`` package and its library never
call it.

It restates, in numpy, what the reference computes:

* ``kv_write_decode`` -- ``PagedKVCache.write_decode`` (``src/llmopt/cache/paged_cache.py:246-277``):
  one token per sequence lands at block ``block_ids[s, off // B]``, slot ``off % B``; a block id
  outside ``[0, num_blocks)`` is replaced by block 0 (``:270-273``).
* ``kv_write`` -- ``PagedKVCache.write`` / ``_write_one`` (``:187-244``): ``q_len`` tokens per
  sequence from ``token_offsets[s]``, block by block, stopping at the first ``-1`` block or the
  end of the table.
* ``kv_gather`` -- ``PagedKVCache.gather`` (``:279-324``): padded ``[seq, max_len, kv_heads,
  head_dim]`` K/V and the validity mask (block id >= 0 and position < context length).
* ``paged_decode_attention`` -- ``PagedAttention.forward`` for one query token per sequence
  (``src/llmopt/attention/paged_attention.py:145-182,218-235``): the query cast to the cache
  dtype, scores ``q . k * scale`` (optionally soft-capped), masked to the valid keys, softmax,
  times V; query head ``h`` reads KV head ``h // (heads / kv_heads)`` (``:184-205``). A
  sequence with no valid key gives zeros (``:233-235``). Computed in float64: the reference's
  own fp16/bf16 intermediate roundings are what the GPU tests' tolerance covers.
* ``paged_prefill_attention`` -- ``PagedAttention.forward`` for ``q_len`` query tokens per
  sequence (``:145-182,210-250``): query token ``j`` sits at ``ctx - q_len + j`` and sees the
  valid keys up to and including its own position (``_build_mask``, ``:210-229``); a query with
  no key gives zeros (``nan_to_num``, ``:248-249``).
* ``merge_states`` -- ``merge_states`` (``:30-56``), the log-sum-exp merge of the split path.

Pinned by tests/test_attention_oracle.py: context length 1 returns that token's value exactly;
identical keys give the mean of the values; a dominant key returns its value; agreement with
torch's ``scaled_dot_product_attention`` in float64 (a library routine) with explicit GQA
expansion and padding masks; the split path (``merge_states`` over chunks) equals the dense
one; write -> gather round trips, including the block-0 substitution and the stop at -1. The
prefill form: one query token at the last position equals the decode form; the first token of a
prompt with no prefix returns the first value exactly; identical keys give the mean of the
values up to each position; agreement with torch's ``scaled_dot_product_attention`` in float64
with the causal + padding mask built independently from positions.
"""

from __future__ import annotations

import math

import numpy as np

from oracle.quant_oracle import round_to_dtype

__all__ = ["kv_gather", "kv_write", "kv_write_decode", "merge_states", "paged_decode_attention",
           "paged_prefill_attention"]


def _cast(values: np.ndarray, dtype: str) -> np.ndarray:
    """``tensor.to(dtype)`` as float32 values ('float32', 'float16' or 'bfloat16')."""
    return round_to_dtype(np.asarray(values, dtype=np.float32), dtype)


def kv_write_decode(key_cache, value_cache, layer, block_ids, token_offsets, keys, values, dtype="float16"):
    """paged_cache.py:246-277. Returns updated copies of the caches (float32 arrays)."""
    kc, vc = key_cache.copy(), value_cache.copy()
    num_blocks, block_size = kc.shape[1], kc.shape[2]
    for s in range(keys.shape[0]):
        off = int(token_offsets[s])
        block = int(block_ids[s, off // block_size])  # an index past the table raises, as in torch
        if not 0 <= block < num_blocks:
            block = 0
        kc[layer, block, off % block_size] = _cast(keys[s], dtype)
        vc[layer, block, off % block_size] = _cast(values[s], dtype)
    return kc, vc


def kv_write(key_cache, value_cache, layer, block_ids, token_offsets, keys, values, dtype="float16"):
    """paged_cache.py:187-244: keys/values ``[seq, q_len, kv_heads, head_dim]``."""
    kc, vc = key_cache.copy(), value_cache.copy()
    block_size = kc.shape[2]
    seqs, q_len = keys.shape[0], keys.shape[1]
    for s in range(seqs):
        pos = int(token_offsets[s])
        for j in range(q_len):
            index = (pos + j) // block_size
            if index >= block_ids.shape[1]:
                break
            block = int(block_ids[s, index])
            if block < 0:
                break
            kc[layer, block, (pos + j) % block_size] = _cast(keys[s, j], dtype)
            vc[layer, block, (pos + j) % block_size] = _cast(values[s, j], dtype)
    return kc, vc


def kv_gather(key_cache, value_cache, layer, block_ids, context_lens):
    """paged_cache.py:279-324: (keys, values, valid) padded to the longest context."""
    seqs = block_ids.shape[0]
    block_size, kv_heads, head_dim = key_cache.shape[2:]
    max_len = int(np.max(context_lens)) if seqs else 0
    keys = np.zeros((seqs, max_len, kv_heads, head_dim), dtype=key_cache.dtype)
    values = np.zeros_like(keys)
    valid = np.zeros((seqs, max_len), dtype=bool)
    for s in range(seqs):
        for t in range(max_len):
            block = int(block_ids[s, t // block_size])
            if block >= 0 and t < int(context_lens[s]):
                valid[s, t] = True
                keys[s, t] = key_cache[layer, block, t % block_size]
                values[s, t] = value_cache[layer, block, t % block_size]
    return keys, values, valid


def paged_decode_attention(query, key_cache, value_cache, layer, block_ids, context_lens,
                           scale=None, softcap=0.0, cache_dtype="float16"):
    """paged_attention.py:145-182 for q_len = 1, in float64.

    query ``[seq, heads, head_dim]``; caches ``[layers, blocks, block_size, kv_heads, head_dim]``
    holding values already in the cache dtype. Returns ``[seq, heads, head_dim]`` float64.
    """
    seqs, heads, head_dim = query.shape
    kv_heads = key_cache.shape[3]
    group = heads // kv_heads
    scale = head_dim ** -0.5 if scale is None else scale
    q = _cast(query, cache_dtype).astype(np.float64)  # q.to(k.dtype)
    keys, values, valid = kv_gather(key_cache, value_cache, layer, block_ids, context_lens)
    out = np.zeros((seqs, heads, head_dim), dtype=np.float64)
    for s in range(seqs):
        mask = valid[s]
        if not mask.any():
            continue
        for h in range(heads):
            g = h // group
            k = keys[s, mask, g].astype(np.float64)
            v = values[s, mask, g].astype(np.float64)
            scores = (k @ q[s, h]) * scale
            if softcap > 0:
                scores = np.tanh(scores / softcap) * softcap
            p = np.exp(scores - scores.max())
            out[s, h] = (p / p.sum()) @ v
    return out


def paged_prefill_attention(query, key_cache, value_cache, layer, block_ids, context_lens,
                            scale=None, softcap=0.0, cache_dtype="float16"):
    """paged_attention.py:145-182, 210-250 for ``q_len`` tokens per sequence, in float64.

    query ``[seq, heads, q_len, head_dim]``; token ``j`` of sequence ``s`` sits at
    ``context_lens[s] - q_len + j`` and attends to the valid keys at positions up to its own.
    Returns ``[seq, heads, q_len, head_dim]`` float64.
    """
    seqs, heads, q_len, head_dim = query.shape
    kv_heads = key_cache.shape[3]
    group = heads // kv_heads
    scale = head_dim ** -0.5 if scale is None else scale
    q = _cast(query, cache_dtype).astype(np.float64)
    keys, values, valid = kv_gather(key_cache, value_cache, layer, block_ids, context_lens)
    out = np.zeros((seqs, heads, q_len, head_dim), dtype=np.float64)
    for s in range(seqs):
        for j in range(q_len):
            pos = int(context_lens[s]) - q_len + j
            mask = valid[s] & (np.arange(valid.shape[1]) <= pos)
            if not mask.any():
                continue
            for h in range(heads):
                g = h // group
                k = keys[s, mask, g].astype(np.float64)
                v = values[s, mask, g].astype(np.float64)
                scores = (k @ q[s, h, j]) * scale
                if softcap > 0:
                    scores = np.tanh(scores / softcap) * softcap
                p = np.exp(scores - scores.max())
                out[s, h, j] = (p / p.sum()) @ v
    return out


def merge_states(output, partial, prefix_lse, suffix_lse):
    """paged_attention.py:30-56: log-sum-exp merge of two partial results (float64)."""
    merged_lse = np.logaddexp(prefix_lse, suffix_lse)
    w1 = np.exp(prefix_lse - merged_lse)[..., None]
    w2 = np.exp(suffix_lse - merged_lse)[..., None]
    return output * w1 + partial * w2, merged_lse


def split_decode_attention(query, key_cache, value_cache, layer, block_ids, context_lens, split,
                           scale=None, cache_dtype="float16"):
    """The split path (paged_attention.py:237-290) for q_len = 1: chunks of ``split`` keys,
    merged with ``merge_states``; float64."""
    seqs, heads, head_dim = query.shape
    kv_heads = key_cache.shape[3]
    group = heads // kv_heads
    scale = head_dim ** -0.5 if scale is None else scale
    q = _cast(query, cache_dtype).astype(np.float64)
    keys, values, valid = kv_gather(key_cache, value_cache, layer, block_ids, context_lens)
    ctx = keys.shape[1]
    acc = acc_lse = None
    for start in range(0, ctx, split):
        end = min(start + split, ctx)
        part = np.zeros((seqs, heads, head_dim))
        lse = np.full((seqs, heads), -math.inf)
        for s in range(seqs):
            mask = valid[s, start:end]
            if not mask.any():
                continue
            for h in range(heads):
                g = h // group
                k = keys[s, start:end][mask, g].astype(np.float64)
                v = values[s, start:end][mask, g].astype(np.float64)
                scores = (k @ q[s, h]) * scale
                top = scores.max()
                p = np.exp(scores - top)
                lse[s, h] = top + math.log(p.sum())
                part[s, h] = (p / p.sum()) @ v
        if acc is None:
            acc, acc_lse = part, lse
        else:
            with np.errstate(invalid="ignore"):
                acc, acc_lse = merge_states(acc, part, acc_lse, lse)
    return np.nan_to_num(acc, nan=0.0)

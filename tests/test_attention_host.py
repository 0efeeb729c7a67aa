"""PagedKVCache and PagedAttention on the host: the reference's own attention tests
(tests/test_paged_attention.py there), restated, plus agreement with the oracle and the
last-token logits helper. CPU only."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from llmopt.attention import AttentionBackend, PagedAttention, PagedAttentionConfig, merge_states
from llmopt.cache import PagedKVCache
from llmopt.logits import last_token_hidden, last_token_logits
from oracle import attention_oracle as ao

SEQ, HEADS, KV_HEADS, HEAD_DIM, BLOCK = 3, 4, 2, 8, 8


def _dense_causal(q, k, v, ctx, q_len, group):
    """Per-sequence causal attention in fp32, as the reference's test computes it."""
    out = torch.empty(q.shape[0], HEADS, q_len, HEAD_DIM)
    for s, length in enumerate(ctx):
        keys = k[s, :length].permute(1, 0, 2).repeat_interleave(group, 0)
        values = v[s, :length].permute(1, 0, 2).repeat_interleave(group, 0)
        scores = (q[s].float() @ keys.float().transpose(-1, -2)) / math.sqrt(HEAD_DIM)
        q_pos = torch.arange(length - q_len, length)[:, None]
        scores = scores.masked_fill(torch.arange(length)[None, :] > q_pos, float("-inf"))
        out[s] = torch.softmax(scores, -1) @ values.float()
    return out


@pytest.fixture
def paged():
    torch.manual_seed(1)
    cache = PagedKVCache(1, 64, BLOCK, KV_HEADS, HEAD_DIM, dtype=torch.float32)
    ctx = [12, 20, 9]  # ragged, none a multiple of the block size
    table = torch.full((SEQ, 8), -1, dtype=torch.long)
    free = list(range(63, -1, -1))  # blocks handed out in a scrambled order
    for s, length in enumerate(ctx):
        n = -(-length // BLOCK)
        table[s, :n] = torch.tensor([free.pop(3 * s % len(free)) for _ in range(n)])
    keys = torch.randn(SEQ, max(ctx), KV_HEADS, HEAD_DIM)
    values = torch.randn(SEQ, max(ctx), KV_HEADS, HEAD_DIM)
    cache.write(0, table, torch.zeros(SEQ, dtype=torch.long), keys, values)
    return cache, table, keys, values, torch.tensor(ctx)


@pytest.mark.parametrize("split_kv", [False, True])
def test_ragged_batched_prefill_matches_dense(paged, split_kv):
    cache, table, keys, values, ctx = paged
    q = torch.randn(SEQ, HEADS, 5, HEAD_DIM)
    cfg = PagedAttentionConfig(block_size=BLOCK, split_kv=split_kv, split_size=4)
    out = PagedAttention(HEADS, KV_HEADS, HEAD_DIM, config=cfg).forward(q, cache, 0, table, ctx, 5)
    want = _dense_causal(q, keys, values, ctx.tolist(), 5, HEADS // KV_HEADS)
    assert torch.allclose(out.float(), want, atol=1e-5)


def test_decode_matches_dense_and_the_oracle(paged):
    cache, table, keys, values, ctx = paged
    q = torch.randn(SEQ, HEADS, 1, HEAD_DIM)
    out = PagedAttention(HEADS, KV_HEADS, HEAD_DIM, config=PagedAttentionConfig(block_size=BLOCK)).forward(
        q, cache, 0, table, ctx, 1
    )
    assert torch.allclose(out.float(), _dense_causal(q, keys, values, ctx.tolist(), 1, 2), atol=1e-5)
    ref = ao.paged_decode_attention(q[:, :, 0].numpy(), cache.key_cache.numpy(), cache.value_cache.numpy(), 0,
                                    table.numpy(), ctx.numpy(), cache_dtype="float32")
    np.testing.assert_allclose(out[:, :, 0].numpy(), ref, atol=1e-6)


def test_split_kv_agrees_with_dense(paged):
    cache, table, _, _, ctx = paged
    q = torch.randn(SEQ, HEADS, 4, HEAD_DIM)
    dense = PagedAttention(HEADS, KV_HEADS, HEAD_DIM, config=PagedAttentionConfig(BLOCK, split_kv=False))
    split = PagedAttention(HEADS, KV_HEADS, HEAD_DIM, config=PagedAttentionConfig(BLOCK, split_kv=True, split_size=3))
    assert torch.allclose(dense.forward(q, cache, 0, table, ctx, 4), split.forward(q, cache, 0, table, ctx, 4),
                          atol=1e-5)


def test_cache_round_trips_written_kv(paged):
    cache, table, keys, values, ctx = paged
    got_k, got_v, valid = cache.gather(0, table, ctx)
    for s, length in enumerate(ctx.tolist()):
        assert torch.equal(got_k[s, :length], keys[s, :length])
        assert torch.equal(got_v[s, :length], values[s, :length])
        assert bool(valid[s, :length].all()) and not bool(valid[s, length:].any())


def test_host_writes_match_the_oracle():
    rng = np.random.default_rng(4)
    cache = PagedKVCache(2, 8, 4, 2, 8, dtype=torch.bfloat16)
    table = np.array([[0, 1, -1, 3], [4, 5, 6, 7], [2, -1, -1, -1]])
    offsets = np.array([2, 3, 1])
    keys = rng.standard_normal((3, 10, 2, 8)).astype(np.float32)
    cache.write(1, torch.from_numpy(table), torch.from_numpy(offsets), torch.from_numpy(keys),
                torch.from_numpy(keys * 3))
    kc0 = np.zeros((2, 8, 4, 2, 8), np.float32)
    want_k, want_v = ao.kv_write(kc0, kc0.copy(), 1, table, offsets, keys, keys * 3, dtype="bfloat16")
    np.testing.assert_array_equal(cache.key_cache.float().numpy(), want_k)
    np.testing.assert_array_equal(cache.value_cache.float().numpy(), want_v)
    dec = rng.standard_normal((3, 2, 8)).astype(np.float32)
    dec_table = np.array([[3, 9, -1, -1], [1, -1, 2, 0], [-1, 6, 5, 4]])  # 9 and -1: block 0
    dec_off = np.array([5, 2, 1])
    cache.write_decode(0, torch.from_numpy(dec_table), torch.from_numpy(dec_off), torch.from_numpy(dec),
                       torch.from_numpy(dec))
    want_k, _ = ao.kv_write_decode(want_k, want_v, 0, dec_table, dec_off, dec, dec, dtype="bfloat16")
    np.testing.assert_array_equal(cache.key_cache.float().numpy(), want_k)


def test_merge_states_is_the_log_sum_exp_merge():
    a, b = torch.randn(2, 3, 4, dtype=torch.float64), torch.randn(2, 3, 4, dtype=torch.float64)
    la, lb = torch.randn(2, 3, dtype=torch.float64), torch.randn(2, 3, dtype=torch.float64)
    out, lse = merge_states(a, b, la, lb)
    want, want_lse = ao.merge_states(a.numpy(), b.numpy(), la.numpy(), lb.numpy())
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-12)
    np.testing.assert_allclose(lse.numpy(), want_lse, rtol=1e-12)


def test_backend_names():
    assert AttentionBackend.detect() == "hip"
    assert AttentionBackend.detect("sdpa") == "sdpa"
    assert AttentionBackend.detect("flash") == "sdpa"
    with pytest.raises(ValueError):
        AttentionBackend.detect("cuda-graphs")
    with pytest.raises(ValueError):
        PagedAttention(6, 4, 8)
    with pytest.raises(ValueError):
        PagedAttentionConfig(block_size=0)


def test_zero_length_query_and_cache_validation():
    cache = PagedKVCache(1, 4, 4, 1, 8)
    out = PagedAttention(2, 1, 8).forward(torch.zeros(3, 2, 0, 8), cache, 0, torch.zeros(3, 1), torch.ones(3), 0)
    assert out.shape == (3, 2, 0, 8)
    with pytest.raises(ValueError):
        PagedKVCache(0, 4, 4, 1, 8)
    with pytest.raises(ValueError):
        PagedKVCache(1, 4, 0, 1, 8)
    assert cache.memory_bytes() == 2 * 4 * 4 * 8 * 2


def test_last_token_logits_match_the_full_projection():
    torch.manual_seed(0)
    head = torch.nn.Linear(64, 1000, bias=False)
    hidden = torch.randn(3 * 7, 64)
    full = head(hidden).view(3, 7, -1)[:, -1]
    assert torch.allclose(last_token_logits(hidden, head, 7), full, atol=1e-5)
    assert torch.equal(last_token_hidden(hidden, 7), hidden.view(3, 7, 64)[:, -1])
    with pytest.raises(ValueError):
        last_token_hidden(hidden, 4)


def test_cache_write_wrappers_reject_short_per_sequence_tensors():
    # The kernels read row s of every per-sequence tensor for s < seqs; the wrappers reject
    # short ones before anything reaches the device (the reference's indexing raises too).
    from llmopt.kernels import ops

    kc = torch.zeros(4, 16, 2, 8, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    q = torch.zeros(3, 4, 8, dtype=torch.bfloat16)
    k = torch.zeros(3, 2, 8, dtype=torch.bfloat16)
    table = torch.zeros(3, 2, dtype=torch.int32)
    offs = torch.zeros(3, dtype=torch.int32)
    pos = torch.zeros(3, dtype=torch.int64)
    cos = torch.ones(32, 8)
    bad = {
        "positions": (pos[:2], offs, table, k),
        "token_offsets": (pos, offs[:1], table, k),
        "block_ids": (pos, offs, table[:2], k),
        "k rows": (pos, offs, table, k[:2]),
    }
    for name, (p, o, t, kk) in bad.items():
        with pytest.raises(ValueError):
            ops.rope_kv_write_decode(q, kk, kk.clone(), p, cos, cos, kc, vc, t, o)
        with pytest.raises(ValueError):
            ops.paged_decode_attention_rope(q, kk, kk.clone(), p, cos, cos, kc, vc, t, offs + 1, o, 0.125)
    lens = offs + 1
    with pytest.raises(ValueError):  # context lengths short
        ops.paged_decode_attention_rope(q, k, k.clone(), pos, cos, cos, kc, vc, table, lens[:2], offs, 0.125)
    with pytest.raises(ValueError):  # q in another dtype than the cache
        ops.paged_decode_attention_rope(q.half(), k, k.clone(), pos, cos, cos, kc, vc, table, lens, offs, 0.125)
    with pytest.raises(ValueError):
        ops.kv_write_decode(kc, vc, table[:1], offs, k, k)
    with pytest.raises(ValueError):
        ops.kv_write_decode(kc, vc, table, offs[:2], k, k)
    with pytest.raises(ValueError):
        ops.kv_write(kc, vc, table[:2], offs, k[:, None], k[:, None])

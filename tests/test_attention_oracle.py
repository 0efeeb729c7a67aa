"""The attention oracle against what the mathematics and a library routine fix (CPU only)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention_oracle as ao


def _cache(layers=1, blocks=16, block_size=4, kv_heads=2, head_dim=8, seed=0):
    rng = np.random.default_rng(seed)
    shape = (layers, blocks, block_size, kv_heads, head_dim)
    return rng.standard_normal(shape).astype(np.float32), rng.standard_normal(shape).astype(np.float32)


def _table(ctx, block_size, width, start=0):
    table = np.full((len(ctx), width), -1, dtype=np.int64)
    nxt = start
    for s, length in enumerate(ctx):
        n = -(-length // block_size)
        table[s, :n] = np.arange(nxt, nxt + n)
        nxt += n
    return table


def test_single_key_returns_its_value():
    kc, vc = _cache()
    table = _table([1], 4, 2)
    q = np.random.default_rng(1).standard_normal((1, 4, 8)).astype(np.float32)
    out = ao.paged_decode_attention(q, kc, vc, 0, table, np.array([1]), cache_dtype="float32")
    for h in range(4):
        np.testing.assert_array_equal(out[0, h], vc[0, table[0, 0], 0, h // 2].astype(np.float64))


def test_identical_keys_average_the_values():
    kc, vc = _cache()
    kc[:] = 0.25  # every score equal -> uniform weights
    table = _table([7], 4, 2)
    q = np.ones((1, 2, 8), dtype=np.float32)
    out = ao.paged_decode_attention(q, kc, vc, 0, table, np.array([7]), cache_dtype="float32")
    vals = np.stack([vc[0, table[0, t // 4], t % 4] for t in range(7)]).astype(np.float64)
    np.testing.assert_allclose(out[0], vals.mean(axis=0), rtol=1e-12)


def test_dominant_key_returns_its_value():
    kc, vc = _cache(kv_heads=1)
    kc[:] = 0.0
    kc[0, 1, 2, 0, :] = 50.0  # token 6 of the sequence (block 1, slot 2)
    table = _table([9], 4, 3)
    q = np.ones((1, 1, 8), dtype=np.float32)
    out = ao.paged_decode_attention(q, kc, vc, 0, table, np.array([9]), cache_dtype="float32")
    np.testing.assert_allclose(out[0, 0], vc[0, 1, 2, 0], rtol=1e-9)


@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (8, 8), (8, 1)])
def test_matches_torch_sdpa_with_gqa_and_padding(heads, kv_heads):
    kc, vc = _cache(blocks=32, kv_heads=kv_heads, seed=heads + kv_heads)
    ctx = [12, 20, 9, 1]
    table = _table(ctx, 4, 6)
    table[1, 2] = -1  # a hole: tokens 8-11 of sequence 1 are not keys
    q = np.random.default_rng(3).standard_normal((4, heads, 8)).astype(np.float32)
    out = ao.paged_decode_attention(q, kc, vc, 0, table, np.array(ctx), cache_dtype="float32")
    keys, values, valid = ao.kv_gather(kc, vc, 0, table, np.array(ctx))
    group = heads // kv_heads
    k = torch.from_numpy(keys).double().permute(0, 2, 1, 3).repeat_interleave(group, dim=1)
    v = torch.from_numpy(values).double().permute(0, 2, 1, 3).repeat_interleave(group, dim=1)
    mask = torch.from_numpy(valid)[:, None, None, :]
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).double()[:, :, None, :], k, v, attn_mask=mask
    )[:, :, 0]
    np.testing.assert_allclose(out, want.numpy(), rtol=1e-10, atol=1e-12)


def test_split_path_equals_dense():
    kc, vc = _cache(blocks=64, seed=5)
    ctx = [37, 5, 64]
    table = _table(ctx, 4, 16)
    q = np.random.default_rng(6).standard_normal((3, 4, 8)).astype(np.float32)
    dense = ao.paged_decode_attention(q, kc, vc, 0, table, np.array(ctx), cache_dtype="float32")
    split = ao.split_decode_attention(q, kc, vc, 0, table, np.array(ctx), 7, cache_dtype="float32")
    np.testing.assert_allclose(split, dense, rtol=1e-10, atol=1e-12)


def test_query_is_cast_to_the_cache_dtype():
    kc, vc = _cache(kv_heads=1)
    table = _table([5], 4, 2)
    q = np.full((1, 1, 8), 1.0 + 2.0**-12, dtype=np.float32)  # rounds to 1.0 in fp16
    a = ao.paged_decode_attention(q, kc, vc, 0, table, np.array([5]), cache_dtype="float16")
    b = ao.paged_decode_attention(np.ones_like(q), kc, vc, 0, table, np.array([5]), cache_dtype="float16")
    np.testing.assert_array_equal(a, b)


def test_no_key_gives_zeros():
    kc, vc = _cache()
    out = ao.paged_decode_attention(np.ones((2, 2, 8), np.float32), kc, vc, 0, _table([0, 3], 4, 2),
                                    np.array([0, 3]), cache_dtype="float32")
    assert not out[0].any() and out[1].any()


def test_write_decode_then_gather_round_trips():
    kc = np.zeros((2, 8, 4, 2, 8), np.float32)
    vc = np.zeros_like(kc)
    table = np.array([[3, 5, -1], [1, -1, -1], [7, 2, 4]])
    offsets = np.array([5, 2, 9])
    rng = np.random.default_rng(7)
    keys = rng.standard_normal((3, 2, 8)).astype(np.float32)
    kc2, vc2 = ao.kv_write_decode(kc, vc, 1, table, offsets, keys, keys * 2, dtype="float32")
    np.testing.assert_array_equal(kc2[1, 5, 1], keys[0])  # block table[0, 1] = 5, slot 1
    np.testing.assert_array_equal(kc2[1, 1, 2], keys[1])
    np.testing.assert_array_equal(vc2[1, 4, 1], keys[2] * 2)
    assert not kc2[0].any()  # other layers untouched


def test_write_decode_replaces_invalid_blocks_by_block_zero():
    kc = np.zeros((1, 4, 4, 1, 8), np.float32)
    table = np.array([[-1, 2], [9, -1]])
    keys = np.ones((2, 1, 8), np.float32)
    kc2, _ = ao.kv_write_decode(kc, kc.copy(), 0, table, np.array([1, 3]), keys, keys, dtype="float32")
    np.testing.assert_array_equal(kc2[0, 0, 1, 0], 1.0)
    np.testing.assert_array_equal(kc2[0, 0, 3, 0], 1.0)


def test_multi_token_write_stops_at_the_first_hole():
    kc = np.zeros((1, 8, 4, 1, 8), np.float32)
    table = np.array([[0, 1, -1, 3], [4, 5, 6, 7]])
    keys = np.arange(2 * 14 * 8, dtype=np.float32).reshape(2, 14, 1, 8)
    kc2, _ = ao.kv_write(kc, kc.copy(), 0, table, np.array([2, 3]), keys, keys, dtype="float32")
    # sequence 0: positions 2..7 written (blocks 0, 1), then block index 2 is -1: stop
    np.testing.assert_array_equal(kc2[0, 0, 2:, 0], keys[0, :2, 0])
    np.testing.assert_array_equal(kc2[0, 1, :, 0], keys[0, 2:6, 0])
    assert not kc2[0, 3].any()
    # sequence 1: positions 3..16 over blocks 4-7, then the row ends
    np.testing.assert_array_equal(kc2[0, 4, 3, 0], keys[1, 0, 0])
    np.testing.assert_array_equal(kc2[0, 7, :, 0], keys[1, 9:13, 0])


def test_prefill_single_token_at_the_end_equals_decode():
    kc, vc = _cache(blocks=32, seed=4)
    ctx = [12, 20, 9]
    table = _table(ctx, 4, 6)
    q = np.random.default_rng(5).standard_normal((3, 4, 8)).astype(np.float32)
    dec = ao.paged_decode_attention(q, kc, vc, 0, table, np.array(ctx), cache_dtype="float32")
    pre = ao.paged_prefill_attention(q[:, :, None, :], kc, vc, 0, table, np.array(ctx), cache_dtype="float32")
    np.testing.assert_array_equal(pre[:, :, 0], dec)


def test_prefill_first_token_sees_only_the_first_key():
    kc, vc = _cache(kv_heads=1, seed=6)
    table = _table([7], 4, 2)
    q = np.random.default_rng(7).standard_normal((1, 2, 7, 8)).astype(np.float32)
    out = ao.paged_prefill_attention(q, kc, vc, 0, table, np.array([7]), cache_dtype="float32")
    for h in range(2):
        np.testing.assert_array_equal(out[0, h, 0], vc[0, table[0, 0], 0, 0].astype(np.float64))


def test_prefill_identical_keys_average_the_values_up_to_each_position():
    kc, vc = _cache(kv_heads=1, seed=8)
    kc[:] = 0.5
    ctx, q_len = 10, 6  # four cached tokens, then six new ones at positions 4..9
    table = _table([ctx], 4, 3)
    q = np.ones((1, 1, q_len, 8), dtype=np.float32)
    out = ao.paged_prefill_attention(q, kc, vc, 0, table, np.array([ctx]), cache_dtype="float32")
    vals = np.stack([vc[0, table[0, t // 4], t % 4, 0] for t in range(ctx)]).astype(np.float64)
    for j in range(q_len):
        np.testing.assert_allclose(out[0, 0, j], vals[: ctx - q_len + j + 1].mean(axis=0), rtol=1e-12)


@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (8, 1)])
def test_prefill_matches_torch_sdpa_with_causal_and_padding_masks(heads, kv_heads):
    kc, vc = _cache(blocks=40, kv_heads=kv_heads, seed=heads)
    ctx, q_len = [12, 20, 5], 5
    table = _table(ctx, 4, 6)
    table[1, 1] = -1  # tokens 4-7 of sequence 1 are not keys
    q = np.random.default_rng(9).standard_normal((3, heads, q_len, 8)).astype(np.float32)
    out = ao.paged_prefill_attention(q, kc, vc, 0, table, np.array(ctx), cache_dtype="float32")
    keys, values, valid = ao.kv_gather(kc, vc, 0, table, np.array(ctx))
    group = heads // kv_heads
    k = torch.from_numpy(keys).double().permute(0, 2, 1, 3).repeat_interleave(group, dim=1)
    v = torch.from_numpy(values).double().permute(0, 2, 1, 3).repeat_interleave(group, dim=1)
    # Position of query j: ctx - q_len + j; key t is visible iff valid and t <= that position.
    qpos = torch.tensor(ctx)[:, None] - q_len + torch.arange(q_len)[None, :]
    causal = torch.arange(keys.shape[1])[None, None, :] <= qpos[:, :, None]
    mask = (torch.from_numpy(valid)[:, None, :] & causal)[:, None]
    want = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q).double(), k, v, attn_mask=mask)
    np.testing.assert_allclose(out, want.numpy(), rtol=1e-10, atol=1e-12)

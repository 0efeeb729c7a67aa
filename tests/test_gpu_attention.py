"""Paged KV-cache writes and decode attention on the GPU against the oracle.

Writes are bit-exact (a copy with one round-to-nearest-even conversion). Attention outputs are
compared with the oracle's float64 attention over the same cached values, as max |err| / max |ref|.
The kernel computes scores, softmax and sums in fp32, feeds the probabilities to the P V product
in the cache dtype (as the reference's probabilities tensor is in the cache dtype) and rounds the
output once into the query dtype; the bound is the coarser of the two dtypes' rounding: 1e-2 for
bf16, 2e-3 for fp16."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from llmopt.attention import PagedAttention, PagedAttentionConfig
from llmopt.cache import PagedKVCache
from llmopt.kernels import _lib, ops
from oracle import attention_oracle as ao

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.bfloat16: 1e-2, torch.float16: 2e-3, torch.float32: 1e-5}
NAMES = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


def _rel(got: np.ndarray, ref: np.ndarray) -> float:
    scale = max(float(np.abs(ref).max()), 1e-30)
    return float(np.abs(got.astype(np.float64) - ref).max()) / scale


def _table(ctx, block_size, width, num_blocks, seed, holes=()):
    rng = np.random.default_rng(seed)
    free = list(rng.permutation(num_blocks))
    table = np.full((len(ctx), width), -1, dtype=np.int32)
    for s, length in enumerate(ctx):
        n = min(-(-length // block_size), width)
        table[s, :n] = [free.pop() for _ in range(n)]
    for s, i in holes:
        table[s, i] = -1
    return table


def _filled_cache(blocks, block_size, kv_heads, head_dim, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    cache = PagedKVCache(1, blocks, block_size, kv_heads, head_dim, dtype=dtype, device=DEV)
    cache.key_cache.copy_(torch.randn(cache.key_cache.shape, generator=g).to(dtype))
    cache.value_cache.copy_(torch.randn(cache.value_cache.shape, generator=g).to(dtype))
    return cache


CASES = [  # (ctx, heads, kv_heads, head_dim, block_size, holes)
    ([12, 20, 9], 4, 2, 64, 8, ()),
    ([1, 15, 16, 17, 0, 33], 32, 8, 128, 16, ()),
    ([200, 75, 130], 16, 1, 128, 16, [(0, 3)]),
    ([64, 64], 8, 8, 64, 32, ()),
    ([300, 5, 1000, 47], 32, 2, 128, 16, [(2, 0), (2, 40)]),
    ([2000], 16, 16, 128, 16, ()),
    ([513, 1, 240], 32, 4, 64, 8, ()),
]


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_decode_attention_matches_oracle(case, cache_dtype, q_dtype):
    ctx, heads, kv_heads, head_dim, bs, holes = CASES[case]
    width = -(-max(ctx) // bs) + 1
    blocks = sum(-(-c // bs) for c in ctx) + 3
    cache = _filled_cache(blocks, bs, kv_heads, head_dim, cache_dtype, seed=case)
    table = _table(ctx, bs, width, blocks, seed=case, holes=holes)
    q = torch.randn(len(ctx), heads, head_dim, generator=torch.Generator().manual_seed(case + 7)).to(q_dtype)
    out = ops.paged_decode_attention(q.to(DEV), cache.key_cache[0], cache.value_cache[0],
                                     torch.from_numpy(table).to(DEV), torch.tensor(ctx).to(DEV), head_dim**-0.5)
    assert out.dtype == q_dtype and out.shape == q.shape
    ref = ao.paged_decode_attention(q.float().numpy(), cache.key_cache.float().cpu().numpy(),
                                    cache.value_cache.float().cpu().numpy(), 0, table, np.array(ctx),
                                    cache_dtype=NAMES[cache_dtype])
    got = out.float().cpu().numpy()
    assert _rel(got, ref) <= max(TOL[q_dtype], TOL[cache_dtype]), (case, cache_dtype, q_dtype)
    for s, c in enumerate(ctx):  # no keys -> exact zeros
        if c == 0:
            assert not got[s].any()


def test_unsplit_launch_agrees_with_split():
    ctx, heads, kv_heads, head_dim, bs = [700, 1500, 3], 32, 8, 128, 16
    blocks = 200
    cache = _filled_cache(blocks, bs, kv_heads, head_dim, torch.bfloat16, seed=3)
    table = torch.from_numpy(_table(ctx, bs, 100, blocks, seed=3)).to(DEV)
    lens = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    q = torch.randn(3, heads, head_dim, device=DEV).to(torch.bfloat16)
    split = ops.paged_decode_attention(q, cache.key_cache[0], cache.value_cache[0], table, lens, 0.125)
    lib = _lib.load_library()
    assert lib.llmopt_paged_attention_workspace(3, heads, kv_heads, head_dim, 100, bs) > 0
    whole = torch.empty_like(q)
    rc = lib.llmopt_paged_attention_decode(
        q.data_ptr(), 2, heads * head_dim, cache.key_cache.data_ptr(), cache.value_cache.data_ptr(), 2, blocks, bs,
        kv_heads, head_dim, table.data_ptr(), 100, lens.data_ptr(), 3, heads, ctypes.c_float(0.125),
        ctypes.c_float(0.0), whole.data_ptr(), None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert _rel(whole.float().cpu().numpy(), split.float().cpu().numpy().astype(np.float64)) <= 1e-2


def test_softcap():
    ctx = [40, 90]
    cache = _filled_cache(16, 16, 2, 64, torch.float16, seed=9)
    cache.key_cache.mul_(4)  # large scores, so the cap matters
    table = _table(ctx, 16, 8, 16, seed=9)
    q = torch.randn(2, 8, 64).to(torch.float16)
    out = ops.paged_decode_attention(q.to(DEV), cache.key_cache[0], cache.value_cache[0],
                                     torch.from_numpy(table).to(DEV), torch.tensor(ctx).to(DEV), 0.125, 5.0)
    ref = ao.paged_decode_attention(q.float().numpy(), cache.key_cache.float().cpu().numpy(),
                                    cache.value_cache.float().cpu().numpy(), 0, table, np.array(ctx), scale=0.125,
                                    softcap=5.0, cache_dtype="float16")
    assert _rel(out.float().cpu().numpy(), ref) <= 2e-3


def test_module_uses_the_kernel_and_agrees_with_the_torch_sequence():
    ctx = [37, 300, 128, 1]
    cache = _filled_cache(64, 16, 8, 128, torch.bfloat16, seed=11)
    table = torch.from_numpy(_table(ctx, 16, 24, 64, seed=11)).to(DEV)
    lens = torch.tensor(ctx, device=DEV)
    q = torch.randn(4, 32, 1, 128, device=DEV).to(torch.bfloat16)
    fast = PagedAttention(32, 8, 128, config=PagedAttentionConfig(block_size=16)).forward(q, cache, 0, table, lens)
    slow = PagedAttention(32, 8, 128, config=PagedAttentionConfig(block_size=16), backend="sdpa").forward(
        q, cache, 0, table, lens)
    assert fast.shape == slow.shape == (4, 32, 1, 128) and fast.dtype == torch.bfloat16
    # The torch sequence rounds scores, probabilities and partial outputs to bf16 on the way.
    assert _rel(fast.float().cpu().numpy(), slow.float().cpu().numpy().astype(np.float64)) <= 2e-2


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("src_dtype", [torch.float32, torch.bfloat16])
def test_write_decode_bit_exact(cache_dtype, src_dtype):
    cache = PagedKVCache(2, 12, 4, 2, 64, dtype=cache_dtype, device=DEV)
    table = np.array([[3, 9, -1], [1, 7, 2], [-1, 6, 5], [4, 30, 8]], dtype=np.int32)  # 30, -1: block 0
    offsets = np.array([5, 9, 1, 6])
    keys = torch.randn(4, 2, 64).to(src_dtype)
    values = torch.randn(4, 2, 64).to(src_dtype)
    cache.write_decode(1, torch.from_numpy(table).to(DEV), torch.from_numpy(offsets).to(DEV), keys.to(DEV),
                       values.to(DEV))
    zero = np.zeros((2, 12, 4, 2, 64), np.float32)
    want_k, want_v = ao.kv_write_decode(zero, zero.copy(), 1, table, offsets, keys.float().numpy(),
                                        values.float().numpy(), dtype=NAMES[cache_dtype])
    np.testing.assert_array_equal(cache.key_cache.float().cpu().numpy(), want_k)
    np.testing.assert_array_equal(cache.value_cache.float().cpu().numpy(), want_v)


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float32])
def test_multi_token_write_bit_exact(cache_dtype):
    cache = PagedKVCache(1, 16, 4, 2, 32, dtype=cache_dtype, device=DEV)
    table = np.array([[0, 1, -1, 3], [4, 5, 6, 7], [9, 10, 11, -1], [12, 13, 14, 15]], dtype=np.int32)
    offsets = np.array([2, 3, 0, 11])
    keys = torch.randn(4, 9, 2, 32)
    cache.write(0, torch.from_numpy(table).to(DEV), torch.from_numpy(offsets).to(DEV), keys.to(DEV),
                (keys * 2).to(DEV))
    zero = np.zeros((1, 16, 4, 2, 32), np.float32)
    want_k, want_v = ao.kv_write(zero, zero.copy(), 0, table, offsets, keys.numpy(), (keys * 2).numpy(),
                                 dtype=NAMES[cache_dtype])
    np.testing.assert_array_equal(cache.key_cache.float().cpu().numpy(), want_k)
    np.testing.assert_array_equal(cache.value_cache.float().cpu().numpy(), want_v)


def test_decode_step_write_then_attend_at_llama_shape():
    """32 sequences of 512-640 tokens, 32 query / 8 KV heads of 128, block 16, bf16 cache: write
    this step's K/V, then attend, against the oracle on the same cache."""
    rng = np.random.default_rng(5)
    ctx = rng.integers(512, 641, size=32)
    blocks = int(sum(-(-c // 16) for c in ctx)) + 8
    cache = _filled_cache(blocks, 16, 8, 128, torch.bfloat16, seed=5)
    table = _table(list(ctx), 16, 41, blocks, seed=5)
    new_k = torch.randn(32, 8, 128).to(torch.bfloat16)
    cache.write_decode(0, torch.from_numpy(table).to(DEV), torch.from_numpy(ctx - 1).to(DEV), new_k.to(DEV),
                       new_k.to(DEV))
    q = torch.randn(32, 32, 128).to(torch.bfloat16)
    out = ops.paged_decode_attention(q.to(DEV), cache.key_cache[0], cache.value_cache[0],
                                     torch.from_numpy(table).to(DEV), torch.from_numpy(ctx).to(DEV), 128**-0.5)
    ref = ao.paged_decode_attention(q.float().numpy(), cache.key_cache.float().cpu().numpy(),
                                    cache.value_cache.float().cpu().numpy(), 0, table, ctx, cache_dtype="bfloat16")
    assert _rel(out.float().cpu().numpy(), ref) <= 1e-2
    last = [(table[s, (c - 1) // 16], (c - 1) % 16) for s, c in enumerate(ctx)]
    got = torch.stack([cache.key_cache[0, b, slot] for b, slot in last]).cpu()
    assert torch.equal(got, new_k)


def test_unsupported_shapes_fall_back_to_the_torch_sequence():
    cache = _filled_cache(8, 8, 2, 8, torch.float32, seed=2)  # head_dim 8, fp32 cache
    table = torch.tensor([[0, 1], [2, 3]], device=DEV)
    q = torch.randn(2, 4, 1, 8, device=DEV)
    with pytest.raises(NotImplementedError):
        ops.paged_decode_attention(q[:, :, 0], cache.key_cache[0], cache.value_cache[0], table,
                                   torch.tensor([10, 5], device=DEV), 0.3)
    out = PagedAttention(4, 2, 8, config=PagedAttentionConfig(block_size=8)).forward(
        q, cache, 0, table, torch.tensor([10, 5], device=DEV))
    ref = ao.paged_decode_attention(q[:, :, 0].cpu().numpy(), cache.key_cache.cpu().numpy(),
                                    cache.value_cache.cpu().numpy(), 0, table.cpu().numpy(), np.array([10, 5]),
                                    cache_dtype="float32")
    assert _rel(out[:, :, 0].cpu().numpy(), ref) <= 1e-5

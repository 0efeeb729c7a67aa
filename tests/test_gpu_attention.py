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


@pytest.mark.parametrize("q_dtype,code", [(torch.bfloat16, 2), (torch.float32, 0)])
def test_unaligned_query_rows_take_element_loads(q_dtype, code):
    """Query rows that are not 16-byte aligned (an odd element offset and row stride) are read
    element by element; the output equals the aligned call's bit for bit."""
    ctx, heads, kv_heads, head_dim, bs = [300, 41, 129], 16, 4, 128, 16
    blocks = 64
    cache = _filled_cache(blocks, bs, kv_heads, head_dim, torch.bfloat16, seed=12)
    table = torch.from_numpy(_table(ctx, bs, 20, blocks, seed=12)).to(DEV)
    lens = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    stride = heads * head_dim + 3
    buf = torch.randn(3 * stride + 8, device=DEV).to(q_dtype)
    q_odd = buf[1 : 1 + 3 * stride].view(3, stride)[:, : heads * head_dim]
    assert q_odd.data_ptr() % 16 != 0
    aligned = ops.paged_decode_attention(q_odd.reshape(3, heads, head_dim).contiguous(), cache.key_cache[0],
                                         cache.value_cache[0], table, lens, 0.1)
    lib = _lib.load_library()
    ws_bytes = lib.llmopt_paged_attention_workspace(3, heads, kv_heads, head_dim, 20, bs)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    odd = torch.empty(3, heads, head_dim, dtype=q_dtype, device=DEV)
    rc = lib.llmopt_paged_attention_decode(
        q_odd.data_ptr(), code, stride, cache.key_cache.data_ptr(), cache.value_cache.data_ptr(), 2, blocks, bs,
        kv_heads, head_dim, table.data_ptr(), 20, lens.data_ptr(), 3, heads, ctypes.c_float(0.1), ctypes.c_float(0.0),
        odd.data_ptr(), ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert torch.equal(odd, aligned)


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


PREFILL_CASES = [  # (ctx, q_len, heads, kv_heads, head_dim, block_size, holes, softcap)
    ([512, 512], 512, 32, 8, 128, 16, (), 0.0),  # Llama-3-8B heads, prompts with no prefix
    ([40, 100, 13], 13, 4, 2, 64, 8, (), 0.0),  # a prefix before the 13 new tokens; a partial tile
    ([300, 77], 64, 16, 1, 128, 16, [(0, 3)], 0.0),  # a hole in the prefix
    ([33, 64], 33, 8, 8, 64, 32, (), 30.0),  # soft-capped scores, one query head per KV head
    ([200], 100, 16, 16, 128, 16, (), 0.0),  # sixteen query heads per KV head: one token per tile
    ([20, 9], 20, 32, 4, 64, 8, (), 0.0),  # context shorter than q_len: early tokens see no key
    ([90, 50], 50, 8, 2, 128, 16, (), 0.0),  # a prefix; the last wave's later column blocks empty
]


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("q_dtype", [None, torch.float32])
@pytest.mark.parametrize("case", range(len(PREFILL_CASES)))
def test_prefill_attention_matches_oracle(case, q_dtype, cache_dtype):
    ctx, q_len, heads, kv_heads, head_dim, bs, holes, softcap = PREFILL_CASES[case]
    q_dtype = q_dtype or cache_dtype
    width = -(-max(ctx) // bs) + 1
    blocks = sum(-(-c // bs) for c in ctx) + 3
    cache = _filled_cache(blocks, bs, kv_heads, head_dim, cache_dtype, seed=case)
    table = _table(ctx, bs, width, blocks, seed=case, holes=holes)
    g = torch.Generator().manual_seed(case + 17)
    # [seq, q_len, heads, d] seen as [seq, heads, q_len, d], the layout the attention layer passes
    q = torch.randn(len(ctx), q_len, heads, head_dim, generator=g).to(q_dtype)
    query = q.to(DEV).permute(0, 2, 1, 3)
    out = ops.paged_prefill_attention(query, cache.key_cache[0], cache.value_cache[0], torch.from_numpy(table).to(DEV),
                                      torch.tensor(ctx).to(DEV), head_dim**-0.5, softcap)
    assert out.shape == (len(ctx), heads, q_len, head_dim) and out.dtype == q_dtype
    ref = ao.paged_prefill_attention(q.permute(0, 2, 1, 3).float().numpy(), cache.key_cache.float().cpu().numpy(),
                                     cache.value_cache.float().cpu().numpy(), 0, table, np.array(ctx),
                                     softcap=softcap, cache_dtype=NAMES[cache_dtype])
    got = out.float().cpu().numpy()
    assert _rel(got, ref) <= max(TOL[q_dtype], TOL[cache_dtype]), (case, cache_dtype, q_dtype)
    no_key = ref == 0  # queries that see no key: exact zeros
    assert not got[no_key.all(axis=-1)].any()
    # A contiguous [seq, heads, q_len, d] query gives the same output bit for bit.
    again = ops.paged_prefill_attention(query.contiguous(), cache.key_cache[0], cache.value_cache[0],
                                        torch.from_numpy(table).to(DEV), torch.tensor(ctx).to(DEV), head_dim**-0.5,
                                        softcap)
    assert torch.equal(again, out)


def test_prefill_module_uses_the_kernel_and_agrees_with_the_torch_sequence(monkeypatch):
    ctx, q_len = [160, 96], 96
    cache = _filled_cache(24, 16, 8, 128, torch.bfloat16, seed=21)
    table = torch.from_numpy(_table(ctx, 16, 12, 24, seed=21)).to(DEV)
    lens = torch.tensor(ctx, device=DEV)
    q = torch.randn(2, 32, q_len, 128, device=DEV).to(torch.bfloat16)
    calls = []
    original = ops.paged_prefill_attention
    monkeypatch.setattr(ops, "paged_prefill_attention", lambda *a, **k: calls.append(1) or original(*a, **k))
    fast = PagedAttention(32, 8, 128, config=PagedAttentionConfig(block_size=16)).forward(q, cache, 0, table, lens)
    slow = PagedAttention(32, 8, 128, config=PagedAttentionConfig(block_size=16), backend="sdpa").forward(
        q, cache, 0, table, lens)
    assert calls == [1]
    assert fast.shape == slow.shape == (2, 32, q_len, 128) and fast.dtype == torch.bfloat16
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


def _private_table(ctx, block_size, width, num_blocks, seed):
    """Block tables drawn from blocks 1 .. num_blocks - 1 (block 0 is never a key), one block per
    started block of each context plus one, -1 past that."""
    rng = np.random.default_rng(seed)
    free = list(rng.permutation(np.arange(1, num_blocks)))
    table = np.full((len(ctx), width), -1, dtype=np.int32)
    for s, length in enumerate(ctx):
        n = min(-(-length // block_size) + 1, width)
        table[s, :n] = [free.pop() for _ in range(n)]
    return table


def _rope_step(ctx, heads, kvh, d, bs, dtype, seed, offsets=None, table=None, softcap=0.0):
    """Both ways of one decode step on the same inputs: rope_kv_write_decode then
    paged_decode_attention, and paged_decode_attention_rope; returns both outputs and caches."""
    from llmopt.model import RotaryEmbedding

    seqs = len(ctx)
    width = -(-max(max(ctx), 1) // bs) + 2
    nb = seqs * width + 2
    if table is None:
        table = _private_table(ctx, bs, width, nb, seed)
    gen = torch.Generator().manual_seed(seed)
    fused = torch.randn(seqs, (heads + 2 * kvh) * d, generator=gen).to(dtype).to(DEV)
    q = fused[:, : heads * d].view(seqs, heads, d)
    k = fused[:, heads * d : (heads + kvh) * d].view(seqs, kvh, d)
    v = fused[:, (heads + kvh) * d :].view(seqs, kvh, d)
    offs = np.array(ctx) - 1 if offsets is None else np.array(offsets)
    pos = torch.from_numpy(np.clip(offs, 0, None)).to(DEV)
    rot = RotaryEmbedding(d, 4096, base=500000.0).to(DEV)
    init_k = torch.randn(nb, bs, kvh, d, generator=gen).to(dtype).to(DEV)
    init_v = torch.randn(nb, bs, kvh, d, generator=gen).to(dtype).to(DEV)
    kc1, vc1 = init_k.clone(), init_v.clone()
    kc2, vc2 = init_k.clone(), init_v.clone()
    t = torch.from_numpy(table).to(DEV)
    lens = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    o = torch.from_numpy(offs.astype(np.int32)).to(DEV)
    q1 = ops.rope_kv_write_decode(q, k, v, pos, rot.cos_cached, rot.sin_cached, kc1, vc1, t, o)
    out1 = ops.paged_decode_attention(q1, kc1, vc1, t, lens, d**-0.5, softcap)
    out2 = ops.paged_decode_attention_rope(q, k, v, pos, rot.cos_cached, rot.sin_cached, kc2, vc2, t, lens, o,
                                           d**-0.5, softcap)
    torch.cuda.synchronize()
    return out1, out2, (kc1, vc1), (kc2, vc2), init_k


ROPE_CASES = [  # (ctx, heads, kv_heads, head_dim, block_size, softcap)
    (list(np.random.default_rng(11).integers(512, 641, size=32)), 32, 8, 128, 16, 0.0),
    ([12, 20, 9], 4, 2, 64, 8, 0.0),
    ([200, 75, 130, 1], 16, 1, 128, 16, 0.0),
    ([64, 64, 3], 8, 8, 64, 32, 30.0),
    ([2000], 16, 16, 128, 16, 0.0),  # the context in five splits, the new token in the last
    ([513, 1, 240], 32, 4, 64, 8, 0.0),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", range(len(ROPE_CASES)))
def test_fused_rope_attention_equals_rope_write_then_attend(case, dtype):
    """The one-launch decode step returns the two calls' output bit for bit and leaves the same
    caches (the new token's k and v at its slot)."""
    ctx, heads, kvh, d, bs, softcap = ROPE_CASES[case]
    out1, out2, c1, c2, init_k = _rope_step([int(c) for c in ctx], heads, kvh, d, bs, dtype, seed=case,
                                            softcap=softcap)
    assert out2.shape == (len(ctx), heads, d) and out2.dtype == dtype
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(c1[0], c2[0]) and torch.equal(c1[1], c2[1])
    assert not torch.equal(c2[0], init_k)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_rope_attention_offsets_off_the_last_position(dtype):
    """Offsets that are not context - 1: past the context (written, not a key), inside it (the key
    at that position is replaced), past the table row or negative (nothing written), and a slot
    whose block id is past the pool (written into block 0, which no sequence reads here)."""
    ctx = [30, 17, 40, 5, 64, 33, 20]
    offsets = [29, 20, 12, 4, 80, 32, -3]
    bs, width, nb = 16, 5, 40
    table = _private_table(ctx, bs, width, nb, seed=3)
    table[5, 2] = nb + 7
    out1, out2, c1, c2, _ = _rope_step(ctx, 8, 2, 128, bs, dtype, seed=4, offsets=offsets, table=table)
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(c1[0], c2[0]) and torch.equal(c1[1], c2[1])


def test_fused_rope_attention_refuses_unaligned_rows():
    """Rows off 16-byte alignment are refused before anything runs (NotImplementedError: the
    attention layer then takes the rotary kernel and the attention kernel), caches untouched."""
    from llmopt.model import RotaryEmbedding

    seqs, heads, kvh, d, bs = 2, 8, 2, 128, 16
    buf = torch.randn(seqs, (heads + 2 * kvh) * d + 1, device=DEV).to(torch.bfloat16)
    q = buf[:, 1 : 1 + heads * d].view(seqs, heads, d)
    k = buf[:, 1 + heads * d : 1 + (heads + kvh) * d].view(seqs, kvh, d)
    v = buf[:, 1 + (heads + kvh) * d :].view(seqs, kvh, d)
    kc = torch.zeros(8, bs, kvh, d, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    rot = RotaryEmbedding(d, 64, base=10000.0).to(DEV)
    table = torch.tensor([[1, 2], [3, 4]], dtype=torch.int32, device=DEV)
    lens = torch.tensor([5, 20], dtype=torch.int32, device=DEV)
    with pytest.raises(NotImplementedError):
        ops.paged_decode_attention_rope(q, k, v, (lens - 1).long(), rot.cos_cached, rot.sin_cached, kc, vc, table,
                                        lens, lens - 1, d**-0.5)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(kc)) == 0 and int(torch.count_nonzero(vc)) == 0


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

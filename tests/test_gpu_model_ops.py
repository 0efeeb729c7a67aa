"""The decoder's fused elementwise kernels against the reference's torch sequences:
llmopt_rope (bit-identical to apply_rotary_pos_emb with the tables cast to the dtype,
src/llmopt/model/rotary.py:23-45,85-102) and llmopt_rmsnorm (RMSNorm.forward with the residual
add before it, src/llmopt/model/layers.py:14-31,185-195)."""

from __future__ import annotations

import pytest
import torch

from llmopt.kernels import ops
from llmopt.model import RMSNorm, RotaryEmbedding, apply_rotary_pos_emb

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads,kv_heads,d", [(32, 8, 128), (4, 2, 64), (6, 0, 16)])
def test_rope_is_bit_identical_to_the_torch_sequence(dtype, heads, kv_heads, d):
    g = torch.Generator(device=DEV).manual_seed(heads + d)
    tokens = 37
    rope = RotaryEmbedding(d, 4096, base=500000.0).to(DEV)
    # q and k as column slices of one fused projection output, as the model passes them
    fused = torch.randn(tokens, (heads + 2 * kv_heads) * d, generator=g, device=DEV).to(dtype)
    q = fused[:, : heads * d].view(tokens, heads, d)
    k = fused[:, heads * d : (heads + kv_heads) * d].view(tokens, kv_heads, d)
    positions = torch.randint(0, 4096, (tokens,), generator=g, device=DEV)
    v = fused[:, (heads + kv_heads) * d :].view(tokens, kv_heads, d)
    got_q, got_k = ops.rope(q, k, positions, rope.cos_cached, rope.sin_cached)
    cos, sin = rope(positions, dtype=dtype)
    want_q, want_k = apply_rotary_pos_emb(q, k, cos[:, None, :], sin[:, None, :])
    assert got_q.is_contiguous() and got_k.is_contiguous()
    assert torch.equal(got_q, want_q)
    assert torch.equal(got_k, want_k)
    q3, k3, v3 = ops.rope(q, k, positions, rope.cos_cached, rope.sin_cached, v=v)
    assert torch.equal(q3, want_q) and torch.equal(k3, want_k)
    assert v3.is_contiguous() and torch.equal(v3, v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_on_unaligned_rows_is_bit_identical_too(dtype):
    # Rows off 16-byte alignment take the element-wise kernel: the same results.
    g = torch.Generator(device=DEV).manual_seed(3)
    tokens, heads, kv_heads, d = 9, 4, 2, 64
    rope = RotaryEmbedding(d, 512, base=10000.0).to(DEV)
    fused = torch.randn(tokens, 1 + (heads + 2 * kv_heads) * d, generator=g, device=DEV).to(dtype)
    q = fused[:, 1 : 1 + heads * d].view(tokens, heads, d)
    k = fused[:, 1 + heads * d : 1 + (heads + kv_heads) * d].view(tokens, kv_heads, d)
    v = fused[:, 1 + (heads + kv_heads) * d :].view(tokens, kv_heads, d)
    positions = torch.randint(0, 512, (tokens,), generator=g, device=DEV)
    got_q, got_k, got_v = ops.rope(q, k, positions, rope.cos_cached, rope.sin_cached, v=v)
    cos, sin = rope(positions, dtype=dtype)
    want_q, want_k = apply_rotary_pos_emb(q, k, cos[:, None, :], sin[:, None, :])
    assert torch.equal(got_q, want_q) and torch.equal(got_k, want_k) and torch.equal(got_v, v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,hidden", [(1, 4096), (32, 4096), (5, 264)])
@torch.no_grad()
def test_rmsnorm_with_residual_matches_the_torch_sequence(dtype, rows, hidden):
    g = torch.Generator(device=DEV).manual_seed(rows * hidden)
    norm = RMSNorm(hidden, eps=1e-5).to(DEV, dtype)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(hidden, generator=g, device=DEV) + 0.5)
    x = torch.randn(rows, hidden, generator=g, device=DEV).to(dtype)
    r = (torch.randn(rows, hidden, generator=g, device=DEV) * 4).to(dtype)
    y, h = ops.rmsnorm(x, norm.weight, norm.eps, r)
    assert torch.equal(h, r + x)  # the add rounds exactly as torch's
    want = norm._reference(r + x)
    # fp32 arithmetic in a different summation order, rounded once: at most one unit in the
    # last place of the dtype (at most 2^-7 relative for bf16, 2^-10 for fp16) on a few elements
    ulp = 2.0**-7 if dtype == torch.bfloat16 else 2.0**-10
    diff = (y.float() - want.float()).abs()
    assert float((diff / want.float().abs().clamp_min(1e-3)).max()) <= 1.01 * ulp
    assert float((diff > 0).float().mean()) < 0.05
    y2, none = ops.rmsnorm(x, norm.weight, norm.eps)
    assert none is None
    assert float(((y2.float() - norm._reference(x).float()).abs() / norm._reference(x).float().abs().clamp_min(1e-3)).max()) <= 1.01 * ulp


@torch.no_grad()
def test_rmsnorm_module_takes_the_kernel_on_hip():
    norm = RMSNorm(4096).to(DEV, torch.bfloat16)
    x = torch.randn(3, 4096, device=DEV).to(torch.bfloat16)
    assert ops.rmsnorm_supported(x, norm.weight)
    assert not ops.rmsnorm_supported(x.float(), norm.weight.float())
    y = norm(x)
    assert torch.equal(y, ops.rmsnorm(x, norm.weight, norm.eps)[0])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@torch.no_grad()
def test_rope_kv_write_decode_matches_rope_then_write(dtype):
    # The fused decode kernel against llmopt_rope followed by llmopt_kv_write_decode: the same
    # q bit for bit and the same caches, including a block id past the pool (-> block 0) and
    # an offset past the table row (nothing written).
    seqs, heads, kvh, d, nb, bs = 6, 8, 2, 128, 12, 16
    gen = torch.Generator().manual_seed(7)
    q = torch.randn(seqs, heads * d + 64, generator=gen).to(dtype).to(DEV)[:, : heads * d].view(seqs, heads, d)
    k = torch.randn(seqs, kvh, d, generator=gen).to(dtype).to(DEV)
    v = torch.randn(seqs, kvh, d, generator=gen).to(dtype).to(DEV)
    pos = torch.tensor([0, 5, 17, 31, 40, 63], device=DEV)
    rot = RotaryEmbedding(d, 128, base=500000.0).to(DEV)
    table = torch.randint(0, nb, (seqs, 4), generator=gen, dtype=torch.int32).to(DEV)
    table[2, 1] = nb + 3
    offsets = torch.tensor([0, 5, 17, 31, 40, 64], dtype=torch.int32, device=DEV)
    init = torch.randn(nb, bs, kvh, d, generator=gen).to(dtype).to(DEV)
    kc1, vc1 = init.clone(), init.clone() * 2
    kc2, vc2 = kc1.clone(), vc1.clone()
    q1, k1, v1 = ops.rope(q, k, pos, rot.cos_cached, rot.sin_cached, v=v)
    ops.kv_write_decode(kc1, vc1, table, offsets, k1, v1)
    q2 = ops.rope_kv_write_decode(q, k, v, pos, rot.cos_cached, rot.sin_cached, kc2, vc2, table, offsets)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2)
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert not torch.equal(kc2, init)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,cols", [(32, 128256), (3, 1001), (1, 8), (5, 7)])
def test_argmax_rows_matches_torch(dtype, rows, cols):
    """The greedy sampler's argmax (torch.argmax(logits, dim=-1), sampler.py:94-95): the first
    maximum of each row, including ties, NaN (above every number, the first one wins), -inf
    rows, a tail past the 16-byte pieces, and rows read element by element (odd stride)."""
    g = torch.Generator().manual_seed(rows * cols)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    if rows >= 3:
        x[0] = 0.0  # all equal: index 0
        x[1, cols // 3] = 50.0
        x[1, cols // 2] = 50.0  # a tie: the first
        x[2] = -float("inf")
        if cols > 4:
            x[2, cols - 2] = float("nan")
            x[2, cols - 1] = float("nan")
    want = torch.argmax(x, dim=-1)
    got = ops.argmax_rows(x.to(DEV))
    assert got.dtype == torch.long and torch.equal(got.cpu(), want)
    assert torch.equal(got, torch.argmax(x.to(DEV), dim=-1))
    wide = torch.zeros(rows, cols + 3, dtype=dtype)
    wide[:, 1 : cols + 1] = x
    odd = wide.to(DEV)[:, 1 : cols + 1]  # rows off 16-byte alignment
    assert torch.equal(ops.argmax_rows(odd).cpu(), want)
    # Into a caller's buffer (the greedy generator's step input).
    buf = torch.full((rows,), -7, dtype=torch.long, device=DEV)
    assert ops.argmax_rows(x.to(DEV), out=buf) is buf and torch.equal(buf.cpu(), want)


def test_argmax_rows_out_is_checked():
    x = torch.randn(4, 100).to(DEV)
    for bad in (torch.empty(4, dtype=torch.int32, device=DEV), torch.empty(5, dtype=torch.long, device=DEV),
                torch.empty(8, dtype=torch.long, device=DEV)[::2], torch.empty(4, dtype=torch.long)):
        with pytest.raises(ValueError):
            ops.argmax_rows(x, out=bad)

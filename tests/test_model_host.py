"""The decoder model on the host: RoPE and RMSNorm against their closed forms, the paged-cache
path against the cache-free causal forward, fused against unfused projections, and the
config checks (src/llmopt/model/*.py, src/llmopt/config.py:34-78)."""

from __future__ import annotations

import math

import pytest
import torch

from llmopt.model import (GreedyGenerator, ModelConfig, RMSNorm, RotaryEmbedding, apply_rotary_pos_emb,
                          fuse_projections_, random_quantized_model, rotate_half)
from llmopt.model.layers import DecoderLayer
from llmopt.quantization import FusedQuantLinear, QuantLinear, QuantSwiGLU


def test_rotate_half_and_rotation_preserve_pair_norms():
    x = torch.arange(8, dtype=torch.float64)
    assert torch.equal(rotate_half(x), torch.tensor([-4, -5, -6, -7, 0, 1, 2, 3], dtype=torch.float64))
    rope = RotaryEmbedding(64, 128, base=10000.0, dtype=torch.float64)
    q = torch.randn(5, 64, dtype=torch.float64, generator=torch.Generator().manual_seed(0))
    cos, sin = rope(torch.arange(5))
    qr, _ = apply_rotary_pos_emb(q, q, cos, sin)
    # dims i and i + 32 form a plane rotated by an angle: their joint norm is unchanged
    assert torch.allclose(q[:, :32] ** 2 + q[:, 32:] ** 2, qr[:, :32] ** 2 + qr[:, 32:] ** 2, atol=1e-12)


def test_rotation_angles_follow_the_rope_formula():
    rope = RotaryEmbedding(16, 64, base=500000.0, dtype=torch.float64)
    cos, sin = rope(torch.tensor([0, 7, 63]))
    for row, p in enumerate((0, 7, 63)):
        for i in range(8):
            theta = p * 500000.0 ** (-2 * i / 16)
            assert math.isclose(float(cos[row, i]), math.cos(theta), abs_tol=1e-6)
            assert math.isclose(float(sin[row, i + 8]), math.sin(theta), abs_tol=1e-6)


def test_rotated_dot_products_depend_only_on_relative_position():
    rope = RotaryEmbedding(32, 256, dtype=torch.float64)
    g = torch.Generator().manual_seed(3)
    q, k = torch.randn(32, dtype=torch.float64, generator=g), torch.randn(32, dtype=torch.float64, generator=g)

    def score(m: int, n: int) -> float:
        cq, sq = rope(torch.tensor([m]))
        ck, sk = rope(torch.tensor([n]))
        qr = q * cq[0] + rotate_half(q) * sq[0]
        kr = k * ck[0] + rotate_half(k) * sk[0]
        return float(qr @ kr)

    # The angle table is built in fp32, as the reference builds it: an angle at position p is off
    # by up to about p * 2^-23 rad, so the invariance holds to |q| |k| (m + n) 2^-23.
    bound = float(q.norm() * k.norm()) * 2.0**-23
    for shift in (1, 17, 100):
        assert abs(score(5, 2) - score(5 + shift, 2 + shift)) <= bound * (7 + 2 * shift + 7)
    assert abs(score(5, 2) - score(6, 2)) > 1e-3  # and it does depend on the relative position


def test_positions_past_the_table_raise():
    rope = RotaryEmbedding(16, 8)
    with pytest.raises(ValueError):
        rope(torch.tensor([8]))


def test_rmsnorm_matches_its_closed_form():
    norm = RMSNorm(48, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(torch.linspace(0.5, 1.5, 48))
    x = torch.randn(7, 48, generator=torch.Generator().manual_seed(1))
    x64 = x.double()
    want = x64 / torch.sqrt((x64 * x64).mean(-1, keepdim=True) + 1e-5) * norm.weight.double()
    assert torch.allclose(norm(x).double(), want, rtol=1e-6, atol=1e-6)
    assert norm(x.to(torch.bfloat16)).dtype == torch.bfloat16


def test_config_checks_and_presets():
    with pytest.raises(ValueError):
        ModelConfig(hidden_size=100, num_attention_heads=16)
    with pytest.raises(ValueError):
        ModelConfig(num_attention_heads=16, num_key_value_heads=5)
    with pytest.raises(ValueError):
        ModelConfig(intermediate_size=2817)
    llama = ModelConfig.llama3_8b()
    assert (llama.head_dim, llama.num_query_groups, llama.vocab_size) == (128, 4, 128256)
    assert ModelConfig.from_dict(llama.to_dict() | {"unknown": 1}) == llama


@pytest.fixture(scope="module")
def tiny_model():
    return random_quantized_model(ModelConfig.tiny(), device="cpu", dtype=torch.float32, seed=0)


def test_random_quantized_model_is_built_on_the_device(tiny_model):
    for name, t in list(tiny_model.named_parameters()) + list(tiny_model.named_buffers()):
        assert t.device.type == "cpu", name
    layer = tiny_model.layers[0]
    assert isinstance(layer.self_attn.qkv_proj, FusedQuantLinear)
    assert isinstance(layer.mlp.gate_up, QuantSwiGLU)
    assert isinstance(layer.self_attn.o_proj, QuantLinear) and isinstance(layer.mlp.down_proj, QuantLinear)
    assert isinstance(tiny_model.lm_head, torch.nn.Linear)


def test_paged_generation_matches_the_cache_free_forward(tiny_model):
    cfg = tiny_model.config
    prompts = torch.randint(0, cfg.vocab_size, (3, 21), generator=torch.Generator().manual_seed(4))
    res = GreedyGenerator(tiny_model, block_size=16).generate(prompts, 7)
    full = torch.cat([prompts, res.tokens[:, :-1]], dim=1)
    seqs, length = full.shape
    out = tiny_model(full.reshape(-1), torch.arange(length).repeat(seqs), q_len=length).logits
    assert torch.equal(out.argmax(-1)[:, prompts.shape[1] - 1:], res.tokens)
    assert torch.allclose(out[:, prompts.shape[1] - 1].float(), res.prefill_logits, rtol=1e-4, atol=1e-5)


def test_teacher_forcing_feeds_the_given_tokens(tiny_model):
    cfg = tiny_model.config
    prompts = torch.randint(0, cfg.vocab_size, (2, 9), generator=torch.Generator().manual_seed(5))
    forced = torch.randint(0, cfg.vocab_size, (2, 5), generator=torch.Generator().manual_seed(6))
    res = GreedyGenerator(tiny_model).generate(prompts, 5, forced=forced)
    full = torch.cat([prompts, forced[:, :-1]], dim=1)
    seqs, length = full.shape
    out = tiny_model(full.reshape(-1), torch.arange(length).repeat(seqs), q_len=length).logits
    assert torch.equal(out.argmax(-1)[:, prompts.shape[1] - 1:], res.tokens)


def test_last_only_logits_equal_the_last_position_of_all_logits(tiny_model):
    ids = torch.randint(0, 512, (2 * 6,), generator=torch.Generator().manual_seed(7))
    pos = torch.arange(6).repeat(2)
    full = tiny_model(ids, pos, q_len=6).logits
    last = tiny_model(ids, pos, q_len=6, last_only=True)
    assert last.logits.shape == (2, 1, 512)
    assert torch.allclose(last.last_logits(), full[:, -1], rtol=1e-5, atol=1e-6)


def test_fused_projections_give_the_unfused_result():
    model = random_quantized_model(ModelConfig.tiny(), device="cpu", dtype=torch.float32, seed=1, fuse=False)
    assert isinstance(model.layers[0].self_attn.q_proj, QuantLinear)
    ids = torch.randint(0, 512, (10,), generator=torch.Generator().manual_seed(8))
    pos = torch.arange(10)
    before = model(ids, pos, q_len=10).logits
    assert fuse_projections_(model) == 2 * len(model.layers)
    assert fuse_projections_(model) == 2 * len(model.layers)  # idempotent
    after = model(ids, pos, q_len=10).logits
    assert torch.allclose(before, after, rtol=1e-4, atol=1e-5)


def test_quantize_model_then_fuse_on_a_dense_model():
    from llmopt.model import DecoderOnlyModel
    from llmopt.quantization import quantize_model_

    torch.manual_seed(0)
    model = DecoderOnlyModel(ModelConfig.tiny())
    quantize_model_(model, bits=4, group_size=128, symmetric=False)
    assert isinstance(model.lm_head, torch.nn.Linear) and not isinstance(model.lm_head, QuantLinear)
    assert fuse_projections_(model) == 4
    layer = next(m for m in model.modules() if isinstance(m, DecoderLayer))
    assert not hasattr(layer.self_attn, "q_proj") and not hasattr(layer.mlp, "gate_proj")


def test_reference_twin_computes_the_same_model_densely():
    from llmopt.model import reference_twin

    model = random_quantized_model(ModelConfig.tiny(), device="cpu", dtype=torch.float32, seed=2, fuse=False)
    twin = reference_twin(model)
    assert type(twin.layers[0].self_attn.q_proj) is torch.nn.Linear
    assert not twin.layers[0].input_layernorm.fused_ops and twin.layers[0].self_attn.attn.backend == "sdpa"
    fuse_projections_(model)
    with pytest.raises(ValueError):
        reference_twin(model)
    prompts = torch.randint(0, 512, (2, 11), generator=torch.Generator().manual_seed(9))
    a = GreedyGenerator(model).generate(prompts, 4)
    b = GreedyGenerator(twin).generate(prompts, 4)
    assert torch.equal(a.tokens, b.tokens)
    assert torch.allclose(a.prefill_logits, b.prefill_logits, rtol=1e-5, atol=1e-6)

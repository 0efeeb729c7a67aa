"""QuantLinear and the model-wide helpers on the host, against the reference's contract.

Includes the reference's own quantization tests (tests/test_engine_and_serving.py:73-96),
run on a small decoder-shaped model with the same awkward shapes as the reference's tiny
preset: hidden 64, FFN 176 (so group 64 falls back to gcd(176, 64) = 16 and the packed
row of down_proj is 88 bytes), and 32-wide k/v projections.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from llmopt.quantization import (
    QuantLinear,
    QuantLinearConfig,
    RoundToNearestQuantizer,
    quantize_model_,
    replace_linear_modules,
)
from llmopt.quantization.calibration import (
    CalibrationHarness,
    HessianCollector,
    apply_quantization,
)
from oracle import quant_oracle as qo


class _Block(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.q_proj = nn.Linear(64, 64, bias=False)
        self.k_proj = nn.Linear(64, 32, bias=False)
        self.v_proj = nn.Linear(64, 32, bias=False)
        self.o_proj = nn.Linear(64, 64, bias=False)
        self.gate_proj = nn.Linear(64, 176, bias=False)
        self.up_proj = nn.Linear(64, 176, bias=False)
        self.down_proj = nn.Linear(176, 64, bias=False)

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        q, k, v = self.q_proj(h), self.k_proj(h), self.v_proj(h)
        mix = torch.cat([k, v], dim=-1) * q.sigmoid()
        h = h + self.o_proj(mix)
        return h + self.down_proj(torch.nn.functional.silu(self.gate_proj(h)) * self.up_proj(h))


class TinyDecoder(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.embed_tokens = nn.Embedding(256, 64)
        self.layers = nn.ModuleList([_Block(), _Block()])
        self.lm_head = nn.Linear(64, 256, bias=False)
        for p in self.parameters():
            with torch.no_grad():
                p.copy_(torch.randn_like(p) * 0.02)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        h = self.embed_tokens(ids)
        for layer in self.layers:
            h = layer(h)
        return self.lm_head(h)


def _tiny():
    torch.manual_seed(0)
    return TinyDecoder()


def test_quantize_model_replaces_linears_and_shrinks_storage():
    model = _tiny()
    float_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
    quantize_model_(model, bits=4, group_size=64)
    layers = [m for m in model.modules() if isinstance(m, QuantLinear)]
    assert len(layers) == 14
    assert isinstance(model.lm_head, nn.Linear) and not isinstance(model.lm_head, QuantLinear)
    packed = sum(
        m.qweight.numel() * m.qweight.element_size()
        + m.scales.numel() * m.scales.element_size()
        + m.qzeros.numel() * m.qzeros.element_size()
        for m in layers
    )
    assert packed < float_bytes
    down = model.layers[0].down_proj
    assert down.config.group_size == 16 and down.qweight.shape == (64, 88)


@pytest.mark.parametrize("bits", [8, 4, 2])
def test_quantized_model_still_runs(bits):
    model = _tiny()
    quantize_model_(model, bits=bits, group_size=64)
    out = model(torch.randint(0, 256, (1, 8)))
    assert torch.isfinite(out).all()


def test_forward_equals_reference_sequence():
    torch.manual_seed(1)
    linear = nn.Linear(256, 48, bias=True)
    qt = RoundToNearestQuantizer(4, 128, False).quantize(linear.weight.detach())
    module = QuantLinear.from_float(linear, qt)
    x = torch.randn(5, 256)
    dense = qo.dequantize(qt.qweight.numpy(), qt.scales.numpy(), qt.zeros.numpy(), 4, 128, False, (48, 256))
    expect = qo.reference_linear(x, torch.from_numpy(dense), linear.bias.detach())
    torch.testing.assert_close(module(x), expect, rtol=0, atol=0)
    assert module.config.compute_dtype == torch.float32
    assert module(x[0]).shape == (48,)
    assert module(torch.randn(2, 3, 256)).shape == (2, 3, 48)


def test_forward_errors_follow_f_linear():
    linear = nn.Linear(64, 16, bias=False)
    qt = RoundToNearestQuantizer(4, 64, True).quantize(linear.weight.detach())
    module = QuantLinear.from_float(linear, qt, compute_dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        module(torch.randn(2, 64))  # fp32 input, bf16 compute dtype
    assert module(torch.randn(2, 64, dtype=torch.bfloat16)).dtype == torch.bfloat16
    empty = QuantLinear(64, 16)
    with pytest.raises(RuntimeError, match="no quantized weight"):
        empty(torch.randn(1, 64, dtype=torch.float16))


def test_constructor_defaults_and_repr():
    module = QuantLinear(32, 8)
    cfg = module.config
    assert (cfg.bits, cfg.group_size, cfg.symmetric, cfg.compute_dtype) == (4, 128, True, torch.float16)
    assert module.qweight is None and module.qzeros.numel() == 0
    assert isinstance(module.bias, nn.Parameter) and module.bias.shape == (8,)
    assert QuantLinear(32, 8, bias=False).bias is None
    assert module.extra_repr() == "in_features=32, out_features=8, bits=4, bias=True"
    cfg2 = QuantLinearConfig(bits=8, group_size=64, symmetric=False, compute_dtype=torch.bfloat16)
    with pytest.raises(AttributeError):
        cfg2.extra = 1  # __slots__


def test_cache_invalidate_and_state_dict():
    linear = nn.Linear(64, 16, bias=False)
    qt = RoundToNearestQuantizer(8, 32, True).quantize(linear.weight.detach())
    module = QuantLinear.from_float(linear, qt)
    x = torch.randn(1, 64)
    module(x)
    assert module._cached_weight is not None
    module.invalidate()
    assert module._cached_weight is None
    state = module.state_dict()
    assert {"qweight", "scales", "qzeros"} <= set(state)
    assert state["qweight"].dtype == torch.int8
    # Moving or casting the module drops the host cache and leaves the codes untouched.
    module(x)
    module.to(torch.float64)
    assert module._cached_weight is None and module.qweight.dtype == torch.int8


def test_replace_linear_modules_swaps_children():
    model = nn.Sequential(nn.Linear(4, 4), nn.ReLU(), nn.Linear(4, 2))
    new = nn.Identity()
    replace_linear_modules(model, {model[2]: new})
    assert model[2] is new
    assert replace_linear_modules(model, {}) is model


def test_gptq_strategy_with_calibration_batches():
    model = _tiny()
    batches = CalibrationHarness(num_samples=2, seq_length=16, seed=3).synthetic(256)
    quantize_model_(model, bits=4, group_size=64, strategy="gptq", calibration_batches=batches)
    assert isinstance(model.layers[1].up_proj, QuantLinear)
    assert torch.isfinite(model(batches[0])).all()


def test_hessian_collector_closed_form():
    layer = nn.Linear(8, 4)
    x1, x2 = torch.randn(3, 8), torch.randn(2, 5, 8)
    with HessianCollector([layer]) as collector:
        layer(x1)
        layer(x2)
    rows = torch.cat([x1, x2.reshape(-1, 8)])
    torch.testing.assert_close(collector.hessian_for(layer), (2.0 / 13) * rows.T @ rows)
    assert collector.count == 2 and layer in collector.results()
    assert HessianCollector([nn.Linear(2, 2)]).hessian_for(layer) is None


def test_apply_quantization_writes_dequantized_weights():
    model = _tiny()
    before = model.layers[0].q_proj.weight.detach().clone()
    result = apply_quantization(model, strategy="rtn", bits=4, group_size=16)
    after = model.layers[0].q_proj.weight.detach()
    qt = result.quantizers["layers.0.q_proj"]
    np.testing.assert_array_equal(after.numpy(), qt.dequantize().numpy())
    assert result.per_layer_error["layers.0.q_proj"] > 0
    assert not torch.equal(before, after)
    assert result.compression_ratio > 1 and "layers to 4-bit" in result.summary()
    assert "quantized=rtn-4bit" in repr(model.layers[0].q_proj)


def test_one_calibration_pass_equals_a_pass_per_layer():
    # collect_hessians hooks every layer at once; a pass per layer (the reference's loop,
    # calibration.py:180-190) must give the same Gram matrices, bit for bit.
    from llmopt.quantization.calibration import collect_hessians

    model = _tiny()
    layers = [m for n, m in model.named_modules() if isinstance(m, nn.Linear) and "lm_head" not in n]
    batches = CalibrationHarness(num_samples=3, seq_length=8, seed=1).synthetic(256)
    together = collect_hessians(model, layers, batches, stop_at_failure=True)
    assert len(together) == len(layers)
    for layer in layers:
        with HessianCollector([layer]) as alone:
            for batch in batches:
                model(batch)
        assert torch.equal(together[layer], alone.hessian_for(layer))


def test_collect_hessians_failure_policies():
    from llmopt.quantization.calibration import collect_hessians

    model = _tiny()
    layer = model.layers[0].q_proj
    good = torch.randint(0, 256, (1, 4))
    bad = torch.full((1, 4), 999)  # out of the embedding's range: the forward raises
    skip = collect_hessians(model, [layer], [good, bad, good], stop_at_failure=False)
    stop = collect_hessians(model, [layer], [good, bad, good], stop_at_failure=True)
    one = collect_hessians(model, [layer], [good], stop_at_failure=True)
    torch.testing.assert_close(skip[layer], one[layer])  # two equal batches: same (2/n) X^T X
    torch.testing.assert_close(stop[layer], one[layer])
    assert collect_hessians(model, [layer], [bad], stop_at_failure=False) == {}
    # 1-D batches get a batch dimension when asked to (apply_quantization's convention).
    flat = collect_hessians(model, [layer], [good[0]], stop_at_failure=True, add_batch_dim=True)
    torch.testing.assert_close(flat[layer], one[layer])


def test_gptq_apply_quantization_uses_calibration_hessians():
    from llmopt.quantization import GPTQQuantizer
    from llmopt.quantization.calibration import collect_hessians

    model = _tiny()
    batches = CalibrationHarness(num_samples=2, seq_length=16, seed=5).synthetic(256)
    layer = model.layers[1].gate_proj
    h = collect_hessians(model, [layer], batches, stop_at_failure=False)[layer]
    expect = GPTQQuantizer(bits=4, group_size=16, symmetric=True).quantize(layer.weight.detach().clone(), h)
    # apply_quantization takes group_size as given (no gcd fallback): 16 divides every width.
    result = apply_quantization(model, strategy="gptq", bits=4, group_size=16, calibration_batches=batches)
    got = result.quantizers["layers.1.gate_proj"]
    assert torch.equal(got.qweight, expect.qweight) and torch.equal(got.scales, expect.scales)
    with pytest.raises(ValueError):
        apply_quantization(_tiny(), strategy="awq")


def test_replace_linear_modules_shared_child_and_nested_replacement():
    shared = nn.Linear(4, 4)
    model = nn.Sequential(nn.Sequential(shared), nn.Sequential(shared))
    new = nn.Sequential(nn.Linear(4, 4))
    replace_linear_modules(model, {shared: new, new[0]: nn.Identity()})
    # One slot per module, the last parent found (quant_linear.py:129-135 keys its map by child).
    assert model[0][0] is shared and model[1][0] is new
    assert isinstance(new[0], nn.Linear)  # the replacement's own children are not visited


def test_harness_batches_follow_the_seeded_per_sample_draws():
    harness = CalibrationHarness(num_samples=4, seq_length=6, seed=9)
    gen = torch.Generator().manual_seed(9)
    expect = [torch.randint(0, 50, (1, 6), generator=gen, dtype=torch.long) for _ in range(4)]
    got = harness.synthetic(50)
    assert len(got) == 4 and all(torch.equal(a, b) for a, b in zip(got, expect))

    class Tok:
        def encode(self, text):
            return [ord(c) for c in text]

    rows = CalibrationHarness(seq_length=5).from_tokenizer(Tok(), ["abc", "", "abcdefg"])
    assert [r.tolist() for r in rows] == [[[97, 98, 99, 0, 0]], [[97, 98, 99, 100, 101]]]
    with pytest.raises(TypeError):
        CalibrationHarness().from_tokenizer(object(), ["x"])


def test_partial_sums_materialize_in_slice_order_then_bias():
    # PartialSums.materialize is the split-K reduction's arithmetic: slices added in order, then
    # the bias, one rounding to the output dtype.
    from llmopt.kernels.ops import PartialSums

    g = torch.Generator().manual_seed(0)
    planes = torch.randn(5, 3, 16, generator=g) * torch.tensor([1e8, 1.0, -1e8, 1e-3, 7.0]).view(5, 1, 1)
    bias = torch.randn(16, generator=g).to(torch.bfloat16)
    got = PartialSums(planes, bias, torch.bfloat16, (3, 16)).materialize()
    v = planes[0]
    for s in range(1, 5):
        v = v + planes[s]
    assert torch.equal(got.view(torch.int16), (v + bias.float()).to(torch.bfloat16).view(torch.int16))
    assert got.shape == (3, 16) and got.dtype == torch.bfloat16

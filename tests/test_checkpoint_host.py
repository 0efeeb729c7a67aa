"""The packed checkpoint (``llmopt.quantization.checkpoint``) round-trips a quantized model.

The reference loses the packed codes on save (``src/llmopt/quantization/quant_linear.py:57,81``)
and reloads dense layers (``src/llmopt/model/modeling.py:149-177``). Here a model quantized with
``quantize_model_`` is saved, a freshly built float model of the same architecture loads the
checkpoint, and its outputs, packed codes and dense layers are identical bit for bit.
"""

from __future__ import annotations

import json

import pytest
import torch
from torch import nn

from llmopt.quantization import QuantLinear, is_quantized_checkpoint, load_quantized_, quantize_model_, save_quantized


class TinyBlock(nn.Module):
    def __init__(self, seed: int, bias: bool = True) -> None:
        super().__init__()
        torch.manual_seed(seed)
        self.embed_tokens = nn.Embedding(32, 256)
        self.up = nn.Linear(256, 512, bias=bias)
        self.down = nn.Linear(512, 256, bias=False)
        self.norm = nn.LayerNorm(256)
        self.lm_head = nn.Linear(256, 32, bias=False)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        h = self.embed_tokens(ids)
        h = h + self.down(torch.relu(self.up(h)))
        return self.lm_head(self.norm(h))


@pytest.mark.parametrize("bits,symmetric,group", [(4, False, 128), (4, True, 64), (8, False, 128), (2, False, 128)])
def test_round_trip_is_bit_exact(tmp_path, bits, symmetric, group):
    model = quantize_model_(TinyBlock(0), bits=bits, group_size=group, symmetric=symmetric)
    ids = torch.randint(0, 32, (3, 7), generator=torch.Generator().manual_seed(1))
    ref = model(ids)
    save_quantized(model, tmp_path / "ckpt")
    assert is_quantized_checkpoint(tmp_path / "ckpt")

    fresh = TinyBlock(seed=99)  # different random init everywhere
    load_quantized_(fresh, tmp_path / "ckpt")
    assert isinstance(fresh.up, QuantLinear) and isinstance(fresh.down, QuantLinear)
    assert isinstance(fresh.lm_head, nn.Linear) and not isinstance(fresh.lm_head, QuantLinear)
    assert torch.equal(fresh.up.qweight, model.up.qweight)
    assert torch.equal(fresh.down.scales, model.down.scales)
    assert torch.equal(fresh.embed_tokens.weight, model.embed_tokens.weight)
    assert torch.equal(fresh(ids), ref)


def test_checkpoint_stores_packed_codes(tmp_path):
    model = quantize_model_(TinyBlock(0), bits=4, group_size=128, symmetric=False)
    save_quantized(model, tmp_path / "ckpt")
    meta = json.loads((tmp_path / "ckpt" / "quantization.json").read_text())
    assert meta["format"] == "llmopt-packed" and meta["version"] == 1
    assert set(meta["modules"]) == {"up", "down"}
    assert meta["modules"]["up"]["bits"] == 4 and meta["modules"]["up"]["bias"] is True
    size = (tmp_path / "ckpt" / "quantized.safetensors").stat().st_size
    dense_linear_bytes = (256 * 512 + 512 * 256) * 4
    assert size < dense_linear_bytes  # the two big linears are stored packed (about 1/7 of fp32)


def test_load_rejects_mismatched_models(tmp_path):
    model = quantize_model_(TinyBlock(0), bits=4, group_size=128, symmetric=False)
    save_quantized(model, tmp_path / "ckpt")

    class Wider(TinyBlock):
        def __init__(self) -> None:
            super().__init__(0)
            self.up = nn.Linear(256, 1024)

    with pytest.raises(ValueError):
        load_quantized_(Wider(), tmp_path / "ckpt")

    class Missing(nn.Module):
        def __init__(self) -> None:
            super().__init__()
            self.up = nn.Linear(256, 512)

    with pytest.raises(KeyError):
        load_quantized_(Missing(), tmp_path / "ckpt")
    with pytest.raises(ValueError):
        load_quantized_(TinyBlock(0), tmp_path)  # not a checkpoint directory
    with pytest.raises(ValueError):
        save_quantized(TinyBlock(0), tmp_path / "dense")  # nothing quantized


def test_non_strict_load_keeps_extra_modules(tmp_path):
    model = quantize_model_(TinyBlock(0), bits=4, group_size=128, symmetric=False)
    save_quantized(model, tmp_path / "ckpt")

    class Extra(TinyBlock):
        def __init__(self) -> None:
            super().__init__(5)
            self.extra = nn.Linear(4, 4)

    with pytest.raises(RuntimeError):
        load_quantized_(Extra(), tmp_path / "ckpt")
    m = load_quantized_(Extra(), tmp_path / "ckpt", strict=False)
    assert isinstance(m.up, QuantLinear)

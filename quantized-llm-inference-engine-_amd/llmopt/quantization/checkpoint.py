"""A persistent packed checkpoint: save a quantized model, load it without re-quantizing.

The reference cannot round-trip a quantized model: ``QuantLinear`` keeps ``qweight`` as a plain
attribute, so ``state_dict`` drops the codes (``src/llmopt/quantization/quant_linear.py:57,81``),
and ``from_pretrained`` rebuilds plain ``nn.Linear`` layers and loads with ``strict=False``
(``src/llmopt/model/modeling.py:149-177``). Every run therefore quantizes again at load time.

Format: a directory with

* ``quantized.safetensors``: every tensor of the model's ``state_dict`` (for a ``QuantLinear``:
  ``qweight`` packed as stored, ``scales``, ``qzeros`` and ``bias``), contiguous, no pickles;
* ``quantization.json``: ``{"format": "llmopt-packed", "version": 1, "modules": {name: {...}}}``
  with, per ``QuantLinear``, ``in_features``, ``out_features``, ``bits``, ``group_size``,
  ``symmetric``, ``compute_dtype`` and ``bias``.

:func:`load_quantized_` takes a model built with plain ``nn.Linear`` layers (as the
architecture code builds it), swaps in ``QuantLinear`` modules made from the stored tensors and
loads every other tensor. Fused projections (:mod:`llmopt.quantization.fused`) are derived from
``QuantLinear`` modules at run time and are not stored.
"""

from __future__ import annotations

import json
import os
from pathlib import Path

import torch
from torch import nn

from llmopt.quantization.quant_linear import QuantLinear, QuantLinearConfig

__all__ = ["FORMAT", "VERSION", "is_quantized_checkpoint", "load_quantized_", "save_quantized"]

FORMAT = "llmopt-packed"
VERSION = 1
TENSORS = "quantized.safetensors"
MANIFEST = "quantization.json"


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).removeprefix("torch.")


def _dtype(name: str) -> torch.dtype:
    value = getattr(torch, name, None)
    if not isinstance(value, torch.dtype):
        raise ValueError(f"unknown dtype in checkpoint: {name!r}")
    return value


def save_quantized(model: nn.Module, output_dir: str | os.PathLike) -> Path:
    """Write ``model``'s packed weights and the rest of its state to ``output_dir``."""
    from safetensors.torch import save_file

    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    modules = {}
    for name, module in model.named_modules():
        if isinstance(module, QuantLinear):
            if module.qweight is None or not hasattr(module, "scales"):
                raise RuntimeError(f"QuantLinear {name!r} has no quantized weight; call from_float()")
            cfg = module.config
            modules[name] = {
                "in_features": module.in_features,
                "out_features": module.out_features,
                "bits": int(cfg.bits),
                "group_size": int(cfg.group_size),
                "symmetric": bool(cfg.symmetric),
                "compute_dtype": _dtype_name(cfg.compute_dtype),
                "bias": module.bias is not None,
            }
    if not modules:
        raise ValueError("the model has no QuantLinear modules to save")
    # safetensors stores contiguous, unshared tensors only.
    state = {k: v.detach().to("cpu").contiguous().clone() for k, v in model.state_dict().items() if v is not None}
    tmp = out / (TENSORS + ".tmp")
    save_file(state, str(tmp), metadata={"format": FORMAT, "version": str(VERSION)})
    os.replace(tmp, out / TENSORS)
    manifest = {"format": FORMAT, "version": VERSION, "modules": modules}
    tmp_json = out / (MANIFEST + ".tmp")
    tmp_json.write_text(json.dumps(manifest, indent=2, sort_keys=True), encoding="utf-8")
    os.replace(tmp_json, out / MANIFEST)
    return out


def is_quantized_checkpoint(path: str | os.PathLike) -> bool:
    """True if ``path`` holds a checkpoint written by :func:`save_quantized`."""
    p = Path(path)
    if not (p / MANIFEST).is_file() or not (p / TENSORS).is_file():
        return False
    try:
        meta = json.loads((p / MANIFEST).read_text(encoding="utf-8"))
    except (OSError, ValueError):
        return False
    return meta.get("format") == FORMAT


def _parent(model: nn.Module, name: str) -> tuple[nn.Module, str]:
    parent_name, _, child = name.rpartition(".")
    return (model.get_submodule(parent_name) if parent_name else model), child


def load_quantized_(
    model: nn.Module,
    checkpoint_dir: str | os.PathLike,
    *,
    strict: bool = True,
    device: torch.device | str | None = None,
) -> nn.Module:
    """Swap ``model``'s linears for the stored ``QuantLinear``s and load all stored tensors.

    ``model`` must have a module (``nn.Linear`` or ``QuantLinear``) at every stored name with the
    stored shape. With ``strict`` every other stored tensor must match a parameter or buffer of
    ``model`` and vice versa (as ``load_state_dict(strict=True)``). Returns ``model``.
    """
    from safetensors.torch import load_file

    path = Path(checkpoint_dir)
    if not is_quantized_checkpoint(path):
        raise ValueError(f"{path} is not an {FORMAT} checkpoint")
    meta = json.loads((path / MANIFEST).read_text(encoding="utf-8"))
    if int(meta.get("version", 0)) > VERSION:
        raise ValueError(f"checkpoint version {meta.get('version')} is newer than supported {VERSION}")
    state = load_file(str(path / TENSORS), device="cpu")

    for name, spec in meta["modules"].items():
        try:
            current = model.get_submodule(name)
        except AttributeError as exc:
            raise KeyError(f"model has no module {name!r} for the stored quantized weight") from exc
        if not isinstance(current, (nn.Linear, QuantLinear)):
            raise TypeError(f"module {name!r} is a {type(current).__name__}, not a linear layer")
        if (current.in_features, current.out_features) != (spec["in_features"], spec["out_features"]):
            raise ValueError(
                f"module {name!r} is {current.in_features}->{current.out_features}, "
                f"the checkpoint stores {spec['in_features']}->{spec['out_features']}"
            )
        config = QuantLinearConfig(spec["bits"], spec["group_size"], spec["symmetric"], _dtype(spec["compute_dtype"]))
        prefix = f"{name}." if name else ""
        q = QuantLinear(spec["in_features"], spec["out_features"], config, bias=spec["bias"])
        q.qweight = state.pop(prefix + "qweight")
        q.register_buffer("scales", state.pop(prefix + "scales"))
        q.register_buffer("qzeros", state.pop(prefix + "qzeros"))
        if spec["bias"]:
            q.bias.data = state.pop(prefix + "bias").to(config.compute_dtype)  # type: ignore[union-attr]
        q.invalidate()
        if device is not None:
            q = q.to(device)
        parent, child = _parent(model, name)
        setattr(parent, child, q)

    quant_names = tuple(f"{n}." for n in meta["modules"])
    rest = {k: v for k, v in state.items() if not k.startswith(quant_names)}
    missing, unexpected = model.load_state_dict(rest, strict=False)
    missing = [k for k in missing if not k.startswith(quant_names)]
    if strict and (missing or unexpected):
        raise RuntimeError(f"checkpoint does not match the model: missing {missing}, unexpected {unexpected}")
    return model

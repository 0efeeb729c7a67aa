"""Calibration for GPTQ: input second moments per layer, and whole-model quantization.

Public surface of ``src/llmopt/quantization/calibration.py`` (``HessianCollector``,
``CalibrationResult``, ``apply_quantization``, ``CalibrationHarness``), built around one
shared step, :func:`collect_hessians`: every target layer is hooked at once and the
calibration batches run through the model a single time. Forward hooks see each layer's
input rows whether one layer or all of them are hooked, so the Gram matrices are the ones
a pass per layer would give, for one forward per batch instead of one per batch and layer.

Offline code: what it produces is the packed layout the HIP kernels consume.
"""

from __future__ import annotations

import contextlib
from collections.abc import Iterable, Iterator, Sequence
from dataclasses import dataclass, field

import torch
from torch import nn

from llmopt.quantization.quantizers import QuantizedTensor, build_quantizer
from llmopt.utils.logging import get_logger

__all__ = ["CalibrationHarness", "CalibrationResult", "HessianCollector", "apply_quantization", "collect_hessians"]

logger = get_logger("quant.calibration")


@dataclass(slots=True)
class _Moments:
    """Running ``X^T X`` (fp32) and the number of rows that went into it."""

    gram: torch.Tensor
    rows: int = 0


class HessianCollector:
    """Accumulates ``X^T X`` of every input row a layer sees, through forward hooks.

    ``hessian_for(layer)`` is ``(2 / rows) X^T X`` in fp32 (``calibration.py:28-86``): the
    GPTQ objective's Hessian. Use as a context manager; the hooks go when it exits.
    """

    def __init__(self, layers: Sequence[nn.Module], device: torch.device | str = "cpu") -> None:
        self.layers = list(layers)
        self.device = torch.device(device)
        self._moments: dict[int, _Moments] = {}
        self._handles: list[torch.utils.hooks.RemovableHandle] = []
        self.count = 0  # hook calls that contributed rows

    def _record(self, layer: nn.Module, inputs: tuple[object, ...], _output: object) -> None:
        x = inputs[0] if inputs else None
        if not isinstance(x, torch.Tensor):
            return
        rows = x.detach().reshape(-1, x.shape[-1]).to(self.device, torch.float32)
        moments = self._moments.get(id(layer))
        if moments is None:
            width = layer.weight.shape[1]
            moments = _Moments(torch.zeros(width, width, dtype=torch.float32, device=self.device))
            self._moments[id(layer)] = moments
        moments.gram.addmm_(rows.T, rows)
        moments.rows += rows.shape[0]
        self.count += 1

    def __enter__(self) -> HessianCollector:
        self._handles.extend(layer.register_forward_hook(self._record) for layer in self.layers)
        return self

    def __exit__(self, *exc: object) -> None:
        while self._handles:
            self._handles.pop().remove()

    def hessian_for(self, module: nn.Module) -> torch.Tensor | None:
        """``(2/n) X^T X`` for ``module``, or ``None`` if it saw no rows."""
        moments = self._moments.get(id(module))
        if moments is None or moments.rows == 0:
            return None
        return moments.gram * (2.0 / moments.rows)

    def results(self) -> dict[nn.Module, torch.Tensor]:
        """Hessians of the layers that saw at least one row, keyed by layer."""
        pairs = ((layer, self.hessian_for(layer)) for layer in self.layers)
        return {layer: h for layer, h in pairs if h is not None}


def collect_hessians(
    model: nn.Module,
    layers: Sequence[nn.Module],
    batches: Iterable[torch.Tensor],
    *,
    stop_at_failure: bool,
    add_batch_dim: bool = False,
) -> dict[nn.Module, torch.Tensor]:
    """Run ``batches`` through ``model`` once with every layer in ``layers`` hooked.

    Each layer's Gram matrix lives on that layer's weight device; batches go to the device
    of the first layer. A batch whose forward raises is skipped, or ends the collection when
    ``stop_at_failure`` is set (rows the layers saw before the failure stay counted, as they
    would with a pass per layer). ``add_batch_dim`` turns 1-D token batches into ``[1, T]``.
    """
    if not layers:
        return {}
    by_device: dict[torch.device, list[nn.Module]] = {}
    for layer in layers:
        by_device.setdefault(layer.weight.device, []).append(layer)
    target = layers[0].weight.device
    with contextlib.ExitStack() as stack:
        collectors = [stack.enter_context(HessianCollector(group, device=dev)) for dev, group in by_device.items()]
        for batch in batches:
            tokens = batch.to(target)
            if add_batch_dim and tokens.dim() == 1:
                tokens = tokens[None]
            try:
                model(tokens)
            except Exception as exc:  # calibration is best effort: a failing batch is not fatal
                logger.debug("calibration batch failed: %s", exc)
                if stop_at_failure:
                    break
    found: dict[nn.Module, torch.Tensor] = {}
    for collector in collectors:
        found.update(collector.results())
    return found


@dataclass(slots=True)
class CalibrationResult:
    """What :func:`apply_quantization` did: packed tensors and errors per layer (``calibration.py:89-112``)."""

    quantizers: dict[str, QuantizedTensor] = field(default_factory=dict)
    mean_relative_error: float = 0.0
    per_layer_error: dict[str, float] = field(default_factory=dict)
    baseline_bits: int = 0
    quant_bits: int = 0

    @property
    def compression_ratio(self) -> float:
        """Dense bytes over packed bytes of all layers (1.0 when nothing was quantized)."""
        tensors = list(self.quantizers.values())
        if not tensors:
            return 1.0
        return sum(t.dense_nbytes() for t in tensors) / max(1, sum(t.nbytes() for t in tensors))

    def summary(self) -> str:
        return (
            f"quantized {len(self.quantizers)} layers to {self.quant_bits}-bit, "
            f"mean relative error {self.mean_relative_error:.5f}, "
            f"{self.compression_ratio:.2f}x compression"
        )


def _eligible(model: nn.Module, ignore: Sequence[str]) -> list[tuple[str, nn.Linear]]:
    """(name, layer) of every ``nn.Linear`` that no ``ignore`` token names and that packs.

    Sub-byte codes go two per byte, so a layer with an odd input width is left dense.
    """

    def wanted(name: str, module: nn.Module) -> bool:
        if not isinstance(module, nn.Linear) or any(tok in name for tok in ignore):
            return False
        if module.in_features % 2:
            logger.debug("skipping %s: in_features=%d is odd", name, module.in_features)
            return False
        return True

    return [(name, module) for name, module in model.named_modules() if wanted(name, module)]


@torch.no_grad()
def _relative_error(original: torch.Tensor, approx: torch.Tensor) -> float:
    """``||W - W_q|| / ||W||`` (Frobenius, fp32); 0 for an all-zero ``W``."""
    ref = original.float()
    norm = float(torch.linalg.vector_norm(ref))
    return 0.0 if norm == 0.0 else float(torch.dist(ref, approx.float())) / norm


@torch.no_grad()
def apply_quantization(
    model: nn.Module,
    *,
    strategy: str = "gptq",
    bits: int = 4,
    group_size: int = 128,
    symmetric: bool = True,
    damping: float = 0.01,
    act_order: bool = True,
    ignore_layers: Sequence[str] = ("lm_head", "embed_tokens"),
    calibration_batches: Sequence[torch.Tensor] | None = None,
    in_place: bool = False,
) -> CalibrationResult:
    """Quantize every eligible ``nn.Linear`` of ``model`` and keep it dense (fake quantization).

    Behaviour of ``calibration.py:137-221``: each layer's weight is replaced by the
    dequantization of its quantized form, and the packed tensors and per-layer relative
    errors are returned. ``strategy`` is ``"gptq"`` or ``"rtn"`` (anything else raises
    ``ValueError`` from :func:`build_quantizer`); GPTQ uses the Hessians that
    ``calibration_batches`` give (batches that fail are skipped) and falls back to
    round-to-nearest for a layer without one. The model is always changed in place
    (``in_place`` is accepted for signature compatibility).
    """
    del in_place
    result = CalibrationResult(quant_bits=bits)
    targets = _eligible(model, ignore_layers)
    if not targets:
        logger.warning("no quantizable linear layers found")
        return result

    hessians: dict[nn.Module, torch.Tensor] = {}
    if strategy == "gptq" and calibration_batches:
        hessians = collect_hessians(model, [m for _, m in targets], calibration_batches,
                                    stop_at_failure=False, add_batch_dim=True)
        logger.info("collected Hessians for %d/%d layers", len(hessians), len(targets))

    quantizer = build_quantizer(strategy, bits=bits, group_size=group_size, symmetric=symmetric,
                                damping=damping, act_order=act_order)
    for name, layer in targets:
        original = layer.weight.detach().clone()
        packed = quantizer.quantize(original, hessians.get(layer))
        approx = packed.dequantize().to(original.dtype)
        error = _relative_error(original, approx)
        result.quantizers[name] = packed
        result.per_layer_error[name] = error
        result.baseline_bits += 8 * original.numel() * original.element_size()
        layer.weight.data = approx.to(layer.weight.device)
        note = f"quantized={quantizer.name}-{bits}bit, group_size={group_size}, err={error:.4f}"
        layer.extra_repr = lambda note=note: note  # type: ignore[method-assign]

    errors = result.per_layer_error.values()
    result.mean_relative_error = sum(errors) / len(errors)
    logger.info(result.summary())
    return result


class CalibrationHarness:
    """Seeded token batches for calibration (``calibration.py:224-260``)."""

    def __init__(self, num_samples: int = 128, seq_length: int = 512, seed: int = 0) -> None:
        self.num_samples = num_samples
        self.seq_length = seq_length
        self.seed = seed

    def synthetic(self, vocab_size: int) -> list[torch.Tensor]:
        """``num_samples`` batches ``[1, seq_length]`` of uniform token ids from a generator seeded
        with ``seed``, drawn in batch order."""
        gen = torch.Generator().manual_seed(self.seed)
        ids = torch.randint(0, vocab_size, (self.num_samples, self.seq_length), generator=gen, dtype=torch.long)
        return [row[None].clone() for row in ids]

    def from_tokenizer(self, tokenizer: object, texts: Sequence[str]) -> list[torch.Tensor]:
        """One ``[1, seq_length]`` batch per non-empty text: its ids, cut to ``seq_length`` and
        padded on the right with id 0."""
        encode = getattr(tokenizer, "encode", None)
        if encode is None:
            raise TypeError("tokenizer must expose an encode() method")
        out: list[torch.Tensor] = []
        for text in texts:
            ids = list(encode(text))[: self.seq_length]
            if ids:
                row = torch.zeros(1, self.seq_length, dtype=torch.long)
                row[0, : len(ids)] = torch.tensor(ids, dtype=torch.long)
                out.append(row)
        return out

    def __iter__(self) -> Iterator[torch.Tensor]:  # pragma: no cover - convenience
        raise NotImplementedError("call synthetic() or from_tokenizer() explicitly")

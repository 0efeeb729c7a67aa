"""GPTQ calibration: per-layer input Hessians and model-wide quantization.

Mirrors ``src/llmopt/quantization/calibration.py``: ``HessianCollector``
accumulates ``X^T X`` through forward hooks and reports ``(2/n) X^T X``;
``apply_quantization`` writes dequantized weights back into each ``nn.Linear``
and returns a :class:`CalibrationResult`; ``CalibrationHarness`` builds token
batches. This is offline code: the layout it produces is what the HIP kernels
consume.
"""

from __future__ import annotations

import contextlib
from collections.abc import Iterator, Sequence
from dataclasses import dataclass, field

import torch
from torch import nn

from llmopt.quantization.quantizers import GPTQQuantizer, QuantizedTensor, build_quantizer
from llmopt.utils.logging import get_logger

__all__ = ["CalibrationHarness", "CalibrationResult", "HessianCollector", "apply_quantization"]

logger = get_logger("quant.calibration")


class HessianCollector:
    """Sum of ``x^T x`` over every input row seen by each layer (``calibration.py:28-86``)."""

    def __init__(self, layers: Sequence[nn.Module], device: torch.device | str = "cpu") -> None:
        self.layers = list(layers)
        self.device = torch.device(device)
        self._sums: dict[int, torch.Tensor] = {}
        self._rows: dict[int, int] = {}
        self._handles: list[torch.utils.hooks.RemovableHandle] = []
        self.count = 0

    def _hook(self, module: nn.Module, inputs: tuple[torch.Tensor, ...], _output: object) -> None:
        if not inputs or not isinstance(inputs[0], torch.Tensor):
            return
        rows = inputs[0].detach()
        rows = rows.reshape(-1, rows.shape[-1]).to(device=self.device, dtype=torch.float32)
        key = id(module)
        if key not in self._sums:
            width = module.weight.shape[1]
            self._sums[key] = torch.zeros(width, width, dtype=torch.float32, device=self.device)
            self._rows[key] = 0
        self._sums[key].addmm_(rows.T, rows)
        self._rows[key] += rows.shape[0]
        self.count += 1

    def __enter__(self) -> HessianCollector:
        self._handles = [layer.register_forward_hook(self._hook) for layer in self.layers]
        return self

    def __exit__(self, *exc: object) -> None:
        for handle in self._handles:
            handle.remove()
        self._handles.clear()

    def hessian_for(self, module: nn.Module) -> torch.Tensor | None:
        """``(2/n) X^T X`` for ``module``, or ``None`` if it saw no rows."""
        key = id(module)
        rows = self._rows.get(key, 0)
        if not rows:
            return None
        return (2.0 / rows) * self._sums[key]

    def results(self) -> dict[nn.Module, torch.Tensor]:
        found: dict[nn.Module, torch.Tensor] = {}
        for layer in self.layers:
            hessian = self.hessian_for(layer)
            if hessian is not None:
                found[layer] = hessian
        return found


@dataclass(slots=True)
class CalibrationResult:
    """Packed tensors per layer plus reconstruction error (``calibration.py:89-112``)."""

    quantizers: dict[str, QuantizedTensor] = field(default_factory=dict)
    mean_relative_error: float = 0.0
    per_layer_error: dict[str, float] = field(default_factory=dict)
    baseline_bits: int = 0
    quant_bits: int = 0

    @property
    def compression_ratio(self) -> float:
        if not self.quantizers:
            return 1.0
        dense = sum(q.dense_nbytes() for q in self.quantizers.values())
        packed = sum(q.nbytes() for q in self.quantizers.values())
        return dense / max(1, packed)

    def summary(self) -> str:
        return (
            f"quantized {len(self.quantizers)} layers to {self.quant_bits}-bit, "
            f"mean relative error {self.mean_relative_error:.5f}, "
            f"{self.compression_ratio:.2f}x compression"
        )


def _module_targets(model: nn.Module, ignore: Sequence[str]) -> list[nn.Linear]:
    """Linear layers not matching ``ignore`` and with an even input width."""
    chosen: list[nn.Linear] = []
    for name, module in model.named_modules():
        if not isinstance(module, nn.Linear) or any(token in name for token in ignore):
            continue
        if module.weight.shape[1] % 2:
            logger.debug("skipping %s: in_features=%d is odd", name, module.weight.shape[1])
            continue
        chosen.append(module)
    return chosen


@torch.no_grad()
def _relative_error(original: torch.Tensor, approx: torch.Tensor) -> float:
    scale = torch.linalg.vector_norm(original.float())
    if float(scale) == 0.0:
        return 0.0
    return float(torch.linalg.vector_norm((original - approx).float()) / scale)


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
    """Quantize every eligible ``nn.Linear`` and write the dequantized weight back.

    Follows ``calibration.py:137-221``: unknown strategies fall back to RTN,
    Hessians come from forward hooks over ``calibration_batches`` (failed
    forwards are ignored), and the per-layer relative error is recorded.
    """
    del in_place
    targets = _module_targets(model, ignore_layers)
    result = CalibrationResult(quant_bits=bits)
    if not targets:
        logger.warning("no quantizable linear layers found")
        return result

    hessians: dict[nn.Module, torch.Tensor] = {}
    if strategy == "gptq" and calibration_batches:
        for module in targets:
            with HessianCollector([module], device=module.weight.device) as collector:
                for batch in calibration_batches:
                    tokens = batch.to(module.weight.device)
                    if tokens.dim() == 1:
                        tokens = tokens.unsqueeze(0)
                    with contextlib.suppress(Exception):
                        model(tokens)
                hessians.update(collector.results())
        logger.info("collected Hessians for %d/%d layers", len(hessians), len(targets))

    target_ids = {id(module) for module in targets}
    for name, module in model.named_modules():
        if id(module) not in target_ids:
            continue
        original = module.weight.detach().clone()
        quantizer = build_quantizer(
            strategy,
            bits=bits,
            group_size=group_size,
            symmetric=symmetric,
            damping=damping,
            act_order=act_order,
        )
        if not isinstance(quantizer, GPTQQuantizer):
            quantizer = build_quantizer("rtn", bits=bits, group_size=group_size, symmetric=symmetric)
        quantized = quantizer.quantize(original, hessians.get(module))
        approx = quantized.dequantize().to(original.dtype)
        error = _relative_error(original, approx)
        result.quantizers[name] = quantized
        result.per_layer_error[name] = error
        result.baseline_bits += original.numel() * original.element_size() * 8
        module.weight.data = approx.to(module.weight.device)
        module.extra_repr = (  # type: ignore[method-assign]
            lambda text=f"quantized={quantizer.name}-{bits}bit, group_size={group_size}, "
            f"err={error:.4f}": text
        )

    errors = list(result.per_layer_error.values())
    result.mean_relative_error = sum(errors) / len(errors) if errors else 0.0
    logger.info(result.summary())
    return result


class CalibrationHarness:
    """Seeded synthetic or tokenizer-encoded calibration batches (``calibration.py:224-260``)."""

    def __init__(self, num_samples: int = 128, seq_length: int = 512, seed: int = 0) -> None:
        self.num_samples = num_samples
        self.seq_length = seq_length
        self.seed = seed

    def synthetic(self, vocab_size: int) -> list[torch.Tensor]:
        """``num_samples`` batches ``[1, seq_length]`` of uniform random token ids."""
        generator = torch.Generator().manual_seed(self.seed)
        return [
            torch.randint(0, vocab_size, (1, self.seq_length), generator=generator, dtype=torch.long)
            for _ in range(self.num_samples)
        ]

    def from_tokenizer(self, tokenizer: object, texts: Sequence[str]) -> list[torch.Tensor]:
        """Encode, truncate and zero-pad ``texts`` to ``seq_length`` tokens each."""
        encode = getattr(tokenizer, "encode", None)
        if encode is None:
            raise TypeError("tokenizer must expose an encode() method")
        batches: list[torch.Tensor] = []
        for text in texts:
            ids = list(encode(text))[: self.seq_length]
            if not ids:
                continue
            batches.append(torch.tensor([ids + [0] * (self.seq_length - len(ids))], dtype=torch.long))
        return batches

    def __iter__(self) -> Iterator[torch.Tensor]:  # pragma: no cover - convenience
        raise NotImplementedError("call synthetic() or from_tokenizer() explicitly")

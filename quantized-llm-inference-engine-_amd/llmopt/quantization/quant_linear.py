"""``QuantLinear``: a linear layer whose weight stays packed on the device.

Same class, constructor, attributes and error behaviour as the reference
(``src/llmopt/quantization/quant_linear.py:18-207``). What differs is how
``forward`` gets its answer:

* On a HIP device the packed codes, scales and zeros are read directly by the
  fused dequantize-and-multiply kernels (``llmopt.kernels``): a split-K MFMA
  skinny GEMM for decode-sized batches and an MFMA GEMM that dequantizes weight
  tiles into LDS for prefill-sized batches. No dense copy of the weight is ever
  materialised, and there is no host fallback: a missing kernel library raises.
* On the host the reference sequence is kept: dequantize once into
  ``compute_dtype``, cache, and call ``F.linear``.

``qweight`` is registered as a buffer (the reference keeps it as a plain
attribute, ``quant_linear.py:57,81``), so ``module.to(device)`` moves the codes
together with ``scales`` and ``qzeros`` and ``state_dict`` keeps them.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from llmopt.quantization.quantizers import QuantizedTensor, dequantize
from llmopt.utils.logging import get_logger

__all__ = ["QuantLinear", "QuantLinearConfig", "quantize_model_", "replace_linear_modules"]

logger = get_logger("quant.nn")


class QuantLinearConfig:
    """Bit width, group size, grid symmetry and compute dtype of a :class:`QuantLinear`.

    Defaults follow ``quant_linear.py:18-33``: 4 bits, group 128, symmetric, fp16.
    """

    __slots__ = ("bits", "compute_dtype", "group_size", "symmetric")

    def __init__(
        self,
        bits: int = 4,
        group_size: int = 128,
        symmetric: bool = True,
        compute_dtype: torch.dtype = torch.float16,
    ) -> None:
        self.bits = bits
        self.group_size = group_size
        self.symmetric = symmetric
        self.compute_dtype = compute_dtype


class QuantLinear(nn.Module):
    """Linear layer over a packed :class:`QuantizedTensor` weight.

    ``forward(x)`` equals ``F.linear(x, dequantize(weight, compute_dtype), bias)``;
    ``x`` (and ``bias``) must already be in ``compute_dtype``, as ``F.linear``
    requires of its operands.
    """

    def __init__(
        self,
        in_features: int,
        out_features: int,
        config: QuantLinearConfig | None = None,
        bias: bool = True,
        device: torch.device | str | None = None,
    ) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.config = config or QuantLinearConfig()
        self.register_buffer("qweight", None)
        self.register_buffer("qzeros", torch.zeros(0), persistent=True)
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, device=device))
        else:
            self.register_buffer("bias", None)
        self._cached_weight: torch.Tensor | None = None

    @classmethod
    def from_float(
        cls,
        linear: nn.Linear,
        quantized: QuantizedTensor,
        compute_dtype: torch.dtype | None = None,
    ) -> QuantLinear:
        """Wrap ``quantized`` with the geometry and bias of ``linear`` (``quant_linear.py:66-87``)."""
        config = QuantLinearConfig(
            bits=quantized.bits,
            group_size=quantized.group_size,
            symmetric=quantized.symmetric,
            compute_dtype=compute_dtype or linear.weight.dtype,
        )
        module = cls(linear.in_features, linear.out_features, config, bias=linear.bias is not None)
        module.qweight = quantized.qweight
        module.register_buffer("scales", quantized.scales)
        module.register_buffer("qzeros", quantized.zeros)
        if linear.bias is not None:
            module.bias.data = linear.bias.data.clone()  # type: ignore[union-attr]
        module.invalidate()
        return module

    def invalidate(self) -> None:
        """Forget the host-side dense weight; the next host forward rebuilds it."""
        self._cached_weight = None

    def _apply(self, fn, recurse: bool = True):  # noqa: ANN001, ANN202 - nn.Module signature
        self._cached_weight = None
        return super()._apply(fn, recurse)

    def quantized_tensor(self) -> QuantizedTensor:
        """The packed weight as a :class:`QuantizedTensor` view of this module's buffers."""
        if self.qweight is None or not hasattr(self, "scales"):
            raise RuntimeError("QuantLinear has no quantized weight; call from_float()")
        return QuantizedTensor(
            qweight=self.qweight,
            scales=self.scales,  # type: ignore[arg-type]
            zeros=self.qzeros,
            bits=self.config.bits,
            group_size=self.config.group_size,
            symmetric=self.config.symmetric,
            shape=(self.out_features, self.in_features),
        )

    def _dequantized_weight(self) -> torch.Tensor:
        """Dense ``[out, in]`` weight in ``compute_dtype`` (cached on the host)."""
        if self._cached_weight is None:
            tensor = self.quantized_tensor()
            weight = dequantize(tensor, self.config.compute_dtype)
            if tensor.qweight.device.type == "cuda":
                return weight
            self._cached_weight = weight.to(tensor.qweight.device)
        return self._cached_weight

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.device.type == "cuda":
            from llmopt.kernels import ops

            return ops.quant_linear(x, self.quantized_tensor(), self.bias, self.config.compute_dtype)
        return torch.nn.functional.linear(x, self._dequantized_weight(), self.bias)

    def forward_deferred(self, x: torch.Tensor):  # noqa: ANN201 - Tensor or ops.PartialSums
        """:meth:`forward`, except that on a HIP device a batch whose plan splits K over the
        decode kernel's slices returns its ``PartialSums`` for a following residual add + RMSNorm
        to add up (``ops.rmsnorm``); the result is the same, bit for bit."""
        if x.device.type == "cuda" and not (self._forward_hooks or self._forward_pre_hooks):
            from llmopt.kernels import ops

            return ops.quant_linear(x, self.quantized_tensor(), self.bias, self.config.compute_dtype, defer=True)
        return self(x)

    def extra_repr(self) -> str:
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, "
            f"bits={self.config.bits}, bias={self.bias is not None}"
        )


def replace_linear_modules(
    model: nn.Module,
    replacements: dict[nn.Module, nn.Module],
) -> nn.Module:
    """Put ``replacements[child]`` in place of every child module that is a key (in place).

    Behaviour of ``quant_linear.py:122-136``. The slots are found first and filled after,
    so a replacement that itself contains replaced modules is not visited. Each module
    keeps one slot, the last one the walk over ``model.modules()`` finds: a module
    registered under several parents is replaced only there, as in the reference.
    ``model`` itself is never replaced.
    """
    slot_of: dict[nn.Module, tuple[nn.Module, str]] = {}
    for parent in model.modules():
        for attr, child in parent.named_children():
            if child in replacements:
                slot_of[child] = (parent, attr)
    for child, (parent, attr) in slot_of.items():
        setattr(parent, attr, replacements[child])
    return model


def quantize_model_(
    model: nn.Module,
    *,
    bits: int = 4,
    group_size: int = 128,
    symmetric: bool = True,
    strategy: str = "rtn",
    calibration_batches: list[torch.Tensor] | None = None,
    ignore_layers: tuple[str, ...] = ("lm_head", "embed_tokens"),
    inplace: bool = True,
) -> nn.Module:
    """Swap every eligible ``nn.Linear`` of ``model`` for a :class:`QuantLinear` and return it.

    Behaviour of ``quant_linear.py:139-207``:

    * eligible: an ``nn.Linear`` whose qualified name contains none of ``ignore_layers``;
    * each layer is quantized with groups of ``gcd(in_features, group_size)`` columns, so a
      width that ``group_size`` does not divide still quantizes;
    * ``strategy="gptq"`` with ``calibration_batches`` uses the layers' input Hessians;
      collection ends at the first batch the model cannot run; GPTQ keeps its default
      damping and activation order;
    * each ``QuantLinear`` computes in its original layer's weight dtype, and the old
      layer's weight is overwritten with its dequantization.

    ``inplace`` is accepted for signature compatibility: the model is always modified.
    """
    from llmopt.quantization.calibration import collect_hessians
    from llmopt.quantization.quantizers import build_quantizer

    del inplace
    layers = [
        module
        for name, module in model.named_modules()
        if isinstance(module, nn.Linear) and not any(tok in name for tok in ignore_layers)
    ]
    hessians: dict[nn.Module, torch.Tensor] = {}
    if strategy == "gptq" and calibration_batches:
        hessians = collect_hessians(model, layers, calibration_batches, stop_at_failure=True)

    swaps: dict[nn.Module, nn.Module] = {}
    for layer in layers:
        group = math.gcd(layer.in_features, group_size) or group_size
        if group != group_size:
            logger.debug("in_features=%d: groups of %d columns instead of %d", layer.in_features, group, group_size)
        packed = build_quantizer(strategy, bits=bits, group_size=group, symmetric=symmetric).quantize(
            layer.weight.detach().to(torch.float32), hessians.get(layer)
        )
        swaps[layer] = QuantLinear.from_float(layer, packed, compute_dtype=layer.weight.dtype)
        layer.weight.data = packed.dequantize().to(layer.weight.dtype)
    return replace_linear_modules(model, swaps)

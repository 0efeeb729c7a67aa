"""Fused projections over packed weights: one kernel launch for several ``QuantLinear``s.

The reference runs ``q_proj``, ``k_proj`` and ``v_proj``, and ``gate_proj`` and ``up_proj``,
as separate linears and applies ``silu(gate(x)) * up(x)`` as two more elementwise passes over
``[M, intermediate]`` (``src/llmopt/model/layers.py:39-44,64-67,106-108``). Packed rows are
independent, so stacking the weights of several projections along ``out_features`` is exact:

* :class:`FusedQuantLinear` concatenates the rows of several ``QuantLinear``s that share
  ``in_features`` and quantization settings; ``forward`` returns one output per part.
* :class:`QuantSwiGLU` interleaves gate and up rows in blocks of four (fused row ``8p + r``
  is gate row ``4p + r``, fused row ``8p + 4 + r`` is up row ``4p + r``) and returns
  ``silu(gate(x)) * up(x)``. On HIP devices the kernels apply the activation in their
  epilogue, so the ``[M, 2 * intermediate]`` product is never written.

On the host both keep the reference sequence: dequantize, ``F.linear``, then split (or
``silu(gate) * up`` in ``compute_dtype``).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
from torch import nn

from llmopt.quantization.quant_linear import QuantLinear, QuantLinearConfig
from llmopt.quantization.quantizers import QuantizedTensor, dequantize

__all__ = ["FusedQuantLinear", "QuantSwiGLU", "concat_rows", "interleave_gate_up"]


def _check_compatible(tensors: Sequence[QuantizedTensor]) -> None:
    if not tensors:
        raise ValueError("nothing to fuse")
    first = tensors[0]
    for t in tensors[1:]:
        if t.shape[1] != first.shape[1]:
            raise ValueError(f"in_features differ: {t.shape[1]} != {first.shape[1]}")
        if (t.bits, t.group_size, t.symmetric) != (first.bits, first.group_size, first.symmetric):
            raise ValueError(
                "fused projections need the same bits, group_size and symmetry, got "
                f"{(t.bits, t.group_size, t.symmetric)} and {(first.bits, first.group_size, first.symmetric)}"
            )
        if t.qweight.dtype != first.qweight.dtype or t.qweight.device != first.qweight.device:
            raise ValueError("fused projections need codes of one dtype on one device")


def _zeros_of(t: QuantizedTensor) -> torch.Tensor:
    """The [N, G] zero-point table (symmetric tensors may carry an empty placeholder)."""
    if t.zeros.shape == t.scales.shape:
        return t.zeros
    return torch.zeros_like(t.scales)


def concat_rows(parts: Sequence[QuantizedTensor]) -> QuantizedTensor:
    """Stack packed weights along ``out_features`` (rows are independent: exact)."""
    _check_compatible(parts)
    first = parts[0]
    return QuantizedTensor(
        qweight=torch.cat([p.qweight for p in parts], dim=0).contiguous(),
        scales=torch.cat([p.scales for p in parts], dim=0).contiguous(),
        zeros=torch.cat([_zeros_of(p) for p in parts], dim=0).contiguous(),
        bits=first.bits,
        group_size=first.group_size,
        symmetric=first.symmetric,
        shape=(sum(int(p.shape[0]) for p in parts), int(first.shape[1])),
    )


def _interleave4(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    rows = gate.shape[0]
    g = gate.reshape(rows // 4, 4, *gate.shape[1:])
    u = up.reshape(rows // 4, 4, *up.shape[1:])
    return torch.stack([g, u], dim=1).reshape(2 * rows, *gate.shape[1:]).contiguous()


def interleave_gate_up(gate: QuantizedTensor, up: QuantizedTensor) -> QuantizedTensor:
    """One packed weight with gate and up rows interleaved in blocks of four."""
    _check_compatible([gate, up])
    rows = int(gate.shape[0])
    if int(up.shape[0]) != rows:
        raise ValueError(f"gate and up have different out_features: {rows} != {up.shape[0]}")
    if rows % 4:
        raise ValueError(f"out_features must be a multiple of 4 to interleave, got {rows}")
    return QuantizedTensor(
        qweight=_interleave4(gate.qweight, up.qweight),
        scales=_interleave4(gate.scales, up.scales),
        zeros=_interleave4(_zeros_of(gate), _zeros_of(up)),
        bits=gate.bits,
        group_size=gate.group_size,
        symmetric=gate.symmetric,
        shape=(2 * rows, int(gate.shape[1])),
    )


def _same_config(modules: Sequence[QuantLinear]) -> QuantLinearConfig:
    cfg = modules[0].config
    for m in modules[1:]:
        if m.in_features != modules[0].in_features:
            raise ValueError(f"in_features differ: {m.in_features} != {modules[0].in_features}")
        if m.config.compute_dtype != cfg.compute_dtype:
            raise ValueError(f"compute_dtype differs: {m.config.compute_dtype} != {cfg.compute_dtype}")
    return QuantLinearConfig(cfg.bits, cfg.group_size, cfg.symmetric, cfg.compute_dtype)


def _bias_or_zeros(module: QuantLinear, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    if module.bias is not None:
        return module.bias.detach().to(dtype)
    return torch.zeros(module.out_features, dtype=dtype, device=device)


class _FusedBase(nn.Module):
    def __init__(self, tensor: QuantizedTensor, config: QuantLinearConfig, bias: torch.Tensor | None) -> None:
        super().__init__()
        self.config = config
        self.in_features = int(tensor.shape[1])
        self.fused_out_features = int(tensor.shape[0])
        self.register_buffer("qweight", tensor.qweight)
        self.register_buffer("scales", tensor.scales)
        self.register_buffer("qzeros", tensor.zeros)
        self.register_buffer("bias", bias)
        self._cached_weight: torch.Tensor | None = None

    def quantized_tensor(self) -> QuantizedTensor:
        return QuantizedTensor(
            qweight=self.qweight,
            scales=self.scales,
            zeros=self.qzeros,
            bits=self.config.bits,
            group_size=self.config.group_size,
            symmetric=self.config.symmetric,
            shape=(self.fused_out_features, self.in_features),
        )

    def invalidate(self) -> None:
        """Forget the host-side dense weight; the next host forward rebuilds it."""
        self._cached_weight = None

    def _apply(self, fn, recurse: bool = True):  # noqa: ANN001, ANN202 - nn.Module signature
        self._cached_weight = None
        return super()._apply(fn, recurse)

    def _host_product(self, x: torch.Tensor) -> torch.Tensor:
        if self._cached_weight is None:
            self._cached_weight = dequantize(self.quantized_tensor(), self.config.compute_dtype)
        return torch.nn.functional.linear(x, self._cached_weight, self.bias)


class FusedQuantLinear(_FusedBase):
    """Several ``QuantLinear``s over one input as one packed weight (e.g. q, k and v).

    ``forward(x)`` returns ``tuple(part(x) for part in parts)``; on HIP devices with one kernel
    launch. The outputs are column slices of one ``[..., sum(out_features)]`` tensor.
    """

    def __init__(self, parts: Sequence[QuantLinear]) -> None:
        if not parts:
            raise ValueError("nothing to fuse")
        config = _same_config(parts)
        tensor = concat_rows([p.quantized_tensor() for p in parts])
        ref = parts[0].scales
        bias = None
        if any(p.bias is not None for p in parts):
            bias = torch.cat([_bias_or_zeros(p, config.compute_dtype, ref.device) for p in parts])
        super().__init__(tensor, config, bias)
        self.out_features = [p.out_features for p in parts]

    def forward(self, x: torch.Tensor) -> tuple[torch.Tensor, ...]:
        if x.device.type == "cuda":
            from llmopt.kernels import ops

            y = ops.quant_linear(x, self.quantized_tensor(), self.bias, self.config.compute_dtype)
        else:
            y = self._host_product(x)
        return tuple(torch.split(y, self.out_features, dim=-1))

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bits={self.config.bits}"


class QuantSwiGLU(_FusedBase):
    """``silu(gate(x)) * up(x)`` for two ``QuantLinear``s, gate and up rows interleaved.

    On HIP devices one kernel computes both projections and applies the activation in its
    epilogue (``llmopt_q_linear_swiglu``); the result is ``[..., intermediate]``.
    """

    def __init__(self, gate: QuantLinear, up: QuantLinear) -> None:
        config = _same_config([gate, up])
        tensor = interleave_gate_up(gate.quantized_tensor(), up.quantized_tensor())
        bias = None
        if gate.bias is not None or up.bias is not None:
            dev = gate.scales.device
            bias = _interleave4(_bias_or_zeros(gate, config.compute_dtype, dev),
                                _bias_or_zeros(up, config.compute_dtype, dev))
        super().__init__(tensor, config, bias)
        self.out_features = gate.out_features

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.device.type == "cuda":
            from llmopt.kernels import ops

            return ops.quant_linear_swiglu(x, self.quantized_tensor(), self.bias, self.config.compute_dtype)
        y = self._host_product(x)
        blocks = y.reshape(*y.shape[:-1], self.out_features // 4, 2, 4)
        gate = blocks[..., 0, :].reshape(*y.shape[:-1], self.out_features)
        up = blocks[..., 1, :].reshape(*y.shape[:-1], self.out_features)
        return torch.nn.functional.silu(gate) * up

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bits={self.config.bits}"

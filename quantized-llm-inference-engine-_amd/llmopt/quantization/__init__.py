"""Weight quantization: RTN, GPTQ, packed storage and ``QuantLinear``.

Exports the same names as the reference's ``src/llmopt/quantization/__init__.py:30-49``, plus
the fused projections of :mod:`llmopt.quantization.fused` and the packed checkpoint of
:mod:`llmopt.quantization.checkpoint` (which have no counterpart there).
"""

from __future__ import annotations

from llmopt.quantization.calibration import (
    CalibrationHarness,
    CalibrationResult,
    HessianCollector,
    apply_quantization,
)
from llmopt.quantization.checkpoint import is_quantized_checkpoint, load_quantized_, save_quantized
from llmopt.quantization.fused import FusedQuantLinear, QuantSwiGLU, concat_rows, interleave_gate_up
from llmopt.quantization.quant_linear import (
    QuantLinear,
    QuantLinearConfig,
    quantize_model_,
    replace_linear_modules,
)
from llmopt.quantization.quantizers import (
    GPTQQuantizer,
    QuantizedTensor,
    Quantizer,
    RoundToNearestQuantizer,
    build_quantizer,
    choose_qparams,
    dequantize,
    pack_int4,
    quantize_to_codes,
    unpack_int4,
)

__all__ = [
    "CalibrationHarness",
    "CalibrationResult",
    "FusedQuantLinear",
    "GPTQQuantizer",
    "HessianCollector",
    "QuantLinear",
    "QuantLinearConfig",
    "QuantSwiGLU",
    "QuantizedTensor",
    "Quantizer",
    "RoundToNearestQuantizer",
    "apply_quantization",
    "build_quantizer",
    "choose_qparams",
    "concat_rows",
    "dequantize",
    "interleave_gate_up",
    "is_quantized_checkpoint",
    "load_quantized_",
    "pack_int4",
    "quantize_model_",
    "quantize_to_codes",
    "replace_linear_modules",
    "save_quantized",
    "unpack_int4",
]

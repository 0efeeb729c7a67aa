"""llmopt on MI355X: the quantized-linear hot path with gfx950 HIP kernels.

The public surface is ``llmopt.quantization`` (same names, constructors and
errors as the reference's ``src/llmopt/quantization/__init__.py:30-49``).
On HIP devices ``QuantLinear.forward`` runs the fused dequantize-and-multiply
kernels in ``libllmopt_qlinear.so`` through a C ABI (``llmopt.kernels``).
"""

__version__ = "0.1.0"

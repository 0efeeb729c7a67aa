"""Write tests/golden/gptq_small.npz from the reference's own GPTQQuantizer.

GPTQ with a non-diagonal Hessian is the one function on this path that no closed form
pins: its codes depend on LAPACK's Cholesky rounding and on the order of the error
feedback (src/llmopt/quantization/quantizers.py:308-457). This script imports the
reference (read-only, from /root/reference/src) in its own process, runs it on small
seeded inputs and stores inputs and outputs as plain arrays. It is run by hand in the
build container; the fixture, not the reference, is what the tests read.

    python tests/golden/make_gptq_fixture.py
"""

from __future__ import annotations

import sys
from pathlib import Path

REFERENCE_SRC = "/root/reference/src"
OUT = Path(__file__).resolve().parent / "gptq_small.npz"

# (name, bits, symmetric, act_order)
CASES = [
    ("b4_sym", 4, True, True),
    ("b4_asym", 4, False, True),
    ("b8_sym", 8, True, True),
    ("b2_asym_noorder", 2, False, False),
]
ROWS, COLS, GROUP, SAMPLES = 64, 256, 128, 64


def main() -> int:
    sys.path.insert(0, REFERENCE_SRC)
    import numpy as np
    import torch

    from llmopt.quantization.quantizers import GPTQQuantizer  # the reference's class

    assert "/root/reference" in sys.modules["llmopt"].__file__, "wrong llmopt imported"
    gen = torch.Generator().manual_seed(1234)
    weight = torch.randn(ROWS, COLS, generator=gen) * 0.02
    # Correlated calibration rows so the Hessian is far from diagonal.
    mix = torch.randn(COLS, COLS, generator=gen) / COLS**0.5
    x = torch.randn(SAMPLES, COLS, generator=gen) @ mix + 0.1 * torch.randn(SAMPLES, COLS, generator=gen)
    hessian = (2.0 / SAMPLES) * (x.T @ x)

    arrays = {"weight": weight.numpy(), "hessian": hessian.numpy()}
    for name, bits, symmetric, act_order in CASES:
        quantizer = GPTQQuantizer(bits=bits, group_size=GROUP, symmetric=symmetric, act_order=act_order)
        qt = quantizer.quantize(weight.clone(), hessian.clone())
        arrays[f"{name}_qweight"] = qt.qweight.numpy()
        arrays[f"{name}_scales"] = qt.scales.numpy()
        arrays[f"{name}_zeros"] = qt.zeros.numpy()
    arrays["cases"] = np.array([f"{n}:{b}:{int(s)}:{int(a)}" for n, b, s, a in CASES])
    arrays["group"] = np.array(GROUP)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes) with torch {torch.__version__}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

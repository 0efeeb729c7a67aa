"""Pins the torch restatement used for the CPU baseline against the numpy oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from llmopt.quantization import RoundToNearestQuantizer
from oracle import quant_oracle as qo
from oracle.cpu_reference import ReferenceLinear, dense_weight


@pytest.mark.parametrize("bits,symmetric", [(4, False), (4, True), (2, False), (8, True), (8, False)])
def test_dense_weight_matches_oracle(bits, symmetric):
    w = torch.randn(40, 256, generator=torch.Generator().manual_seed(bits)) * 0.02
    qt = RoundToNearestQuantizer(bits, 64, symmetric).quantize(w)
    args = (qt.qweight, qt.scales, qt.zeros, bits, 64, symmetric, qt.shape)
    oracle = qo.dequantize(*(t.numpy() for t in args[:3]), bits, 64, symmetric, qt.shape)
    np.testing.assert_array_equal(dense_weight(*args, torch.float32).numpy(), oracle)
    bf16 = dense_weight(*args, torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16, qo.bf16_bits(oracle))


def test_reference_linear_caches_and_matches():
    w = torch.randn(16, 128) * 0.02
    qt = RoundToNearestQuantizer(4, 128, False).quantize(w)
    ref = ReferenceLinear(qt.qweight, qt.scales, qt.zeros, 4, 128, False, qt.shape, torch.float32)
    x = torch.randn(3, 128)
    y = ref(x)
    assert ref.cached is not None
    dense = torch.from_numpy(qo.dequantize(qt.qweight.numpy(), qt.scales.numpy(), qt.zeros.numpy(), 4, 128, False, qt.shape))
    torch.testing.assert_close(y, qo.reference_linear(x, dense), rtol=0, atol=0)
    ref.invalidate()
    assert ref.cached is None

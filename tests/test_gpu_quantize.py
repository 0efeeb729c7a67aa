"""On-device round-to-nearest quantizer against the oracle: codes, scales and zero points
bit-exact, for every width, both grids, fp32/fp16/bf16 weights, both kernels (teams of lanes
per group, and one thread per group) and the special groups the reference's arithmetic has."""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from llmopt.kernels import ops
from llmopt.quantization import QuantizedTensor, RoundToNearestQuantizer, quantize_model_
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _oracle(weight: torch.Tensor, bits: int, group: int, symmetric: bool):
    w32 = weight.to(torch.float32).numpy()
    return qo.rtn_quantize(w32, bits, group, symmetric)


def _check(got: QuantizedTensor, weight: torch.Tensor, bits: int, group: int, symmetric: bool) -> None:
    q, s, z = _oracle(weight, bits, group, symmetric)
    got_q = got.qweight.cpu()
    assert got_q.dtype == (torch.int8 if bits == 8 and symmetric else torch.uint8)
    np.testing.assert_array_equal(got_q.numpy(), q)
    # Bit patterns: a zero point of -0.0 (all-positive group) must match too.
    np.testing.assert_array_equal(got.scales.cpu().numpy().view(np.uint32), s.view(np.uint32))
    np.testing.assert_array_equal(got.zeros.cpu().numpy().view(np.uint32), z.view(np.uint32))


SHAPES = [  # (rows, cols, group): teams of 16 / 64 lanes, several chunks per lane, generic kernel
    (48, 256, 128),
    (33, 512, 64),
    (8, 2048, 1024),
    (16, 96, 12),
    (8, 100, 10),
    (5, 1536, 768),
    (64, 48, 16),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits,symmetric", [(4, False), (4, True), (2, False), (2, True), (8, False), (8, True)])
@pytest.mark.parametrize("rows,cols,group", SHAPES)
def test_rtn_bit_exact(dtype, bits, symmetric, rows, cols, group):
    gen = torch.Generator().manual_seed(rows * cols + bits)
    weight = (torch.randn(rows, cols, generator=gen) * 0.02).to(dtype)
    got = RoundToNearestQuantizer(bits, group, symmetric).quantize(weight.to(DEV))
    assert got.shape == (rows, cols) and got.group_size == group
    _check(got, weight, bits, group, symmetric)


@pytest.mark.parametrize("bits,symmetric", [(4, False), (4, True), (8, False), (8, True)])
def test_rtn_special_groups(bits, symmetric):
    # Groups of 32: all zero (s = 1e-8), all positive (z = -0.0), all negative (z = 2^b - 1),
    # constant, a single outlier, ties of w / s at .5, and tiny magnitudes below 1e-8.
    g = 32
    rows = [
        np.zeros(g),
        np.linspace(0.01, 0.3, g),
        -np.linspace(0.01, 0.3, g),
        np.full(g, 0.125),
        np.r_[np.zeros(g - 1), 5.0],
        np.arange(g) * 0.5 - 7.5,
        np.linspace(-1e-9, 3e-9, g),
        np.linspace(-4.0, 1.0, g),
    ]
    weight = torch.tensor(np.stack(rows), dtype=torch.float32)
    got = RoundToNearestQuantizer(bits, g, symmetric).quantize(weight.to(DEV))
    _check(got, weight, bits, g, symmetric)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bits,symmetric", [(2, False), (2, True), (4, False), (4, True), (8, False), (8, True)])
def test_rtn_scales_near_the_fp32_limit(dtype, bits, symmetric):
    # The kernel's division-free quotient holds for scales up to 2^120; larger scales, and
    # those that overflow to infinity (max - min past the fp32 range), divide instead. Rows
    # on both sides of that bound, next to an ordinary row, stay bit-exact with the oracle.
    g = 32
    rows = [
        np.linspace(-1e37, 3e37, g),  # s above 2^120 at 2 and 4 bits, below at 8
        np.linspace(-3e38, 3e38, g),  # max - min overflows: s = inf
        np.linspace(1e36, 2e38, g),  # all positive, large
        np.r_[np.zeros(g - 1), 3.3e38],  # one outlier near the top of the range
        np.linspace(-2e38, -1e35, g),  # all negative
        np.arange(g) * 0.5 - 7.5,  # ordinary magnitudes in the same launch
    ]
    weight = torch.tensor(np.stack(rows), dtype=torch.float32).to(dtype)
    got = RoundToNearestQuantizer(bits, g, symmetric).quantize(weight.to(DEV))
    with np.errstate(over="ignore"):  # the oracle's max - min overflows on purpose
        _check(got, weight, bits, g, symmetric)


def test_rtn_full_size_gate_up_bf16():
    gen = torch.Generator(device=DEV).manual_seed(0)
    weight = (torch.randn(28672, 4096, generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
    got = RoundToNearestQuantizer(4, 128, symmetric=False).quantize(weight)
    _check(got, weight.cpu(), 4, 128, False)


def test_rtn_matches_the_host_path_and_round_trips():
    gen = torch.Generator().manual_seed(7)
    weight = torch.randn(96, 384, generator=gen) * 0.05
    host = RoundToNearestQuantizer(4, 64, symmetric=False).quantize(weight)
    dev = RoundToNearestQuantizer(4, 64, symmetric=False).quantize(weight.to(DEV))
    assert torch.equal(host.qweight, dev.qweight.cpu())
    assert torch.equal(host.scales, dev.scales.cpu()) and torch.equal(host.zeros, dev.zeros.cpu())
    # Reconstruction error of an in-range weight is at most half a step.
    dense = dev.dequantize().cpu()
    step = dev.scales.cpu().repeat_interleave(64, dim=1)
    assert bool(((dense - weight).abs() <= step / 2 * (1 + 1e-6)).all())


def test_rtn_strided_and_float64_inputs():
    gen = torch.Generator().manual_seed(3)
    base = torch.randn(40, 512, generator=gen, dtype=torch.float64) * 0.02
    got = ops.quantize_rtn(base.to(DEV)[:, 128:384], 4, 128, False)
    q, s, z = _oracle(base[:, 128:384].to(torch.float32), 4, 128, False)
    np.testing.assert_array_equal(got[0].cpu().numpy(), q)
    np.testing.assert_array_equal(got[1].cpu().numpy(), s)
    np.testing.assert_array_equal(got[2].cpu().numpy(), z)


def test_rtn_errors_match_the_reference():
    w = torch.randn(4, 96, device=DEV)
    with pytest.raises(ValueError, match="not divisible"):
        ops.quantize_rtn(w, 4, 64, False)
    with pytest.raises(ValueError, match="bit width"):
        ops.quantize_rtn(w, 3, 32, False)
    with pytest.raises(ValueError, match="2D"):
        ops.quantize_rtn(w[0], 4, 32, False)


def test_quantize_model_on_device_matches_host():
    from torch import nn

    gen = torch.Generator().manual_seed(11)
    model = nn.Sequential(nn.Linear(256, 192), nn.SiLU(), nn.Linear(192, 64))
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    dev_model = quantize_model_(copy.deepcopy(model).to(DEV), bits=4, group_size=64)
    host_model = quantize_model_(copy.deepcopy(model), bits=4, group_size=64)
    for name in ("0", "2"):
        a, b = host_model.get_submodule(name), dev_model.get_submodule(name)
        assert torch.equal(a.qweight, b.qweight.cpu())
        assert torch.equal(a.scales, b.scales.cpu())


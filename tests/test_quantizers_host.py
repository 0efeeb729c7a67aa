"""Host (CPU) behaviour of llmopt.quantization against the oracle and the reference's contract.

The package's torch implementations must be bit-identical to the oracle for every
producer and consumer of the packed layout, raise the reference's exceptions, and
reproduce the reference GPTQ codes stored in tests/golden/gptq_small.npz.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from llmopt.quantization import (
    GPTQQuantizer,
    QuantizedTensor,
    RoundToNearestQuantizer,
    build_quantizer,
    choose_qparams,
    dequantize,
    pack_int4,
    quantize_to_codes,
    unpack_int4,
)
from llmopt.quantization.quantizers import dequantize_codes, expand_group_metadata
from oracle import quant_oracle as qo

GOLDEN = Path(__file__).resolve().parent / "golden" / "gptq_small.npz"


def _weight(rows, cols, seed, scale=0.02):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(rows, cols, generator=gen) * scale


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize("group", [16, 64, 128, 0])
def test_rtn_matches_oracle_bit_for_bit(bits, symmetric, group):
    w = _weight(48, 256, seed=bits * 100 + group + symmetric)
    w[3, :] = 0.0
    w[5, :16] = 0.5
    w[7, :16] = -0.5
    qt = RoundToNearestQuantizer(bits, group if group > 0 else 256, symmetric).quantize(w)
    ref_q, ref_s, ref_z = qo.rtn_quantize(w.numpy(), bits, group if group > 0 else 256, symmetric)
    np.testing.assert_array_equal(qt.qweight.numpy(), ref_q)
    np.testing.assert_array_equal(qt.scales.numpy(), ref_s)
    np.testing.assert_array_equal(qt.zeros.numpy(), ref_z)
    dense = qt.dequantize()
    assert dense.dtype == torch.float32
    np.testing.assert_array_equal(
        dense.numpy(), qo.dequantize(ref_q, ref_s, ref_z, bits, qt.group_size, symmetric, (48, 256))
    )
    for dtype, name in [(torch.bfloat16, "bfloat16"), (torch.float16, "float16")]:
        cast = dequantize(qt, dtype).to(torch.float32).numpy()
        np.testing.assert_array_equal(cast, qo.round_to_dtype(dense.numpy(), name))


def test_choose_qparams_group_nonpositive_and_errors():
    w = _weight(4, 32, 1)
    s, z = choose_qparams(w, 4, 0, False)
    assert s.shape == (4, 1)
    with pytest.raises(ValueError):
        choose_qparams(w, 4, 5, False)
    with pytest.raises(ValueError):
        choose_qparams(w[0], 4, 4, False)
    s16, _ = choose_qparams(w.to(torch.bfloat16), 4, 8, True)
    assert s16.dtype == torch.float32


def test_pack_unpack_contract():
    codes = torch.arange(16, dtype=torch.uint8).repeat(3, 2)
    packed = pack_int4(codes)
    assert packed.shape == (3, 16) and packed.dtype == torch.uint8
    np.testing.assert_array_equal(packed.numpy(), qo.pack_nibbles(codes.numpy()))
    np.testing.assert_array_equal(unpack_int4(packed, 32).numpy(), codes.numpy())
    np.testing.assert_array_equal(unpack_int4(packed, 7).numpy(), codes[:, :7].numpy())
    every = torch.arange(256, dtype=torch.int64).to(torch.uint8).reshape(1, 256)
    np.testing.assert_array_equal(unpack_int4(every, 512).numpy(), qo.unpack_nibbles(every.numpy(), 512))
    with pytest.raises(ValueError, match="even number of columns"):
        pack_int4(torch.zeros(2, 3, dtype=torch.uint8))


def test_quantize_and_dequantize_codes_match_oracle():
    w = _weight(8, 64, 9, scale=0.3)
    for bits, sym in [(4, True), (8, True), (8, False), (2, True)]:
        s, z = choose_qparams(w, bits, 16, sym)
        q = quantize_to_codes(w, s, z, bits, 16, sym)
        ref = qo.quantize_codes(w.numpy(), s.numpy(), z.numpy(), bits, 16, sym)
        assert q.numpy().dtype == ref.dtype
        np.testing.assert_array_equal(q.numpy(), ref)
        deq = dequantize_codes(q.to(torch.float32), s, z, bits, 16, torch.float32, sym)
        np.testing.assert_array_equal(deq.numpy(), qo.dequantize_codes(ref, s.numpy(), z.numpy(), bits, 16, sym))


def test_quantizer_validation_and_factory():
    with pytest.raises(ValueError, match="unsupported bit width"):
        RoundToNearestQuantizer(3)
    with pytest.raises(ValueError, match="positive even"):
        RoundToNearestQuantizer(4, group_size=7)
    with pytest.raises(ValueError, match="positive even"):
        GPTQQuantizer(4, group_size=0)
    with pytest.raises(ValueError, match="unknown quantization strategy"):
        build_quantizer("none", bits=4)
    q = build_quantizer("gptq", bits=8, group_size=64, symmetric=False, damping=0.1, bogus=1)
    assert isinstance(q, GPTQQuantizer) and q.damping == 0.1 and q.block_size == 64
    r = build_quantizer("rtn", bits=2, group_size=32, damping=0.5)
    assert isinstance(r, RoundToNearestQuantizer) and r.bits == 2
    with pytest.raises(ValueError, match="2D"):
        RoundToNearestQuantizer(4, 16).quantize(torch.zeros(16))
    with pytest.raises(ValueError, match="2D"):
        GPTQQuantizer(4, 16).quantize(torch.zeros(16), torch.eye(16))


def test_quantized_tensor_helpers():
    qt = RoundToNearestQuantizer(4, 64, True).quantize(_weight(32, 128, 2))
    assert qt.code_offset == 8 and qt.pack_factor == 8
    assert qt.nbytes() == 32 * 64 + 2 * 32 * 2 * 4
    assert qt.dense_nbytes() == 32 * 128 * 2
    assert qt.compression_ratio() == pytest.approx(qt.dense_nbytes() / qt.nbytes())
    asym = RoundToNearestQuantizer(8, 64, False).quantize(_weight(4, 128, 3))
    assert asym.code_offset == 0 and asym.pack_factor == 1
    with pytest.raises(Exception):
        qt.bits = 2  # frozen dataclass


def test_gptq_without_hessian_is_rtn_and_diagonal_hessian_gives_rtn_codes():
    w = _weight(32, 256, 4)
    rtn = RoundToNearestQuantizer(4, 128, False).quantize(w)
    none = GPTQQuantizer(4, 128, False).quantize(w, None)
    np.testing.assert_array_equal(none.qweight.numpy(), rtn.qweight.numpy())
    # A diagonal Hessian has a diagonal inverse Cholesky factor: no error is propagated,
    # whatever the column order, so the codes equal round-to-nearest.
    diag = torch.diag(torch.linspace(0.5, 4.0, 256))
    gptq = GPTQQuantizer(4, 128, False).quantize(w, diag)
    np.testing.assert_array_equal(gptq.qweight.numpy(), rtn.qweight.numpy())
    np.testing.assert_array_equal(gptq.scales.numpy(), rtn.scales.numpy())


def test_gptq_matches_reference_golden_vectors():
    data = np.load(GOLDEN, allow_pickle=False)
    weight = torch.from_numpy(data["weight"])
    hessian = torch.from_numpy(data["hessian"])
    group = int(data["group"])
    for case in data["cases"]:
        name, bits, sym, order = str(case).split(":")
        quantizer = GPTQQuantizer(
            bits=int(bits), group_size=group, symmetric=bool(int(sym)), act_order=bool(int(order))
        )
        qt = quantizer.quantize(weight.clone(), hessian.clone())
        np.testing.assert_array_equal(qt.qweight.numpy(), data[f"{name}_qweight"], err_msg=name)
        np.testing.assert_array_equal(qt.scales.numpy(), data[f"{name}_scales"], err_msg=name)
        np.testing.assert_array_equal(qt.zeros.numpy(), data[f"{name}_zeros"], err_msg=name)


def test_gptq_reduces_output_error_on_its_calibration_data():
    data = np.load(GOLDEN, allow_pickle=False)
    weight = torch.from_numpy(data["weight"])
    hessian = torch.from_numpy(data["hessian"])
    rtn = RoundToNearestQuantizer(4, 128, False).quantize(weight).dequantize()
    gptq = GPTQQuantizer(4, 128, False).quantize(weight, hessian).dequantize()

    def proxy(dense):
        delta = dense - weight
        return float(torch.einsum("nk,kl,nl->", delta, hessian, delta))

    assert proxy(gptq) < proxy(rtn)


def test_expand_group_metadata():
    s = torch.tensor([[1.0, 2.0]])
    z = torch.tensor([[3.0, 4.0]])
    ps, pz = expand_group_metadata(s, z, 2, 4)
    assert ps.tolist() == [[1.0, 1.0, 2.0, 2.0]] and pz.tolist() == [[3.0, 3.0, 4.0, 4.0]]


def test_quantized_tensor_dequantize_dtype_flow():
    qt = RoundToNearestQuantizer(4, 32, False).quantize(_weight(4, 64, 6))
    assert isinstance(qt, QuantizedTensor)
    assert dequantize(qt, torch.float64).dtype == torch.float64
    np.testing.assert_array_equal(
        dequantize(qt, torch.float64).numpy(), dequantize(qt).numpy().astype(np.float64)
    )

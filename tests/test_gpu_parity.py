"""Parity of the gfx950 kernels with the CPU oracle, through the C ABI.

* unpack and dequantize: bit-exact with the oracle for every bit width, grid, group
  size and output dtype (fp32 exactly; bf16/fp16 as the round-to-nearest-even cast of
  the oracle's fp32 value).
* quantized linear (every kernel: generic, decode, prefill, and the automatic choice):
  max|y - y_ref| / max|y_ref| <= 1e-2 for bf16/fp16 and <= 2e-3 for fp32, where y_ref is
  the reference's own sequence (oracle dequantization, cast to the compute dtype,
  ``F.linear`` on the CPU). At full Llama-3-8B projection sizes the check uses sampled
  output columns, a torch fp32 GPU matmul of the bit-exact dequantized weight, and two
  size-independent properties: one-hot activation rows must return the dequantized
  weight column bit for bit, and scaling x by 2 must scale y by 2 exactly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from llmopt.kernels import _lib, ops
from llmopt.kernels._lib import ALGO_AUTO, ALGO_DECODE, ALGO_GENERIC, ALGO_PREFILL
from llmopt.quantization import QuantizedTensor, RoundToNearestQuantizer, dequantize, unpack_int4
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu

DEV = "cuda"
NP_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}
TOL = {torch.float32: 2e-3, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _host_qt(rows, cols, bits, group, symmetric, seed, scale=0.02):
    gen = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, cols, generator=gen) * scale
    return RoundToNearestQuantizer(bits, group, symmetric).quantize(w)


def _to_device(qt: QuantizedTensor) -> QuantizedTensor:
    return QuantizedTensor(
        qweight=qt.qweight.to(DEV),
        scales=qt.scales.to(DEV),
        zeros=qt.zeros.to(DEV),
        bits=qt.bits,
        group_size=qt.group_size,
        symmetric=qt.symmetric,
        shape=qt.shape,
    )


def _oracle_dense(qt: QuantizedTensor) -> np.ndarray:
    return qo.dequantize(
        qt.qweight.cpu().numpy(), qt.scales.cpu().numpy(), qt.zeros.cpu().numpy(),
        qt.bits, qt.group_size, qt.symmetric, qt.shape,
    )


def _bits_of(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy()
    return t.view(torch.int16).numpy()


def _expected_bits(dense32: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    if dtype == torch.float32:
        return dense32.view(np.int32)
    if dtype == torch.bfloat16:
        return qo.bf16_bits(dense32).view(np.int16)
    with np.errstate(over="ignore"):  # extreme scales overflow to inf, as torch's cast does
        return dense32.astype(np.float16).view(np.int16)


def _rel_err(y: torch.Tensor, ref: torch.Tensor) -> float:
    y = y.detach().float().cpu()
    ref = ref.detach().float().cpu()
    denom = float(ref.abs().max())
    return float((y - ref).abs().max()) / (denom if denom > 0 else 1.0)


def _reference_linear(x_cpu, dense32, bias_cpu, dtype, cols=None):
    """The reference's sequence: dense weight cast to compute dtype, then F.linear on the CPU."""
    w = torch.from_numpy(qo.round_to_dtype(dense32 if cols is None else dense32[cols], NP_NAMES[dtype]))
    b = None if bias_cpu is None else (bias_cpu if cols is None else bias_cpu[cols])
    return qo.reference_linear(x_cpu, w.to(dtype), b)


# ---- unpack ------------------------------------------------------------------------------------

@pytest.mark.parametrize(
    "shape,columns",
    [((4, 8), 16), ((3, 88), 176), ((5, 7), 13), ((2, 3, 16), 32), ((4096, 2048), 4096), ((1, 256), 512), ((6, 10), 4)],
)
def test_unpack_bit_exact(shape, columns):
    gen = torch.Generator().manual_seed(sum(shape) + columns)
    packed = torch.randint(0, 256, shape, generator=gen, dtype=torch.int32).to(torch.uint8)
    got = unpack_int4(packed.to(DEV), columns)
    np.testing.assert_array_equal(got.cpu().numpy(), qo.unpack_nibbles(packed.numpy(), columns))


def test_unpack_every_byte_value_and_views():
    packed = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(1, 256)
    np.testing.assert_array_equal(unpack_int4(packed.to(DEV), 512).cpu().numpy(), qo.unpack_nibbles(packed.numpy(), 512))
    # A transposed (non-contiguous) input is read through its values, like the reference.
    base = torch.randint(0, 256, (16, 12), dtype=torch.int32).to(torch.uint8)
    view = base.to(DEV).t()
    np.testing.assert_array_equal(unpack_int4(view, 32).cpu().numpy(), qo.unpack_nibbles(base.t().numpy(), 32))


# ---- dequantize --------------------------------------------------------------------------------

@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize(
    "rows,cols,group",
    # 8-code chunks (the vectorized kernel), then K % 8 != 0 and group % 8 != 0 (the generic one)
    [(48, 256, 128), (64, 176, 16), (33, 96, 32), (16, 512, 0), (8, 100, 10), (16, 96, 12)],
)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_dequant_bit_exact(bits, symmetric, rows, cols, group, dtype):
    qt = _host_qt(rows, cols, bits, group if group else cols, symmetric, seed=rows + cols + bits)
    if group == 0:
        qt = QuantizedTensor(qt.qweight, qt.scales, qt.zeros, qt.bits, 0, qt.symmetric, qt.shape)
    got = dequantize(_to_device(qt), dtype)
    assert got.dtype == dtype and got.shape == (rows, cols)
    np.testing.assert_array_equal(_bits_of(got), _expected_bits(_oracle_dense(qt), dtype))


@pytest.mark.parametrize("bits,symmetric", [(4, False), (4, True), (2, False), (2, True)])
@pytest.mark.parametrize("rows,cols,group", [(33, 2048, 128), (7, 6144, 32), (5, 4096, 2048), (3, 2048, 0)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dequant_whole_line_kernel_bit_exact(bits, symmetric, rows, cols, group, dtype):
    # Nibble codes into 16-bit weights with rows of whole 2048-code chunks: one wave per chunk,
    # 256-byte code loads and 1 KB stores (odd row counts, groups smaller and larger than a
    # wave's 512-code stride, a whole-row group).
    qt = _host_qt(rows, cols, bits, group if group else cols, symmetric, seed=rows + cols + bits)
    if group == 0:
        qt = QuantizedTensor(qt.qweight, qt.scales, qt.zeros, qt.bits, 0, qt.symmetric, qt.shape)
    got = dequantize(_to_device(qt), dtype)
    np.testing.assert_array_equal(_bits_of(got), _expected_bits(_oracle_dense(qt), dtype))


def test_dequant_more_rows_than_one_grid_dimension():
    # 70000 rows exceed the 65535 workgroups of one grid dimension: rows are strided.
    qt = _host_qt(70000, 16, 4, 8, False, seed=11)
    got = dequantize(_to_device(qt), torch.bfloat16)
    np.testing.assert_array_equal(_bits_of(got), _expected_bits(_oracle_dense(qt), torch.bfloat16))


def test_dequant_extreme_scales_bit_exact():
    # Denormal products, bf16 overflow to infinity and non-integer zero points.
    qt = _host_qt(8, 128, 4, 32, False, seed=5)
    scales = qt.scales.clone()
    scales[0] = 1e-41
    scales[1] = 3e37
    scales[2] = -0.37
    zeros = qt.zeros.clone()
    zeros[3] = 2.5
    odd = QuantizedTensor(qt.qweight, scales, zeros, 4, 32, False, qt.shape)
    dense = _oracle_dense(odd)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        np.testing.assert_array_equal(_bits_of(dequantize(_to_device(odd), dtype)), _expected_bits(dense, dtype))


def test_dequant_full_size_gate_up_bit_exact():
    qt = _host_qt(28672, 4096, 4, 128, False, seed=0)
    got = dequantize(_to_device(qt), torch.bfloat16)
    np.testing.assert_array_equal(_bits_of(got), _expected_bits(_oracle_dense(qt), torch.bfloat16))


# ---- quantized linear: small shapes against the CPU reference sequence ------------------------

SMALL_SHAPES = [  # (N, K, group)
    (48, 256, 128),
    (32, 64, 64),  # tiny-model k/v projection
    (64, 176, 16),  # tiny-model down_proj: 88-byte packed rows
    (200, 512, 128),  # N not a multiple of any tile
    (96, 384, 64),
    (64, 448, 32),  # 7 k-stages of 64 (a three-stage tail), two groups per stage
    (80, 768, 256),  # a group spanning four k-stages
    (64, 1024, 512),
    (80, 1024, 128),  # eight 128-code steps: the multi-tile decode kernel
    (48, 2048, 256),
]


@pytest.mark.parametrize("algo", [ALGO_AUTO, ALGO_GENERIC, ALGO_DECODE, ALGO_PREFILL])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bits,symmetric", [(4, False), (4, True), (8, False), (8, True), (2, False)])
@pytest.mark.parametrize("n,k,group", SMALL_SHAPES)
@pytest.mark.parametrize("m", [1, 5, 16, 33, 64, 200])
def test_linear_small_shapes(algo, dtype, bits, symmetric, n, k, group, m):
    qt = _host_qt(n, k, bits, group, symmetric, seed=n * 7 + k + bits)
    gen = torch.Generator().manual_seed(m + n)
    x = torch.randn(m, k, generator=gen).to(dtype)
    try:
        y = ops.quant_linear(x.to(DEV), _to_device(qt), None, dtype, algo=algo)
    except NotImplementedError:
        assert algo in (ALGO_DECODE, ALGO_PREFILL)  # outside that kernel's envelope
        if algo == ALGO_DECODE:
            assert m > 64 or dtype == torch.float32 or group % 64 or k % 64
        return
    ref = _reference_linear(x, _oracle_dense(qt), None, dtype)
    assert y.dtype == dtype and y.shape == (m, n)
    assert _rel_err(y, ref) <= TOL[dtype], (algo, dtype, bits, symmetric, n, k, m)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize("m", [5, 8, 16, 24, 33, 48])
def test_linear_batched_decode_shapes(dtype, symmetric, m):
    # K = 4096 (32 steps of 128 codes), 64 tiles of 16 features: up to M = 32 the multi-tile
    # kernel with every wave's range loaded up front; above 32 the split-K GEMM.
    qt = _host_qt(1024, 4096, 4, 128, symmetric, seed=m)
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, 4096, generator=gen).to(dtype)
    bias = torch.randn(1024, generator=gen).to(dtype)
    y = ops.quant_linear(x.to(DEV), _to_device(qt), bias.to(DEV), dtype)
    assert _rel_err(y, _reference_linear(x, _oracle_dense(qt), bias, dtype)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [20, 32])
@pytest.mark.parametrize("n", [6144, 16384])
def test_linear_batched_decode_ring_configuration(dtype, m, n):
    # M = 17-32: 384 tiles of 16 features on two-wave, two-tile workgroups; 1024 tiles on
    # eight-wave workgroups of one tile per wave.
    qt = _host_qt(n, 4096, 4, 128, False, seed=m)
    x = torch.randn(m, 4096, generator=torch.Generator().manual_seed(m)).to(dtype)
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None, dtype)
    assert _rel_err(y, _reference_linear(x, _oracle_dense(qt), None, dtype)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [5, 8, 16, 17, 32, 33, 47, 64])
@pytest.mark.parametrize("n, bits, group, symmetric", [(16400, 4, 128, False), (16384, 4, 256, True),
                                                     (16384, 2, 128, False)])
def test_linear_n_split_decode(dtype, m, n, bits, group, symmetric):
    # 5-32 tokens over at least 1024 tiles of 16 features: eight single-tile waves per
    # workgroup sharing the activations through LDS. N = 16400 leaves the last workgroup one
    # live tile (rows past N); groups of 256 codes span two steps; 2-bit codes; bias on.
    qt = _host_qt(n, 4096, bits, group, symmetric, seed=m + n)
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, 4096, generator=gen).to(dtype)
    bias = torch.randn(n, generator=gen).to(dtype)
    y = ops.quant_linear(x.to(DEV), _to_device(qt), bias.to(DEV), dtype)
    assert _rel_err(y, _reference_linear(x, _oracle_dense(qt), bias, dtype)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [5, 12, 17, 32])
@pytest.mark.parametrize("n, k, group, symmetric", [(6144, 4096, 128, False), (4096, 14336, 128, False),
                                                   (2048, 8192, 256, True), (4096, 9216, 128, False)])
def test_linear_n_split_over_k_slices(dtype, m, n, k, group, symmetric):
    # Fewer than 1024 tiles: the kernels that split K over workgroups (fp32 partial sums in the
    # workspace, then the fixed-order reduction, which adds the bias), and the same call through
    # the C-ABI without a workspace, which takes the other decode kernels.
    qt = _host_qt(n, k, 4, group, symmetric, seed=m + k)
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, k, generator=gen).to(dtype)
    bias = torch.randn(n, generator=gen).to(dtype)
    ref = _reference_linear(x, _oracle_dense(qt), bias, dtype)
    dq = _to_device(qt)
    xd, bd = x.to(DEV), bias.to(DEV)
    y = ops.quant_linear(xd, dq, bd, dtype)
    assert _rel_err(y, ref) <= TOL[dtype]
    lib = _lib.load_library()
    # The K-sliced kernel takes K a multiple of 2048 from 5 tokens with K >= 8192 and from 17
    # with shorter rows, except the 5-32 tokens over K = 4096 in groups of 128 that the
    # resident-activation kernel takes unsplit; the N-split kernel slices K = 9216 from 12 tokens
    # (8 or 4 steps a chunk, 9 slices give the 32 workgroups of 8 tiles 288 in all).
    kr = k == 4096 and group == 128 and 5 <= m <= 32
    ks = k % 2048 == 0 and m >= (5 if k >= 8192 else 17) and not kr
    nx = k == 9216 and m >= 12
    assert (lib.llmopt_q_linear_workspace(m, n, k, 4, group) > 0) == (ks or nx)
    y2 = torch.empty(m, n, dtype=dtype, device=DEV)
    qw, ldq, sc, zr, _, _, grp, signed = ops._weight_args(dq, xd.device)
    rc = lib.llmopt_q_linear(xd.data_ptr(), m, k, k, qw.data_ptr(), ldq, sc.data_ptr(),
                             zr.data_ptr() if zr is not None else None, bd.data_ptr(), y2.data_ptr(), n, n,
                             _lib.DTYPE_CODES[dtype], 4, grp, int(symmetric), int(signed), None, 0,
                             torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert _rel_err(y2, ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [24, 32])
def test_linear_long_rows_at_24_to_32_tokens(dtype, m):
    # K >= 8192 from 24 tokens: a kernel that splits K over workgroups when the workspace is
    # there (ops passes it; the K-sliced decode kernel on this grid), the decode kernels that
    # need none when it is not (a C-ABI caller without one).
    qt = _host_qt(512, 8192, 4, 128, False, seed=m)
    x = torch.randn(m, 8192, generator=torch.Generator().manual_seed(m)).to(dtype)
    ref = _reference_linear(x, _oracle_dense(qt), None, dtype)
    dq = _to_device(qt)
    y = ops.quant_linear(x.to(DEV), dq, None, dtype)
    assert _rel_err(y, ref) <= TOL[dtype]
    lib = _lib.load_library()
    assert lib.llmopt_q_linear_workspace(m, 512, 8192, 4, 128) > 0
    xd = x.to(DEV)
    y2 = torch.empty(m, 512, dtype=dtype, device=DEV)
    rc = lib.llmopt_q_linear(xd.data_ptr(), m, 8192, 8192, dq.qweight.data_ptr(), 4096, dq.scales.data_ptr(),
                             dq.zeros.data_ptr(), None, y2.data_ptr(), 512, 512, _lib.DTYPE_CODES[dtype], 4, 128, 0, 0,
                             None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert _rel_err(y2, ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 40, 300])
def test_linear_bias_and_leading_dims(dtype, m):
    qt = _host_qt(96, 256, 4, 128, False, seed=3)
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, 256, generator=gen).to(dtype)
    bias = torch.randn(96, generator=gen).to(dtype)
    y = ops.quant_linear(x.to(DEV).reshape(1, m, 256), _to_device(qt), bias.to(DEV), dtype)
    ref = _reference_linear(x, _oracle_dense(qt), bias, dtype)
    assert y.shape == (1, m, 96)
    assert _rel_err(y.reshape(m, 96), ref) <= TOL[dtype]


def test_linear_strided_and_one_dimensional_inputs():
    qt = _host_qt(64, 256, 4, 128, True, seed=8)
    dqt = _to_device(qt)
    big = torch.randn(7, 512).to(torch.bfloat16)
    strided = big.to(DEV)[:, 128:384]  # row stride 512, 16-byte aligned start
    y = ops.quant_linear(strided, dqt, None, torch.bfloat16)
    ref = _reference_linear(big[:, 128:384].contiguous(), _oracle_dense(qt), None, torch.bfloat16)
    assert _rel_err(y, ref) <= 1e-2
    odd = big.to(DEV)[:, 3:259]  # misaligned start: taken by the generic kernel
    ref_odd = _reference_linear(big[:, 3:259].contiguous(), _oracle_dense(qt), None, torch.bfloat16)
    assert _rel_err(ops.quant_linear(odd, dqt, None, torch.bfloat16), ref_odd) <= 1e-2
    v = torch.randn(256).to(torch.bfloat16)
    y1 = ops.quant_linear(v.to(DEV), dqt, None, torch.bfloat16)
    assert y1.shape == (64,)
    assert _rel_err(y1, _reference_linear(v[None], _oracle_dense(qt), None, torch.bfloat16)[0]) <= 1e-2


def test_linear_empty_batch_and_errors():
    dqt = _to_device(_host_qt(32, 128, 4, 64, False, seed=1))
    y = ops.quant_linear(torch.empty(0, 128, dtype=torch.bfloat16, device=DEV), dqt, None, torch.bfloat16)
    assert y.shape == (0, 32)
    with pytest.raises(RuntimeError):
        ops.quant_linear(torch.randn(2, 128, device=DEV), dqt, None, torch.bfloat16)
    with pytest.raises(RuntimeError):
        ops.quant_linear(torch.randn(2, 100, device=DEV, dtype=torch.bfloat16), dqt, None, torch.bfloat16)
    with pytest.raises(RuntimeError):
        bad_bias = torch.zeros(32, device=DEV)
        ops.quant_linear(torch.randn(2, 128, device=DEV, dtype=torch.bfloat16), dqt, bad_bias, torch.bfloat16)


def test_linear_is_deterministic():
    dqt = _to_device(_host_qt(4096, 4096, 4, 128, False, seed=2))
    for m in (1, 32, 512):
        x = torch.randn(m, 4096, device=DEV).to(torch.bfloat16)
        a = ops.quant_linear(x, dqt, None, torch.bfloat16)
        b = ops.quant_linear(x, dqt, None, torch.bfloat16)
        assert torch.equal(a, b)


# ---- full Llama-3-8B projection sizes ---------------------------------------------------------

PROJECTIONS = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (28672, 4096), "down": (4096, 14336)}


@pytest.fixture(scope="module")
def projections():
    out = {}
    for i, (name, (n, k)) in enumerate(PROJECTIONS.items()):
        qt = _host_qt(n, k, 4, 128, False, seed=i)
        out[name] = (qt, _to_device(qt), _oracle_dense(qt))
    return out


@pytest.mark.parametrize("name", list(PROJECTIONS))
@pytest.mark.parametrize("m", [1, 8, 32, 64, 256, 2048, 8192])
def test_projection_sampled_columns_and_gpu_fp32(projections, name, m):
    # Decode and prefill batches of the Llama-3-8B projections, up to the 8192-token prefill.
    # The CPU reference runs on 256 sampled output columns (and, above 2048 tokens, 256
    # sampled rows: each output row depends only on its own activation row); every output
    # is checked against a torch fp32 GPU matmul of the bit-exact dequantized weight.
    qt, dqt, dense = projections[name]
    n, k = qt.shape
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16)
    y = ops.quant_linear(x.to(DEV), dqt, None, torch.bfloat16)
    cols = np.sort(np.random.default_rng(m).choice(n, size=256, replace=False))
    rows = np.arange(m) if m <= 2048 else np.sort(np.random.default_rng(m + 1).choice(m, size=256, replace=False))
    ref = _reference_linear(x[torch.from_numpy(rows)], dense, None, torch.bfloat16, cols=cols)
    got = y[torch.from_numpy(rows).to(DEV)][:, torch.from_numpy(cols).to(DEV)]
    assert _rel_err(got, ref) <= 1e-2
    w32 = dequantize(dqt, torch.bfloat16).float()  # bit-exact (checked above)
    ref_gpu = torch.matmul(x.to(DEV).float(), w32.t().contiguous())
    assert _rel_err(y, ref_gpu) <= 1e-2


def _gpu_rel_err(y: torch.Tensor, ref: torch.Tensor) -> float:
    """max|y - ref| / max|ref| computed on the device (for outputs of a few GB)."""
    d = float(ref.float().abs().max())
    return float((y.float() - ref.float()).abs().max()) / (d if d > 0 else 1.0)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name", list(PROJECTIONS))
def test_projection_end_to_end_prefill_batch(projections, name):
    # The end-to-end workload's prefill: 32 prompts x 512 tokens = 16384 rows through each
    # projection in one call (src/llmopt/model/layers.py:39-44,106-108,142). Sampled rows x
    # columns against the CPU reference; every output against a torch fp32 GPU matmul of the
    # bit-exact dequantized weight; scaling x by 2 scales y by 2 exactly; one-hot activation
    # rows return the dequantized weight's columns bit for bit.
    m = 16384
    qt, dqt, dense = projections[name]
    n, k = qt.shape
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    xd = x.to(DEV)
    y = ops.quant_linear(xd, dqt, None, torch.bfloat16)
    rng = np.random.default_rng(m + n)
    rows = np.sort(rng.choice(m, size=256, replace=False))
    cols = np.sort(rng.choice(n, size=256, replace=False))
    ref = _reference_linear(x[torch.from_numpy(rows)], dense, None, torch.bfloat16, cols=cols)
    got = y[torch.from_numpy(rows).to(DEV)][:, torch.from_numpy(cols).to(DEV)]
    assert _rel_err(got, ref) <= 1e-2
    w = dequantize(dqt, torch.bfloat16)  # bit-exact with the oracle (checked above)
    ref_gpu = torch.matmul(xd.float(), w.float().t().contiguous())
    assert _gpu_rel_err(y, ref_gpu) <= 1e-2
    del ref_gpu
    assert torch.equal(ops.quant_linear(xd * 2, dqt, None, torch.bfloat16), y * 2)
    del y
    picks = torch.from_numpy(rng.choice(k, size=m, replace=True)).to(DEV)
    one_hot = torch.zeros(m, k, dtype=torch.bfloat16, device=DEV)
    one_hot[torch.arange(m, device=DEV), picks] = 1.0
    y1 = ops.quant_linear(one_hot, dqt, None, torch.bfloat16)
    assert torch.equal(y1.view(torch.int16), w[:, picks].t().contiguous().view(torch.int16))


@pytest.mark.parametrize("name", list(PROJECTIONS))
@pytest.mark.parametrize("m", [1, 64, 2048, 8192])
def test_projection_one_hot_rows_return_weight_columns(projections, name, m):
    _, dqt, dense = projections[name]
    n, k = dense.shape
    picks = np.random.default_rng(k + m).choice(k, size=m, replace=m > k)
    x = torch.zeros(m, k, dtype=torch.bfloat16)
    x[torch.arange(m), torch.from_numpy(picks)] = 1.0
    y = ops.quant_linear(x.to(DEV), dqt, None, torch.bfloat16)
    expect = qo.bf16_bits(np.ascontiguousarray(dense[:, picks].T)).view(np.int16)
    np.testing.assert_array_equal(_bits_of(y), expect)


@pytest.mark.parametrize("name,m", [("down", 1), ("down", 32), ("down", 2048)]
                         + [(name, 8192) for name in PROJECTIONS])
def test_projection_scaling_by_two_is_exact(projections, name, m):
    qt, dqt, _ = projections[name]
    x = torch.randn(m, qt.shape[1], device=DEV).to(torch.bfloat16)
    y1 = ops.quant_linear(x, dqt, None, torch.bfloat16)
    y2 = ops.quant_linear(x * 2, dqt, None, torch.bfloat16)
    assert torch.equal(y2, y1 * 2)


@pytest.mark.parametrize("bits,symmetric,m", [(8, False, 1), (8, False, 32), (8, False, 2048), (2, False, 1),
                                              (2, False, 12), (2, False, 16), (2, False, 32), (2, False, 2048),
                                              (8, True, 32)])
def test_down_projection_bit_width_sweep(bits, symmetric, m):
    qt = _host_qt(4096, 14336, bits, 128, symmetric, seed=bits)
    dqt = _to_device(qt)
    dense = _oracle_dense(qt)
    x = torch.randn(m, 14336, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    y = ops.quant_linear(x.to(DEV), dqt, None, torch.bfloat16)
    cols = np.sort(np.random.default_rng(bits + m).choice(4096, size=128, replace=False))
    ref = _reference_linear(x, dense, None, torch.bfloat16, cols=cols)
    assert _rel_err(y[:, torch.from_numpy(cols).to(DEV)], ref) <= 1e-2


@pytest.mark.parametrize("m", [33, 48, 64])
@pytest.mark.parametrize("bits, group", [(8, 128), (4, 32), (4, 64), (4, 128)])
def test_wide_grids_at_33_to_64_tokens_every_format(m, bits, group):
    # 33-64 tokens over 1024 tiles of 16 features with K = 4096: 2/4-bit codes in groups of a
    # multiple of 128 run on the N-split decode kernel, other formats on the split-K GEMM.
    n, k = 16384, 4096
    qt = _host_qt(n, k, bits, group, False, seed=m + bits + group)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None, torch.bfloat16)
    cols = np.sort(np.random.default_rng(m + group).choice(n, size=256, replace=False))
    ref = _reference_linear(x, _oracle_dense(qt), None, torch.bfloat16, cols=cols)
    assert _rel_err(y[:, torch.from_numpy(cols).to(DEV)], ref) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 12, 16, 24, 32, 33, 40, 48, 49, 64])
@pytest.mark.parametrize("n, k, bits, symmetric, with_bias", [
    (6144, 4096, 4, True, False), (28672, 4096, 4, True, False), (4100, 4096, 4, False, True),
    (4096, 14336, 4, True, False), (1000, 2048, 2, False, True)])
def test_linear_groups_of_64(dtype, m, n, k, bits, symmetric, with_bias):
    # Groups of 64 codes (the reference engine's quantize_model_(bits=4, group_size=64),
    # src/llmopt/engine/llm_engine.py:258-264): two groups per 128-code step on the one-shot
    # (M <= 8) and multi-tile (M <= 32) decode kernels, with the code words transposed across
    # the wave's rows; ragged N, bias, 2-bit codes, long rows; up to 48 tokens on the K-sliced
    # kernel (three token blocks from 33), 49-64 on the skinny kernel.
    qt = _host_qt(n, k, bits, 64, symmetric, seed=m + n + k)
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, k, generator=gen).to(dtype)
    bias = torch.randn(n, generator=gen).to(dtype) if with_bias else None
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None if bias is None else bias.to(DEV), dtype)
    cols = np.sort(np.random.default_rng(m + k).choice(n, size=min(n, 256), replace=False))
    ref = _reference_linear(x, _oracle_dense(qt), bias, dtype, cols=cols)
    assert _rel_err(y[:, torch.from_numpy(cols).to(DEV)], ref) <= TOL[dtype]


@pytest.mark.parametrize("m", [1, 4, 8, 16, 32, 48])
def test_groups_of_64_one_hot_rows_return_weight_columns(m):
    # One-hot activation rows return the dequantized weight's columns bit for bit: every other
    # group and step adds exactly zero, and s * ((OFF + q) - (OFF + z)) rounds (q - z) * s once.
    n, k = 6144, 4096
    qt = _host_qt(n, k, 4, 64, False, seed=m)
    dense = _oracle_dense(qt)
    picks = np.random.default_rng(k + m).choice(k, size=m, replace=False)
    x = torch.zeros(m, k, dtype=torch.bfloat16)
    x[torch.arange(m), torch.from_numpy(picks)] = 1.0
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None, torch.bfloat16)
    expect = qo.bf16_bits(np.ascontiguousarray(dense[:, picks].T)).view(np.int16)
    np.testing.assert_array_equal(_bits_of(y), expect)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("n, k, symmetric, with_bias", [
    (6144, 4096, False, False), (4100, 4096, True, True), (4096, 14336, False, False), (4096, 14336, True, False),
    (16400, 4096, False, True)])
def test_linear_byte_codes_decode(dtype, m, n, k, symmetric, with_bias):
    # 8-bit codes (uint8 asymmetric, int8 symmetric, quantizers.py:231-234) at 1-64 tokens: the
    # line kernel's byte form at one token on long rows, the one-shot kernel's (32 bytes per
    # lane and step) at 1-8 tokens where it fits, the K-sliced kernel's (1024-code slices) from
    # 3 tokens on long rows and from 9 on K = 4096, on any grid (N = 16400: 1025 tiles), the
    # streaming kernel for the rest; ragged N, bias, long rows.
    qt = _host_qt(n, k, 8, 128, symmetric, seed=m + n + k)
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, k, generator=gen).to(dtype)
    bias = torch.randn(n, generator=gen).to(dtype) if with_bias else None
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None if bias is None else bias.to(DEV), dtype)
    cols = np.sort(np.random.default_rng(m + k).choice(n, size=256, replace=False))
    ref = _reference_linear(x, _oracle_dense(qt), bias, dtype, cols=cols)
    assert _rel_err(y[:, torch.from_numpy(cols).to(DEV)], ref) <= TOL[dtype]


@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize("m", [1, 2])
def test_byte_codes_one_hot_rows_return_weight_columns(symmetric, m):
    # Byte operands are the codes themselves (bf16): a one-hot row returns (q - z) * s rounded
    # once, then to bf16, bit for bit.
    n, k = 4096, 14336
    qt = _host_qt(n, k, 8, 128, symmetric, seed=m + 40)
    dense = _oracle_dense(qt)
    picks = np.random.default_rng(k + m).choice(k, size=m, replace=False)
    x = torch.zeros(m, k, dtype=torch.bfloat16)
    x[torch.arange(m), torch.from_numpy(picks)] = 1.0
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None, torch.bfloat16)
    expect = qo.bf16_bits(np.ascontiguousarray(dense[:, picks].T)).view(np.int16)
    np.testing.assert_array_equal(_bits_of(y), expect)


def _unusual_metadata_qt():
    """W4 g128 weights whose metadata leaves what the quantizers produce: fractional and
    negative zero points, zero points of 16, scales of 2^100 and 2^121."""
    qt = _host_qt(512, 1024, 4, 128, False, seed=7)
    scales, zeros = qt.scales.clone(), qt.zeros.clone()
    zeros[0::5] += 0.5
    zeros[1::5] = -3.0
    zeros[2::5] = 16.0
    scales[3::10] *= 2.0 ** 100
    scales[8::10] *= 2.0 ** 121
    return QuantizedTensor(qt.qweight, scales, zeros, 4, 128, False, qt.shape)


@pytest.mark.parametrize("m", [256, 2048])
def test_prefill_unusual_zero_points_and_scales(m):
    # The prefill GEMM's dequantization adds 16 - z to the code bytes when z is an integer in
    # [-224, 16] and |s| < 2^120 (bit-exact), and falls back to fma(q, s, -z s) otherwise.
    qt = _unusual_metadata_qt()
    dqt = _to_device(qt)
    dense = _oracle_dense(qt)
    x = torch.randn(m, 1024, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    y = ops.quant_linear(x.to(DEV), dqt, None, torch.bfloat16, algo=ALGO_PREFILL).float().cpu()
    ref = _reference_linear(x, dense, None, torch.bfloat16).float()
    # Rows differ in scale by up to 2^121: compare each output feature against its own range.
    err = (y - ref).abs().amax(dim=0) / ref.abs().amax(dim=0).clamp_min(1e-30)
    assert float(err.max()) <= 1e-2
    # One-hot rows return the weight column bit for bit where the zero point is an integer in
    # range and the scale below 2^120 (every row but the fractional-zero and 2^121-scale ones).
    picks = np.random.default_rng(m).choice(1024, size=m, replace=True)
    oh = torch.zeros(m, 1024, dtype=torch.bfloat16)
    oh[torch.arange(m), torch.from_numpy(picks)] = 1.0
    y1 = ops.quant_linear(oh.to(DEV), dqt, None, torch.bfloat16, algo=ALGO_PREFILL)
    exact_rows = np.array([r for r in range(512) if r % 5 != 0 and r % 10 != 8])
    expect = qo.bf16_bits(np.ascontiguousarray(dense[:, picks].T)).view(np.int16)
    np.testing.assert_array_equal(_bits_of(y1)[:, exact_rows], expect[:, exact_rows])


def test_fp32_compute_single_linear_config():
    # The reference's CPU configuration: K = N = 4096, fp32, M = 1, RTN b4 asym g128.
    qt = _host_qt(4096, 4096, 4, 128, False, seed=0)
    x = torch.randn(1, 4096, generator=torch.Generator().manual_seed(1))
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None, torch.float32)
    ref = _reference_linear(x, _oracle_dense(qt), None, torch.float32)
    assert _rel_err(y, ref) <= 2e-3


# ---- GPTQ-quantized weights through the kernels ------------------------------------------------

@pytest.fixture(scope="module")
def gptq_down():
    """The down projection (K 14336, N 4096) quantized by GPTQQuantizer: 4 bits, groups of
    128, damping 0.01, activation order, calibrated on H = (2/128) X^T X of 128 token rows
    gathered from a seeded N(0, 1) embedding table (seed 2) at seeded random ids (seed 3).
    Weights 0.02 N(0, 1), seed 0. Runs on the GPU (torch), asymmetric and symmetric grids."""
    from llmopt.quantization import GPTQQuantizer

    k, n = 14336, 4096
    table = torch.randn(1024, k, generator=torch.Generator().manual_seed(2))
    ids = torch.randint(0, 1024, (128,), generator=torch.Generator().manual_seed(3))
    x_cal = table[ids].to(DEV)
    hessian = (2.0 / 128) * (x_cal.t() @ x_cal)
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(0)) * 0.02).to(DEV)
    out = {}
    for symmetric in (False, True):
        qt = GPTQQuantizer(bits=4, group_size=128, symmetric=symmetric).quantize(w, hessian)
        host = QuantizedTensor(qt.qweight.cpu(), qt.scales.cpu(), qt.zeros.cpu(), 4, 128, symmetric, qt.shape)
        out[symmetric] = (qt, _oracle_dense(host))
    return out


@pytest.mark.timeout(600)
@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize("m", [1, 32, 2048])
def test_gptq_down_projection_through_the_kernels(gptq_down, symmetric, m):
    qt, dense = gptq_down[symmetric]
    assert qt.qweight.device.type == "cuda" and qt.qweight.shape == (4096, 7168)
    x = torch.randn(m, 14336, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    y = ops.quant_linear(x.to(DEV), qt, None, torch.bfloat16)
    cols = np.sort(np.random.default_rng(m + 7).choice(4096, size=256, replace=False))
    ref = _reference_linear(x, dense, None, torch.bfloat16, cols=cols)
    assert _rel_err(y[:, torch.from_numpy(cols).to(DEV)], ref) <= 1e-2
    # The device dequantization of a GPTQ weight is the oracle's, bit for bit.
    np.testing.assert_array_equal(_bits_of(dequantize(qt, torch.bfloat16)), _expected_bits(dense, torch.bfloat16))
    # One-hot rows read back single weight columns exactly.
    picks = np.random.default_rng(m).choice(14336, size=min(m, 64), replace=False)
    hot = torch.zeros(len(picks), 14336, dtype=torch.bfloat16)
    hot[torch.arange(len(picks)), torch.from_numpy(picks)] = 1.0
    yh = ops.quant_linear(hot.to(DEV), qt, None, torch.bfloat16)
    np.testing.assert_array_equal(_bits_of(yh), qo.bf16_bits(np.ascontiguousarray(dense[:, picks].T)).view(np.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [2, 5, 16, 17, 31, 32, 33, 48, 64])
@pytest.mark.parametrize("n, k, bits, group, symmetric, with_bias", [
    (4100, 14336, 4, 128, False, True),  # 257 tiles, the last partial; 7 K slices, 36 workgroups each
    (6144, 4096, 4, 128, True, False),   # qkv: 2 slices of 128 workgroups, three tiles each
    (1000, 2048, 4, 256, False, True),   # one slice (no reduction kernel), groups of two steps
    (4096, 8192, 2, 128, False, False),  # 2-bit codes, 4 slices
    (2048, 6144, 4, 384, True, True),    # groups of three steps, 3 slices
])
def test_linear_k_sliced_decode(dtype, m, n, k, bits, group, symmetric, with_bias):
    # Fewer than 1024 tiles of 16 features, 5-64 tokens on rows of at least 8192 codes and 17-64
    # on shorter ones: workgroups own a K slice of 2048 codes and walk a strided list of tiles,
    # the slices' sums meeting in the reduction kernel (the other token counts check the kernels
    # that take them on the same shapes).
    qt = _host_qt(n, k, bits, group, symmetric, seed=m + n + k)
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, k, generator=gen).to(dtype)
    bias = torch.randn(n, generator=gen).to(dtype) if with_bias else None
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None if bias is None else bias.to(DEV), dtype)
    assert _rel_err(y, _reference_linear(x, _oracle_dense(qt), bias, dtype)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [5, 9, 16, 17, 24, 32])
@pytest.mark.parametrize("n, bits, symmetric, with_bias, strided", [
    (4100, 4, False, True, True),     # 257 tiles, two per workgroup, the last one partial; x rows strided
    (4096, 2, True, False, False),    # 2-bit codes, one tile per workgroup
    (12288, 4, False, False, False),  # 768 tiles: four per workgroup
    (28672, 4, True, True, False),    # gate_up: seven tiles per workgroup, 256 workgroups
])
def test_linear_resident_activation_decode(dtype, m, n, bits, symmetric, with_bias, strided):
    # 5-32 tokens over K = 4096 with groups of 128: eight waves per workgroup, each holding the
    # activations of its 512 codes of K, loaded in whole lines and rearranged through LDS.
    k = 4096
    qt = _host_qt(n, k, bits, 128, symmetric, seed=m + n)
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, k + (64 if strided else 0), generator=gen).to(dtype)[:, :k]
    bias = torch.randn(n, generator=gen).to(dtype) if with_bias else None
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None if bias is None else bias.to(DEV), dtype)
    assert _rel_err(y, _reference_linear(x, _oracle_dense(qt), bias, dtype)) <= TOL[dtype]


@pytest.mark.parametrize("m", [5, 17, 32])
def test_linear_resident_activation_one_hot_rows(m):
    # One-hot activation rows through the resident-activation kernel return dequantized weight
    # columns bit for bit: every other term of each MFMA sum and step correction is exactly zero.
    qt = _host_qt(4096, 4096, 4, 128, False, seed=m)
    dense = _oracle_dense(qt)
    picks = np.random.default_rng(m).choice(4096, size=m, replace=False)
    x = torch.zeros(m, 4096, dtype=torch.bfloat16)
    x[torch.arange(m), torch.from_numpy(picks)] = 1.0
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None, torch.bfloat16)
    expect = qo.bf16_bits(np.ascontiguousarray(dense[:, picks].T)).view(np.int16)
    np.testing.assert_array_equal(_bits_of(y), expect)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("n, k, symmetric, with_bias", [(16400, 4096, False, True), (28672, 4096, True, False),
                                                        (16384, 2048, False, False), (20480, 6144, False, True)])
def test_linear_persistent_line_decode(dtype, m, n, k, symmetric, with_bias):
    # 1-8 tokens over at least 1024 tiles of 16 features: one workgroup per CU walks a strided
    # list of tiles (N = 16400: 1025 tiles, the last one partial; K 2048 / 4096 / 6144 give
    # 1, 2 and 3 blocks of 256 codes per wave, the first and last taken by other kernels).
    qt = _host_qt(n, k, 4, 128, symmetric, seed=m + n + k)
    gen = torch.Generator().manual_seed(m)
    x = torch.randn(m, k, generator=gen).to(dtype)
    bias = torch.randn(n, generator=gen).to(dtype) if with_bias else None
    y = ops.quant_linear(x.to(DEV), _to_device(qt), None if bias is None else bias.to(DEV), dtype)
    assert _rel_err(y, _reference_linear(x, _oracle_dense(qt), bias, dtype)) <= TOL[dtype]

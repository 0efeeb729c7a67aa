"""Which shapes split K, and into how many slices, as the C ABI reports it on the host.

``llmopt_q_linear_workspace`` is the host side of the kernel choice: it returns the bytes of
fp32 partial sums (``slices * M * N * 4``) of the kernel a call of that size would pick when it
splits K over workgroups, and 0 when it does not. These tests pin that choice for the
Llama-3-8B projections without a GPU (no kernel is launched):

* nothing for the resident-activation decode kernel: 5-32 tokens over K = 4096 with groups of
  128 (qkv, o, gate_up) keep all of K in each workgroup;
* the K-sliced decode kernel: fewer than 1024 tiles of 16 output features, 2/4-bit codes in
  groups of a multiple of 128, K a multiple of 2048, 5-64 tokens when K >= 8192 and 17-64 on
  shorter rows where the resident-activation kernel does not take them; one slice per 2048
  codes (down: 7, qkv and o at 33-64 tokens: 2);
* the N-split kernel over K slices, only where the K-sliced kernel does not take the shape
  (K >= 8192 not a multiple of 2048, 12-32 tokens);
* nothing for gate_up up to 64 tokens (its N-split kernel keeps all of K per workgroup), nor at
  1-4 tokens anywhere;
* the prefill GEMM's own plan above 64 tokens;
* from 1024 tokens the two-pass path: the dense weight in the compute dtype (256-byte aligned)
  and 32 MiB for hipBLASLt, or the fused plan's bytes where those are more (what runs when
  hipBLASLt has no algorithm); fp32 activations from 65 tokens.
"""

from __future__ import annotations

import pytest
import torch  # noqa: F401 - load torch's HIP runtime before the library

from llmopt.kernels import _lib

QKV, O, GATE_UP, DOWN = (6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().exists():
        pytest.fail(f"kernel library not built: {_lib.library_path()} (run __graft_entry__.build())")
    return _lib.load_library()


def _ws(lib, m, shape, bits=4, group=128):
    n, k = shape
    return lib.llmopt_q_linear_workspace(m, n, k, bits, group)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("m", [5, 8, 16, 24, 32, 33, 48, 64])
def test_down_takes_seven_k_slices_from_five_tokens(lib, bits, m):
    assert _ws(lib, m, DOWN, bits) == 7 * m * 4096 * 4


@pytest.mark.parametrize("shape", [QKV, O])
def test_qkv_and_o_take_two_k_slices_from_thirty_three_tokens(lib, shape):
    n = shape[0]
    for m in range(1, 33):
        assert _ws(lib, m, shape) == 0, m
    for m in (33, 48, 64):
        assert _ws(lib, m, shape) == 2 * m * n * 4, m


def test_resident_activation_shapes_keep_all_of_k(lib):
    # K = 4096, groups of 128, 5-32 tokens: no split, whatever the grid (up to 7 tiles per
    # workgroup over 256 workgroups); K = 4096 with other groups, or 8192, still splits.
    for n in (16, 4100, 12288, 28672):
        for m in (5, 17, 32):
            assert _ws(lib, m, (n, 4096)) == 0, (n, m)
    assert _ws(lib, 24, (1000, 4096), group=256) == 2 * 24 * 1000 * 4
    assert _ws(lib, 24, (2048, 8192)) == 4 * 24 * 2048 * 4


def test_no_split_at_one_to_four_tokens(lib):
    for shape in (QKV, O, GATE_UP, DOWN):
        for m in range(1, 5):
            assert _ws(lib, m, shape) == 0, (shape, m)


def test_gate_up_keeps_all_of_k_up_to_64_tokens(lib):
    for m in (1, 5, 8, 16, 32, 33, 48, 64):
        assert _ws(lib, m, GATE_UP) == 0, m


def test_slices_follow_k(lib):
    # One slice per 2048 codes: K = 2048 runs unsplit, 8192 in four slices (4096 in two, where
    # the resident-activation kernel does not take the shape).
    assert _ws(lib, 24, (1000, 2048)) == 0
    assert _ws(lib, 24, (2048, 8192)) == 4 * 24 * 2048 * 4
    assert _ws(lib, 24, (2048, 6144), group=384) == 3 * 24 * 2048 * 4


def test_n_split_k_slices_where_the_k_sliced_kernel_does_not_fit(lib):
    # K = 9216 is not a multiple of 2048: 9 slices of the N-split kernel from 12 to 32 tokens.
    for m in range(5, 12):
        assert _ws(lib, m, (4096, 9216)) == 0, m
    for m in (12, 16, 17, 32):
        assert _ws(lib, m, (4096, 9216)) == 9 * m * 4096 * 4, m


def test_groups_of_32_never_take_the_decode_splits(lib):
    for m in (5, 8, 16):
        assert _ws(lib, m, DOWN, group=32) == 0


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 16, 32, 33, 64])
def test_groups_of_64_take_k_slices_up_to_32_tokens(lib, m):
    # Groups of 64 (nibble codes) run on the K-sliced kernel with four groups per block: down
    # (7 slices) from 3 tokens, K = 4096 (2 slices) from 9, on any grid; above 32 tokens the
    # split-K GEMM's own plan.
    down, gate_up = _ws(lib, m, DOWN, group=64), _ws(lib, m, GATE_UP, group=64)
    if m <= 32:
        assert down == (7 * m * 4096 * 4 if m >= 3 else 0)
        assert gate_up == (2 * m * 28672 * 4 if m >= 9 else 0)
    else:
        assert down % (m * 4096 * 4) == 0 and gate_up % (m * 28672 * 4) == 0


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 9, 16, 24, 32, 33, 48, 64])
def test_byte_codes_take_k_slices_of_1024_codes(lib, m):
    # 8-bit codes: a K slice of the K-sliced kernel is eight blocks of 128 bytes per row, 1024
    # codes, so down (K 14336) splits into 14 slices from 3 tokens; K = 4096 into 4 from 9
    # tokens, on any grid (gate_up too: no other fast kernel takes byte codes there).
    assert _ws(lib, m, DOWN, bits=8) == (14 * m * 4096 * 4 if m >= 3 else 0)
    assert _ws(lib, m, QKV, bits=8) == (4 * m * 6144 * 4 if m >= 9 else 0)
    assert _ws(lib, m, GATE_UP, bits=8) == (4 * m * 28672 * 4 if m >= 9 else 0)


def test_prefill_plans_above_64_tokens(lib):
    # The GEMM's K split is sized by its own plan: a multiple of one fp32 plane of M x N.
    for shape in (QKV, O, GATE_UP, DOWN):
        n = shape[0]
        for m in (65, 256, 1023):
            ws = _ws(lib, m, shape)
            assert ws % (m * n * 4) == 0 and ws // (m * n * 4) in (0, 2, 3, 4, 5, 6, 7, 8), (shape, m, ws)


BLAS_WS = 32 << 20


def _dense(n, k, es):
    return -(-n * k * es // 256) * 256 + BLAS_WS


@pytest.mark.parametrize("m", [1024, 2048, 8192, 16384])
def test_long_batches_take_the_two_pass_path(lib, m):
    for n, k in (QKV, O, GATE_UP, DOWN):
        assert lib.llmopt_q_linear_dense_workspace(n, k, _lib.DTYPE_CODES[torch.bfloat16]) == _dense(n, k, 2)
        assert lib.llmopt_q_linear_dense_workspace(n, k, _lib.DTYPE_CODES[torch.float32]) == _dense(n, k, 4)
        # The dense weight is larger than any split plan of these shapes.
        assert _ws(lib, m, (n, k)) == _dense(n, k, 2), (n, k, m)
        for bits, group in ((8, 128), (2, 64), (4, 32)):
            assert _ws(lib, m, (n, k), bits, group) == _dense(n, k, 2)
        # Fused gate/up + SwiGLU: the [M, N] product in the compute dtype, then the same.
        sw = lib.llmopt_q_linear_swiglu_workspace(m, n, k, 4, 128)
        assert sw == -(-m * n * 2 // 256) * 256 + _dense(n, k, 2)


def test_fp32_takes_the_two_pass_path_from_65_tokens(lib):
    f32 = _lib.DTYPE_CODES[torch.float32]
    n, k = GATE_UP
    assert lib.llmopt_q_linear_workspace_ex(64, n, k, 4, 64, f32) < _dense(n, k, 4)
    for m in (65, 256, 2048):
        assert lib.llmopt_q_linear_workspace_ex(m, n, k, 4, 64, f32) >= _dense(n, k, 4)
    # A small weight with a long batch: the pieces' workspace (3 M K bf16 pieces ...) is larger.
    assert lib.llmopt_q_linear_workspace_ex(4096, 256, 4096, 4, 64, f32) > _dense(256, 4096, 4)


def test_wide_grids_at_33_to_64_tokens_keep_the_gemm_for_other_formats(lib):
    # 33-64 tokens over >= 1024 tiles (N >= 16384) with K < 8192 leave the split-K GEMM only
    # for the N-split decode kernel, which takes 2/4-bit codes in groups of a multiple of 128;
    # 8-bit codes and groups of 32 or 64 stay on the GEMM and its K split.
    n, k = 16384, 4096
    for m in (33, 48, 64):
        assert _ws(lib, m, (n, k)) == 0, m
        for bits, group in ((8, 128), (4, 32), (4, 64)):
            ws = _ws(lib, m, (n, k), bits=bits, group=group)
            assert ws > 0 and ws % (m * n * 4) == 0, (m, bits, group, ws)


def test_swiglu_workspace_names_the_decode_k_split(lib):
    # Where the fused SwiGLU product runs on the K-sliced decode kernel with several slices,
    # the query returns its partial sums, so a caller sizing by it gets that kernel.
    ws = lib.llmopt_q_linear_swiglu_workspace
    assert ws(16, 8192, 8192, 4, 128) == 4 * 16 * 8192 * 4
    assert ws(48, 8192, 4096, 4, 128) == 2 * 48 * 8192 * 4
    assert ws(48, 8192, 4096, 4, 128) == _ws(lib, 48, (8192, 4096))
    # Resident-activation and N-split shapes keep all of K.
    assert ws(16, 28672, 4096, 4, 128) == 0
    assert ws(64, 28672, 4096, 4, 128) == 0

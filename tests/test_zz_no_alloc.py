"""llmopt_q_linear_noalloc (the entry point that allocates nothing) against llmopt_q_linear.

Both run the same plan and kernels; the allocation-free one takes its K-split partial sums
from the library's static device scratch instead of a workspace, so its output must equal
llmopt_q_linear's bit for bit. Two calls in a row, the second with a smaller input, check that
the scratch left by a larger call does not leak into a smaller one; shapes whose plan needs
more scratch than the static array holds are refused before anything is launched.
"""

from __future__ import annotations

import pytest
import torch

from llmopt.kernels import _lib
from llmopt.quantization import RoundToNearestQuantizer

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _weight(n, k, seed):
    w = torch.randn(n, k, generator=torch.Generator().manual_seed(seed)) * 0.02
    qt = RoundToNearestQuantizer(4, 128, False).quantize(w)
    return qt.qweight.to(DEV), qt.scales.to(DEV), qt.zeros.to(DEV)


def _args(x, qw, sc, zr, y, n, k, m):
    return (x.data_ptr(), m, k, k, qw.data_ptr(), k // 2, sc.data_ptr(), zr.data_ptr(), None, y.data_ptr(), n, n,
            _lib.DTYPE_CODES[torch.bfloat16], 4, 128, 0, 0)


def _pair(lib, n, k, m, seed):
    qw, sc, zr = _weight(n, k, seed)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(seed + 1)).to(torch.bfloat16).to(DEV)
    stream = torch.cuda.current_stream().cuda_stream
    need = lib.llmopt_q_linear_workspace(m, n, k, 4, 128)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
    want = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    rc = lib.llmopt_q_linear(*_args(x, qw, sc, zr, want, n, k, m), ws.data_ptr() if need else None, need, stream)
    assert rc == 0, lib.llmopt_q_last_error()
    got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    rc = lib.llmopt_q_linear_noalloc(*_args(x, qw, sc, zr, got, n, k, m), stream)
    assert rc == 0, lib.llmopt_q_last_error()
    torch.cuda.synchronize()
    return need, got, want


@pytest.mark.parametrize("first,second", [
    ((4096, 14336, 256), (4096, 14336, 32)),  # split-K GEMM, then the decode K slices
    ((6144, 4096, 64), (4096, 4096, 48)),     # split-K GEMM twice, the second smaller
    ((28672, 4096, 8), (4096, 14336, 16)),    # no scratch, then the decode K slices
])
def test_noalloc_equals_the_workspace_entry_point(first, second):
    lib = _lib.load_library()
    for (n, k, m), seed in ((first, 1), (second, 2)):
        need, got, want = _pair(lib, n, k, m, seed)
        assert need <= lib.llmopt_q_linear_noalloc_max_scratch()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (n, k, m)


def test_noalloc_refuses_plans_beyond_its_scratch():
    lib = _lib.load_library()
    cap = lib.llmopt_q_linear_noalloc_max_scratch()
    assert cap == 32 << 20
    # The Llama-3-8B projections' split plans all fit (at most 32 MiB); a 768-token batch
    # over 6144 x 8192 splits into 54 MiB of partial sums.
    n, k, m = 6144, 8192, 768
    assert lib.llmopt_q_linear_workspace(m, n, k, 4, 128) > cap
    qw, sc, zr = _weight(n, k, 3)
    # A non-zero input and a NaN-filled output: any kernel that ran would overwrite the NaNs.
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    rc = lib.llmopt_q_linear_noalloc(*_args(x, qw, sc, zr, y, n, k, m), torch.cuda.current_stream().cuda_stream)
    assert rc == -4 and b"static scratch" in lib.llmopt_q_last_error()
    torch.cuda.synchronize()
    assert bool(torch.isnan(y).all())  # nothing was launched


def test_noalloc_long_batches_run_the_fused_gemm():
    # From 1024 tokens llmopt_q_linear dequantizes into its workspace and calls hipBLASLt; the
    # dense weight does not fit the static scratch, so the allocation-free entry point runs the
    # fused GEMM instead: llmopt_q_linear_ex with LLMOPT_ALGO_PREFILL, bit for bit.
    lib = _lib.load_library()
    n, k, m = 4096, 4096, 1024
    qw, sc, zr = _weight(n, k, 5)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(DEV)
    stream = torch.cuda.current_stream().cuda_stream
    need = lib.llmopt_q_linear_workspace(m, n, k, 4, 128)
    assert need > lib.llmopt_q_linear_noalloc_max_scratch()
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    want = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    rc = lib.llmopt_q_linear_ex(*_args(x, qw, sc, zr, want, n, k, m), ws.data_ptr(), need, stream, _lib.ALGO_PREFILL)
    assert rc == 0, lib.llmopt_q_last_error()
    got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    rc = lib.llmopt_q_linear_noalloc(*_args(x, qw, sc, zr, got, n, k, m), stream)
    assert rc == 0, lib.llmopt_q_last_error()
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))

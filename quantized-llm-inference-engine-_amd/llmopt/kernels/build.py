"""Build ``libllmopt_qlinear.so`` from ``csrc/*.hip`` with hipcc for gfx950.

Usage: ``python -m llmopt.kernels.build`` (or :func:`build_library`). Objects go to
``<package>/_build/``; the library is written next to this file so it ships with the
source tree. The library's run path lists torch's bundled ROCm libraries first, so the
process uses one HIP runtime whichever of torch and this library is loaded first.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PACKAGE_ROOT = HERE.parent.parent  # quantized-llm-inference-engine-_amd/
CSRC = PACKAGE_ROOT / "csrc"
INCLUDE = PACKAGE_ROOT.parent / "include"
BUILD_DIR = PACKAGE_ROOT / "_build"
LIBRARY = HERE / "libllmopt_qlinear.so"
ARCH = os.environ.get("LLMOPT_OFFLOAD_ARCH", "gfx950")

COMPILE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # The dequantization must round exactly like the reference's torch code: no
    # contraction of (q - z) * s into an fma, and fp32 denormals kept.
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    # Packed fp32 arithmetic stays off on this target.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build the kernels")
    return found


def _torch_lib_dir() -> str | None:
    try:
        import torch
    except ImportError:  # pragma: no cover - torch is a hard dependency of the package
        return None
    return str(Path(torch.__file__).resolve().parent / "lib")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every ``csrc/*.hip`` and link the shared library. Always rebuilds."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")

    def compile_one(src: Path) -> Path:
        obj = BUILD_DIR / (src.stem + ".o")
        cmd = [hipcc, *COMPILE_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stdout}\n{proc.stderr}")
        return obj

    workers = jobs or min(len(srcs), 8)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(compile_one, srcs))

    tmp = LIBRARY.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    torch_lib = _torch_lib_dir()
    if torch_lib:
        link.append(f"-Wl,-rpath,{torch_lib}")
    # hipBLASLt for the two-pass prefill's dense GEMM.
    link += ["-L/opt/rocm/lib", "-lhipblaslt"]
    if verbose:
        print(" ".join(link), flush=True)
    proc = subprocess.run(link, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


def main() -> int:
    path = build_library(verbose="-v" in sys.argv)
    print(path)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

"""ctypes binding of ``libllmopt_qlinear.so`` (C ABI in ``include/llmopt_qlinear.h``).

The library is loaded after ``torch`` so that both share torch's HIP runtime (the
library's own run path points at the same copy). A missing library raises: the HIP
path has no host substitute.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

__all__ = [
    "ALGO_AUTO",
    "ALGO_DECODE",
    "ALGO_GENERIC",
    "ALGO_PREFILL",
    "ALGO_DENSE",
    "DTYPE_CODES",
    "EXPORTED_SYMBOLS",
    "call",
    "library_path",
    "load_library",
]

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

ALGO_AUTO = 0
ALGO_GENERIC = 1
ALGO_DECODE = 2
ALGO_PREFILL = 3
ALGO_DENSE = 4

ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_size = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/llmopt_qlinear.h.
_SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "llmopt_q_abi_version": (_int, []),
    "llmopt_q_last_error": (ctypes.c_char_p, []),
    "llmopt_q_unpack": (_int, [_p, _p, _i64, _i64, _i64, _p]),
    "llmopt_q_dequant": (
        _int,
        [_p, _i64, _p, _p, _p, _int, _i64, _i64, _int, _int, _int, _int, _p],
    ),
    "llmopt_q_quantize_rtn": (
        _int,
        [_p, _int, _i64, _i64, _i64, _int, _int, _int, _p, _i64, _p, _p, _p],
    ),
    "llmopt_q_linear_workspace": (_size, [_i64, _i64, _i64, _int, _int]),
    "llmopt_kv_write_decode": (
        _int,
        [_p, _p, _int, _i64, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _int, _i64, _i64, _p],
    ),
    "llmopt_kv_write": (
        _int,
        [_p, _p, _int, _i64, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _int, _i64, _i64, _i64, _i64, _p],
    ),
    "llmopt_paged_attention_workspace": (_size, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "llmopt_rmsnorm": (
        _int,
        [_p, _i64, _p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, ctypes.c_float, _int, _p],
    ),
    "llmopt_rmsnorm_planes": (
        _int,
        [_p, _i64, _p, _p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, ctypes.c_float, _int, _p],
    ),
    "llmopt_rope": (
        _int,
        [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _int, _p],
    ),
    "llmopt_rope_kv_write_decode": (
        _int,
        [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _int, _p, _p, _i64, _i64,
         _p, _i64, _p, _p],
    ),
    "llmopt_paged_attention_decode": (
        _int,
        [_p, _int, _i64, _p, _p, _int, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64,
         ctypes.c_float, ctypes.c_float, _p, _p, _size, _p],
    ),
    "llmopt_argmax_rows": (_int, [_p, _int, _i64, _i64, _i64, _p, _p]),
    "llmopt_paged_attention_prefill": (
        _int,
        [_p, _int, _i64, _i64, _i64, _p, _p, _int, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64,
         ctypes.c_float, ctypes.c_float, _p, _i64, _i64, _i64, _p],
    ),
    "llmopt_paged_attention_decode_rope": (
        _int,
        [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _i64, _int, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _p, _p,
         _i64, _i64, ctypes.c_float, ctypes.c_float, _p, _p, _size, _p],
    ),
    "llmopt_q_linear_swiglu_workspace": (_size, [_i64, _i64, _i64, _int, _int]),
    "llmopt_q_linear_swiglu_workspace_ex": (_size, [_i64, _i64, _i64, _int, _int, _int]),
    "llmopt_q_linear_workspace_ex": (_size, [_i64, _i64, _i64, _int, _int, _int]),
    "llmopt_q_linear_dense_workspace": (_size, [_i64, _i64, _int]),
    "llmopt_q_linear_swiglu": (
        _int,
        [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64, _int, _int, _int, _int, _int,
         _p, _size, _p],
    ),
    "llmopt_q_linear": (
        _int,
        [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64, _int, _int, _int, _int, _int,
         _p, _size, _p],
    ),
    "llmopt_q_linear_deferred": (
        _int,
        [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64, _int, _int, _int, _int, _int,
         _p, _size, _p, ctypes.POINTER(ctypes.c_int)],
    ),
    "llmopt_q_linear_noalloc": (
        _int,
        [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64, _int, _int, _int, _int, _int, _p],
    ),
    "llmopt_q_linear_noalloc_max_scratch": (_size, []),
    "llmopt_q_linear_ex": (
        _int,
        [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64, _int, _int, _int, _int, _int,
         _p, _size, _p, _int],
    ),
}
EXPORTED_SYMBOLS = tuple(_SIGNATURES)
ABI_VERSION = 1

_lock = threading.Lock()
_handle: ctypes.CDLL | None = None


def library_path() -> Path:
    override = os.environ.get("LLMOPT_QLINEAR_LIB")
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / "libllmopt_qlinear.so"


def load_library() -> ctypes.CDLL:
    """Load (once) and return the kernel library; raise if it has not been built."""
    global _handle
    if _handle is not None:
        return _handle
    with _lock:
        if _handle is None:
            path = library_path()
            if not path.exists():
                raise RuntimeError(
                    f"llmopt HIP kernel library not found at {path}; build it with "
                    "`python -m llmopt.kernels.build` (hipcc, gfx950)"
                )
            lib = ctypes.CDLL(str(path))
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            version = lib.llmopt_q_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
            _handle = lib
    return _handle


def call(rc: int, what: str) -> None:
    """Raise the Python exception matching a negative status code."""
    if rc == 0:
        return
    message = load_library().llmopt_q_last_error().decode(errors="replace")
    if rc == ERR_INVALID_ARG:
        raise ValueError(f"{what}: {message}")
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {message}")
    raise RuntimeError(f"{what}: {message}")

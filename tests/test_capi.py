"""The C ABI library: it loads, exports every entry point of include/*.h, and validates
arguments on the host before anything reaches a device. No kernel is launched here."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch  # noqa: F401 - load torch's HIP runtime before the library

from llmopt.kernels import _lib

HEADER_DIR = Path(__file__).resolve().parent.parent / "include"


def _declared_functions() -> set[str]:
    names = set()
    for header in HEADER_DIR.glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(llmopt_\w+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().exists():
        pytest.fail(f"kernel library not built: {_lib.library_path()} (run __graft_entry__.build())")
    return _lib.load_library()


def test_every_declared_symbol_is_exported(lib):
    declared = _declared_functions()
    assert declared == set(_lib.EXPORTED_SYMBOLS)
    dynsym = subprocess.run(
        ["nm", "-D", "--defined-only", str(_lib.library_path())], capture_output=True, text=True, check=True
    ).stdout
    exported = set(re.findall(r"\bT (llmopt_\w+)$", dynsym, flags=re.M))
    assert declared <= exported
    for name in declared:
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_metadata_calls(lib):
    assert lib.llmopt_q_abi_version() == 1
    assert lib.llmopt_q_linear_workspace(1, 4096, 4096, 4, 128) == 0
    assert isinstance(lib.llmopt_q_last_error(), bytes)


def test_host_side_validation_reports_errors(lib):
    # Bad bit width: rejected before any device work.
    rc = lib.llmopt_q_dequant(None, 8, None, None, None, 2, 4, 16, 9, 16, 1, 0, None)
    assert rc == -1 and b"bit width" in lib.llmopt_q_last_error()
    # Group that does not divide K.
    rc = lib.llmopt_q_dequant(None, 8, None, None, None, 2, 4, 16, 4, 6, 1, 0, None)
    assert rc == -1 and b"not divisible" in lib.llmopt_q_last_error()
    # Packed row too short for K.
    rc = lib.llmopt_q_linear(None, 1, 64, 64, None, 16, None, None, None, None, 8, 8, 2, 4, 32, 1, 0, None, 0, None)
    assert rc == -1 and b"cannot hold" in lib.llmopt_q_last_error()
    # Asymmetric grid without zeros.
    rc = lib.llmopt_q_linear(1, 1, 64, 64, 1, 32, 1, None, None, 1, 8, 8, 2, 4, 32, 0, 0, None, 0, None)
    assert rc == -1 and b"zeros" in lib.llmopt_q_last_error()
    # Unknown dtype and algorithm codes.
    assert lib.llmopt_q_linear(1, 1, 64, 64, 1, 32, 1, 1, None, 1, 8, 8, 7, 4, 32, 0, 0, None, 0, None) == -1
    assert lib.llmopt_q_linear_ex(1, 1, 64, 64, 1, 32, 1, 1, None, 1, 8, 8, 2, 4, 32, 0, 0, None, 0, None, 9) == -1
    # Unpack asked for more columns than the bytes hold.
    assert lib.llmopt_q_unpack(None, None, 2, 4, 9, None) == -1
    # Quantizer: bad width, group not dividing K, odd group under nibble packing, short rows.
    q = lib.llmopt_q_quantize_rtn
    assert q(1, 2, 64, 4, 64, 3, 32, 0, 1, 32, 1, 1, None) == -1
    assert b"bit width" in lib.llmopt_q_last_error()
    assert q(1, 2, 64, 4, 64, 4, 48, 0, 1, 32, 1, 1, None) == -1
    assert b"not divisible" in lib.llmopt_q_last_error()
    assert q(1, 2, 66, 4, 66, 4, 33, 0, 1, 33, 1, 1, None) == -1
    assert b"even number of columns" in lib.llmopt_q_last_error()
    assert q(1, 2, 64, 4, 64, 8, 32, 0, 1, 32, 1, 1, None) == -1
    assert b"cannot hold" in lib.llmopt_q_last_error()
    assert q(1, 5, 64, 4, 64, 4, 32, 0, 1, 32, 1, 1, None) == -1  # dtype code
    assert q(None, 2, 64, 0, 64, 4, 32, 0, None, 32, None, None, None) == 0  # no rows: no-op
    # Empty batches are a no-op that succeeds without touching the device.
    assert lib.llmopt_q_linear(None, 0, 64, 64, 1, 32, 1, 1, None, None, 8, 8, 2, 4, 32, 0, 0, None, 0, None) == 0


def test_python_wrapper_maps_status_codes(lib):
    with pytest.raises(ValueError):
        _lib.call(-1, "x")
    with pytest.raises(NotImplementedError):
        _lib.call(-2, "x")
    with pytest.raises(RuntimeError):
        _lib.call(-3, "x")
    _lib.call(0, "x")

"""Register-allocation guard for the hot kernels (host-only: compiles to gfx950 assembly).

A change to a kernel's epilogue once raised register pressure enough that the prefill GEMM
spilled inside its main loop, an 18x slowdown that no parity test notices. This test compiles
the GEMM and decode sources with the library's own flags and checks that no instantiation
touches scratch memory between its main loop's header and back edge.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from llmopt.kernels import build

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _kernels(asm: str) -> dict[str, list[str]]:
    """Function name -> its lines, for every kernel symbol in an assembly file."""
    out: dict[str, list[str]] = {}
    name = None
    for line in asm.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            name = m.group(1)
            out[name] = []
        elif name is not None:
            out[name].append(line)
            if "s_endpgm" in line:
                name = None
    return out


def _scratch_in_loops(lines: list[str]) -> int:
    """Scratch accesses inside any loop: from a loop header label to its last back edge."""
    labels = {}
    for i, line in enumerate(lines):
        m = re.match(r"^(\.LBB\S+):.*Loop Header", line)
        if m:
            labels[m.group(1)] = i
    count = 0
    for label, start in labels.items():
        ends = [i for i, line in enumerate(lines) if re.search(r"s_(c)?branch\S*\s+" + re.escape(label) + r"\b", line)]
        if ends:
            count += sum("scratch_" in line for line in lines[start : max(ends) + 1])
    return count


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
@pytest.mark.parametrize("source", ["qlinear_gemm.hip", "qlinear_decode.hip"])
def test_no_spills_in_main_loops(tmp_path, source):
    src = build.CSRC / source
    out = tmp_path / (source + ".s")
    flags = [f for f in build.COMPILE_FLAGS if f not in ("-fPIC",)]
    cmd = [HIPCC, *flags, f"-I{build.INCLUDE}", f"-I{build.CSRC}", "--cuda-device-only", "-S", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    kernels = _kernels(out.read_text())
    hot = {k: v for k, v in kernels.items() if "gemm_kernel" in k or "decode_" in k}
    assert hot, "no kernels found in the assembly"
    bad = {k: n for k, v in hot.items() if (n := _scratch_in_loops(v))}
    assert not bad, f"scratch accesses inside main loops: {bad}"

"""The RTN quantizer kernel computes rne(w / s) without a division, by Markstein's correction
(csrc/quantize_rtn.hip, rint_quotients). This checks that identity exhaustively on the CPU over
the cases where it could change a code (tests/quotient_exactness.c states the argument), so the
kernel's bit-exactness with the reference's correctly rounded `w / s` (quantizers.py:167-201)
does not rest on the GPU tests' random weights alone."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "quotient_exactness.c")


def _build(tmp_path, flags):
    exe = str(tmp_path / "quotient_exactness")
    cmd = ["gcc", "-O3", "-ffp-contract=off", "-fno-fast-math", *flags, SRC, "-o", exe, "-lm"]
    ok = subprocess.run(cmd, capture_output=True, text=True).returncode == 0
    return exe if ok else None


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_quotient_matches_division(tmp_path):
    # Hardware fma (x86 FMA3) and OpenMP make the full sweep (1.9e10 cases) take seconds;
    # without them the software fmaf is correct but slow, so every 64th significand is taken.
    exe = _build(tmp_path, ["-mfma", "-fopenmp"])
    stride = "1"
    if exe is None:
        exe = _build(tmp_path, [])
        stride = "64"
    assert exe is not None, "quotient_exactness.c does not compile"
    env = dict(os.environ, OMP_NUM_THREADS=str(min(os.cpu_count() or 1, 16)))
    res = subprocess.run([exe, stride], capture_output=True, text=True, timeout=600, env=env)
    assert res.returncode == 0, res.stdout + res.stderr
    fields = res.stdout.split()
    assert fields[0] == "cases" and int(fields[1]) > 0
    assert fields[2:] == ["wrong", "0", "wrong_rint", "0"], res.stdout

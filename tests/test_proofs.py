"""Arithmetic facts the device kernels rely on, checked on the CPU."""

from __future__ import annotations

import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_markstein_quotient_is_the_correctly_rounded_division(tmp_path):
    """rotate_quant divides by the per-row scale with q0 = a*inv, r = fma(-q0, d, a), q1 = fma(r, inv, q0): exact
    RN(a / d) for every bf16-precision a and fp32 d (proof program tests/proofs/markstein_quotient.c; the full run
    checks all 2^23 divisor significands, this test every 64th)."""
    exe = tmp_path / "markstein"
    src = os.path.join(HERE, "proofs", "markstein_quotient.c")
    build = subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-fopenmp", src, "-o", str(exe), "-lm"],
                           capture_output=True, text=True)
    if build.returncode != 0:
        pytest.fail(build.stderr)
    run = subprocess.run([str(exe), "64"], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "0 differ from RN(a/d), 0 round to a different integer" in run.stdout

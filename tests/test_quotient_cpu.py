"""The quantizers' division shortcut is the IEEE quotient on their whole input domain.

quant.hip computes the spec's correctly rounded t = RN((x - z) / s) as RN(d r) plus one
fma remainder and one fma correction, with r = RN(1 / s) (Markstein's theorem; its
exceptions need a 24-ones divisor significand, and s is an fp16 value). The C program
tests/cpu_checks/quotient_check.c compares that sequence with IEEE division bit for bit
for every finite fp16 s (about 4 million cases); the planted variant without the
correction must fail, which shows the check can see a difference. The GPU kernels
themselves are held to the numpy spec bit for bit by tests/test_quant_gpu.py.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cpu_checks", "quotient_check.c")


def _clang():
    for c in ("/opt/rocm/llvm/bin/clang", shutil.which("clang")):
        if c and os.path.exists(c):
            return c
    return None


@pytest.fixture(scope="module")
def binary(tmp_path_factory):
    cc = _clang()
    if cc is None:
        pytest.skip("no clang with __fp16 support")
    out = str(tmp_path_factory.mktemp("quotient") / "quotient_check")
    subprocess.run([cc, "-O2", "-ffp-contract=off", SRC, "-o", out, "-lm"], check=True)
    return out


def test_fma_quotient_equals_ieee_division(binary):
    r = subprocess.run([binary], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout


def test_check_detects_a_missing_correction(binary):
    r = subprocess.run([binary, "plain"], capture_output=True, text=True, timeout=300)
    assert r.returncode != 0, "the check must see RN(d r) differ from RN(d / s)"

"""The FDM's short-latency fp64 math (csrc/fdm_math.h) against 80-bit references, on the host.

fm_div / fm_rcp / fm_sqrt start from the hardware reciprocal and reciprocal square root; the
check replaces those with values off by the hardware's worst measured relative error (4.5e-8,
both signs) so the Newton/Goldschmidt refinements are exercised from a start at least as bad as
the device's.  fm_exp / fm_log are series forms; their bounds are the ulp errors of the method
(truncation < 5e-17 relative plus a few roundings).  The per-step FDM parity against the CPU
restatement (<= 1e-10 relative, tests/test_fdm_gpu.py) is the end-to-end check of the same code
on the GPU."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "2026_ai_pilot_challenge-1st_solution_amd", "csrc")


@pytest.fixture(scope="module")
def result(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("fdm_math")
    os.makedirs(d / "hip")
    (d / "hip" / "hip_runtime.h").write_text("")   # the header's only include; nothing used
    exe = d / "check"
    subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", "-I", str(d), "-I", CSRC,
                    "-o", str(exe), os.path.join(HERE, "fdm_math_check.cpp")], check=True)
    out = subprocess.run([str(exe), "400000"], check=True, capture_output=True, text=True).stdout
    toks = out.split()
    return {toks[i]: float(toks[i + 1]) for i in range(0, len(toks), 2)}


def test_division_and_reciprocal_correctly_rounded(result):
    assert result["div"] <= 0.5 + 1e-9
    assert result["rcp"] <= 0.5 + 1e-9
    assert result["div_ne_ieee"] == 0        # every quotient equals IEEE division's


def test_sqrt_correctly_rounded(result):
    assert result["sqrt"] <= 0.5 + 1e-9


def test_exp_log_within_three_ulp(result):
    assert result["exp"] <= 3.0
    assert result["log"] <= 3.0


def test_special_operands_follow_ieee(result):
    assert result["special_bad"] == 0

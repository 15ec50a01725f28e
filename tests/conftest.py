import importlib
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = "2026_ai_pilot_challenge-1st_solution_amd"
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


def import_pkg(sub=None):
    return importlib.import_module(PKG + ("." + sub if sub else ""))


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def pkg():
    return import_pkg()


@pytest.fixture(scope="session")
def orc():
    import oracle_lib
    return oracle_lib.load()


@pytest.fixture(scope="session")
def gpu():
    if not gpu_available():
        pytest.fail("GPU test collected on a host without a HIP device")
    import torch
    return torch.device("cuda")


# Measured worst errors of the parity tests, printed beside their bounds at the end of the run.
_WORST = []


@pytest.fixture(scope="session")
def worst():
    """worst(name, value, bound): record a test's measured worst error against its bound."""
    def rec(name, value, bound):
        _WORST.append((name, float(value), float(bound)))
    return rec


def pytest_terminal_summary(terminalreporter):
    if not _WORST:
        return
    terminalreporter.section("measured worst errors (value / bound)")
    best = {}
    for name, v, b in _WORST:
        if name not in best or v > best[name][0]:
            best[name] = (v, b)
    for name, (v, b) in best.items():
        terminalreporter.write_line(f"{name}: {v:.3e} / {b:.1e}")

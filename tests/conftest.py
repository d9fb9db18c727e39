"""Shared test configuration.

Markers: ``gpu`` tests need an MI355X and call libpkx.so through its C ABI;
everything else runs on the CPU (the oracle against its pins, host logic, the
library's exported symbols).  No test module imports torch at module level:
the GPU process must load exactly one HIP runtime (libpkx.so's).
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "parakeet.cpp_amd", "python"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libpkx.so")


def rel_l2(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


@pytest.fixture(scope="session")
def gpu():
    """The pkx binding with a live device and one stream for the session."""
    import pkx
    n = pkx.device_count()
    if n < 1:
        pytest.skip("no GPU visible")
    return pkx


@pytest.fixture(scope="session")
def stream(gpu):
    return gpu.Stream()

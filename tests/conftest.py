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


def tie_excluded(ref_logits, rel=1e-6):
    """Frames whose reference top-2 logits are an exact f32 tie up to rel*|max|:
    the only frames on the f32 path where the first-max argmax
    (src/decode_common.hpp:5-9, src/search.cpp:57-61) may legitimately differ."""
    top2 = np.sort(np.asarray(ref_logits, dtype=np.float64), axis=-1)[..., -2:]
    return (top2[..., 1] - top2[..., 0]) <= rel * np.maximum(np.abs(top2[..., 1]), 1e-30)


def argmax_identical(got_ids, ref_ids, ref_logits, label, rel=1e-6):
    """Asserts ids are identical on every frame except exact f32 ties; prints the
    number of excluded frames.  Returns that number."""
    ex = tie_excluded(ref_logits, rel)
    got_ids, ref_ids = np.asarray(got_ids), np.asarray(ref_ids)
    bad = (got_ids != ref_ids) & ~ex
    print(f"  [{label}] argmax: {int(ex.sum())} of {ex.size} frames excluded as f32 ties, "
          f"{int((got_ids != ref_ids).sum())} differ", flush=True)
    assert not bad.any(), (label, np.flatnonzero(bad)[:10])
    return int(ex.sum())


def argmax_within_error(got_ids, ref_ids, ref_logits, got_logits, label, max_frac=0.01):
    """Reduced-precision (F16 mode) argmax bar: a frame may differ only where the
    reference's top-2 margin is within twice the measured logit error of that
    frame, and such frames are at most max_frac of all.  Returns (excusable, differ)."""
    ref_logits = np.asarray(ref_logits, dtype=np.float64)
    err = np.abs(np.asarray(got_logits, dtype=np.float64) - ref_logits).max(axis=-1)
    top2 = np.sort(ref_logits, axis=-1)[..., -2:]
    excusable = (top2[..., 1] - top2[..., 0]) <= 2.0 * err
    differ = np.asarray(got_ids) != np.asarray(ref_ids)
    print(f"  [{label}] argmax: {int(differ.sum())} of {differ.size} frames differ, "
          f"{int(excusable.sum())} within twice the logit error "
          f"(max logit error {float(err.max()):.2e})", flush=True)
    assert not (differ & ~excusable).any(), (label, np.flatnonzero(differ & ~excusable)[:10])
    assert excusable.mean() <= max_frac, (label, float(excusable.mean()))
    return int(excusable.sum()), int(differ.sum())

"""Pins of the oracle's quantisers (ggml's quantize_row_q8_0_ref and
quantize_row_q4_K_ref, the algorithms parakeet-cli quantize runs through
ggml_quantize_chunk, examples/cli/main.cpp:322-426).

q8_0 is pinned by its closed form: d = f16(amax / 127), q = roundf(x / d)
with ties away from zero (C roundf), computed with 1/d in f32.  q4_K has no
closed form (a weighted least-squares search per 32-value sub-block); it is
pinned by properties a plausible slip breaks: the round-trip error bound, the
search never doing worse than its own min/max starting point, constant blocks
and the 6-bit code range.  No ggml test vector exists here (ggml is absent):
byte parity of the q4_K quantiser with ggml is unpinned.
"""
import numpy as np
import pytest

import oracle

Q8, Q4K = 8, 12


def quant(gtype, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    nb = oracle.lib().orc_row_bytes(gtype, x.size)
    out = np.zeros(nb, np.uint8)
    assert oracle.lib().orc_quantize(gtype, oracle.fp(x), out.ctypes.data, x.size) == 0
    return out


def dequant(gtype, raw, n):
    out = np.zeros(n, np.float32)
    assert oracle.lib().orc_dequantize(gtype, raw.ctypes.data, oracle.fp(out), n) == 0
    return out


def c_roundf(v):
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def test_q8_0_closed_form():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(32 * 64).astype(np.float32)
    x[:32] = 0.0                                              # an all-zero block: d = 0, q = 0
    raw = quant(Q8, x).reshape(-1, 34)
    for b in range(64):
        v = x[32 * b:32 * b + 32]
        amax = np.float32(np.max(np.abs(v)))
        d = np.float32(amax / np.float32(127))
        idv = np.float32(1) / d if d != 0 else np.float32(0)
        assert raw[b, :2].view(np.uint16)[0] == np.float16(d).view(np.uint16)
        q = c_roundf((v * idv).astype(np.float32)).astype(np.int8)
        assert np.array_equal(raw[b, 2:].view(np.int8), q)


def test_q8_0_ties_round_away_from_zero():
    v = np.zeros(32, np.float32)
    v[0], v[1], v[2], v[3] = 127.0, 2.5, -2.5, 0.5            # d = 1: x * (1/d) = x exactly
    raw = quant(Q8, v)
    q = raw[2:].view(np.int8)
    assert (q[0], q[1], q[2], q[3]) == (127, 3, -3, 1)


def test_q4_k_roundtrip_bound_and_codes():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(256 * 32) * 0.02).astype(np.float32)
    raw = quant(Q4K, x)
    y = dequant(Q4K, raw, x.size)
    blk = raw.reshape(-1, 144)
    for b in range(32):
        xs = x[256 * b:256 * b + 256].reshape(8, 32)
        err = np.abs(y[256 * b:256 * b + 256].reshape(8, 32) - xs)
        # the 4-bit grid spans each sub-block's range in 15 steps; allow the
        # 6-bit scale / min coding on top
        span = xs.max(1) - np.minimum(xs.min(1), 0)
        assert np.all(err.max(1) <= span / 15 * 1.5 + 1e-7)


def test_q4_k_search_beats_its_starting_point():
    """make_qkx2_quants starts from the min/max grid and only accepts better
    weighted fits, so the final sub-block error cannot exceed the plain
    min/max 4-bit quantisation of the same block (up to the 6-bit / f16 coding
    of the scales, which is applied to both)."""
    rng = np.random.default_rng(2)
    worse = 0
    for b in range(64):
        x = (rng.standard_normal(256) * rng.uniform(0.005, 0.05)).astype(np.float32)
        y = dequant(Q4K, quant(Q4K, x), 256)
        naive = np.empty(256, np.float32)
        for j in range(8):
            v = x[32 * j:32 * j + 32]
            mn = min(v.min(), 0.0)
            sc = (v.max() - mn) / 15
            naive[32 * j:32 * j + 32] = np.clip(np.rint((v - mn) / sc), 0, 15) * sc + mn
        worse += np.sum((y - x) ** 2) > 1.5 * np.sum((naive - x) ** 2)
    assert worse == 0


def test_q4_k_constant_and_zero_blocks():
    for val in (0.0, 0.25, -0.25):
        x = np.full(256, val, np.float32)
        y = dequant(Q4K, quant(Q4K, x), 256)
        assert np.max(np.abs(y - x)) <= abs(val) / 15 * 1.5 + 1e-7


def test_pin_detects_planted_q8_mistake():
    """Rounding ties to even (numpy's rint) instead of C roundf must fail the pin."""
    v = np.zeros(32, np.float32)
    v[0], v[1] = 127.0, 2.5
    q = quant(Q8, v)[2:].view(np.int8)
    assert q[1] != np.rint(2.5)

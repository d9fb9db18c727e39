"""Pins of the oracle's quantisers (ggml's quantize_row_q8_0_ref and
quantize_row_q4_K_ref, the algorithms parakeet-cli quantize runs through
ggml_quantize_chunk, examples/cli/main.cpp:322-426).

q8_0 is pinned by its closed form: d = f16(amax / 127), q = roundf(x / d)
with ties away from zero (C roundf), computed with 1/d in f32.

q4_K has no closed form in general (a weighted least-squares search per
32-value sub-block), so it is pinned two ways.  Known-answer super-blocks whose
bytes follow by hand from the mathematics of the search: sub-blocks already on
an exactly representable 4-bit affine grid (the min/max start fits exactly, so
no candidate can replace it), a sub-block whose every candidate fit has a
positive intercept (the clamp to min = 0 and the through-origin refit decide
the scale), and constant blocks (every candidate has a zero determinant).  And
properties a plausible slip breaks on random data: the round-trip error bound
and the search never doing worse than its own min/max starting point.  No ggml
test vector exists here (ggml is absent); on random data, byte parity with
ggml rests on those properties and on the restatement following ggml's
published steps.
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


def _q4k_fields(raw):
    blk = raw.reshape(144)
    return blk[0:2].view(np.uint16)[0], blk[2:4].view(np.uint16)[0], list(blk[4:16]), blk[16:]


def _q4k_nibbles(L):
    """ggml's q4_K code layout: byte 32*g + i holds sub-block 2g's code i in
    the low nibble and sub-block 2g+1's code i in the high nibble."""
    L = np.asarray(L, np.uint8).reshape(8, 32)
    return np.concatenate([L[2 * g] | (L[2 * g + 1] << 4) for g in range(4)])


# sub-block j of the exact-grid block: x = s_j * l - m_j with codes l covering
# 0..15, so min = -m_j and max - min = 15 * s_j, both exact in f32
GRID_S = [1 / 8, 1 / 4, 1 / 2, 1, 1 / 8, 1 / 4, 1 / 2, 1]
GRID_M = [0, 0.5, 1, 2, 1.5, 0.25, 0, 1]


def _grid_codes(j):
    return (7 * np.arange(32) + 3 * j) % 16                      # every code 0..15, twice


def _grid_block():
    return np.concatenate([np.float32(GRID_S[j]) * _grid_codes(j).astype(np.float32) - np.float32(GRID_M[j])
                           for j in range(8)]).astype(np.float32)


def test_q4_k_exact_grid_known_answer():
    """Hand derivation.  Per sub-block the start is iscale = 15 / (15 s_j) =
    1 / s_j exactly, so the codes are l and the weighted error is exactly 0;
    the search accepts only a strictly smaller error, so scale = s_j and
    min = m_j stay.  max scale = 1, max min = 2:
      d  = f16(1/63) = 0x2410,  dmin = f16(2/63) = 0x2810
      scale codes round(63 s_j)    = 8 16 32 63 8 16 32 63  (31.5 -> 32: ties to even)
      min codes   round(31.5 m_j)  = 0 16 32 63 47 8 0 32   (15.75, 31.5, 47.25, 7.875)
    packed by get_scale_min_k4's layout: bytes 0-3 hold the low six bits of
    scale codes 0-3 and the top two bits of scale codes 4-7, bytes 4-7 the
    same for the min codes, bytes 8-11 the low nibbles of codes 4-7 (scale low,
    min high).  The re-quantisation round((x + dmin*mc) / (d*sc)) stays within
    0.3 of l for every sub-block (the 6-bit scales are within 1.6% of s_j and
    the offsets within 0.07 of a step), so the codes are l."""
    raw = quant(Q4K, _grid_block())
    dh, mh, sc, q = _q4k_fields(raw)
    assert (dh, mh) == (0x2410, 0x2810)
    assert sc == [0x08, 0x50, 0xA0, 0xFF, 0x80, 0x10, 0x20, 0xBF, 0xF8, 0x80, 0x00, 0x0F]
    assert np.array_equal(q, _q4k_nibbles([_grid_codes(j) for j in range(8)]))


def test_q4_k_positive_intercept_clamp_known_answer():
    """Sub-block 0 holds 20 ones and 12 thirteens (weights av_x + |x| with
    av_x = sqrt((20 + 12*169) / 32) = 8: w = 9 and 21); sub-blocks 1-7 are the
    exact grid above (max scale 1, max min 2).  Hand derivation for sub-block 0:
    min is clamped to 0, the start (iscale 15/13) codes are (1, 15) with error
    180 (13/15 - 1)^2 = 3.2.  Candidates iscale (14 + 0.1 is) / 13 give codes
    (1, 14) for is <= 4 and (1, 15) for is >= 6.  Both two-point fits have a
    positive intercept (1/13 and 1/7), so both take the clamp: min = 0,
    scale = sum w x l / sum w l^2.  For (1, 14) that is 46044 / 49572 =
    0.928831 with error 0.915 (all sums exact integers in f32), for (1, 15)
    49320 / 56880 = 0.867089 with error 3.19; is = 0 is (1, 14) and nothing
    later beats it.  Scale code round(63 * 0.928831) = round(58.516) = 59 (the
    unclamped slope 12/13 would give 58); min code 0 (an unclamped intercept
    would give a negative min and code 63).  Re-quantisation with
    d = f16(1/63) * 59 = 0.93628: 1 -> 1.07 -> 1, 13 -> 13.88 -> 14."""
    x = _grid_block()
    sub0 = np.where(np.arange(32) % 8 < 5, 1.0, 13.0).astype(np.float32)
    x[:32] = sub0
    raw = quant(Q4K, x)
    dh, mh, sc, q = _q4k_fields(raw)
    assert (dh, mh) == (0x2410, 0x2810)
    assert sc == [0x3B, 0x50, 0xA0, 0xFF, 0x80, 0x10, 0x20, 0xBF, 0xF8, 0x80, 0x00, 0x0F]
    codes = [np.where(sub0 == 1.0, 1, 14)] + [_grid_codes(j) for j in range(1, 8)]
    assert np.array_equal(q, _q4k_nibbles(codes))


@pytest.mark.parametrize("val,dh,mh,sc,qbyte", [
    # max == min after the clamp of min to <= 0: codes 0, scale 0, min 0
    (0.0, 0x0000, 0x0000, [0] * 12, 0x00),
    # min clamps to 0, iscale = 15 / 0.25 = 60, codes 15; every candidate has
    # equal codes, so D = sum_w sum_l2 - sum_l^2 = 0 and none is fitted:
    # scale = f32(1/60), d = f16(f32(1/60) / 63) = 0x0C56, scale codes 63,
    # re-quantised codes round(0.25 / (63 d)) = round(14.995) = 15
    (0.25, 0x0C56, 0x0000, [0xFF] * 4 + [0x00] * 4 + [0x0F] * 4, 0xFF),
    # max == min = -0.25: codes 0, scale 0, min 0.25; dmin = f16(0.25/63) =
    # 0x1C10, min codes 63, d = 0 so no re-quantisation
    (-0.25, 0x0000, 0x1C10, [0x00] * 4 + [0xFF] * 4 + [0xF0] * 4, 0x00),
])
def test_q4_k_constant_blocks_known_answer(val, dh, mh, sc, qbyte):
    x = np.full(256, val, np.float32)
    raw = quant(Q4K, x)
    got = _q4k_fields(raw)
    assert (got[0], got[1], got[2]) == (dh, mh, sc)
    assert np.all(got[3] == qbyte)
    y = dequant(Q4K, raw, 256)
    assert np.max(np.abs(y - x)) <= abs(val) / 15 * 1.5 + 1e-7


def test_pin_detects_planted_q8_mistake():
    """Rounding ties to even (numpy's rint) instead of C roundf must fail the pin."""
    v = np.zeros(32, np.float32)
    v[0], v[1] = 127.0, 2.5
    q = quant(Q8, v)[2:].view(np.int8)
    assert q[1] != np.rint(2.5)

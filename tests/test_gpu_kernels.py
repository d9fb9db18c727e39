"""Kernel-level parity: HIP path (through the C ABI) vs the CPU oracle.

Bars: dequantisation bit-exact; f32 path within 1e-5 relative L2 of the
oracle's f32 arithmetic; f16 path (f16 operands, f32 accumulation) within
2e-3 relative L2 for a single GEMM.
"""
import numpy as np
import pytest

import oracle
import pk_model as pm
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _rng(seed=7):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("gtype,n", [(pm.GGML_Q8_0, 32 * 1000), (pm.GGML_Q4_K, 256 * 300),
                                     (pm.GGML_F16, 4096)])
def test_dequantize_bit_exact(gpu, stream, gtype, n):
    rng = _rng()
    if gtype == pm.GGML_Q8_0:
        raw = pm.synth_q8_0(rng, n)
    elif gtype == pm.GGML_Q4_K:
        raw = pm.synth_q4_k(rng, n)
    else:
        raw = rng.normal(0, 1, n).astype(np.float16).view(np.uint16)
    print(f"[dequant] type={gtype} n={n}", flush=True)
    ref = oracle.dequantize(gtype, raw, n)
    d_raw = gpu.DeviceArray.from_numpy(raw.view(np.uint8), stream)
    out = gpu.DeviceArray((n,), np.float32)
    gpu.dequantize(gtype, d_raw, n, out, stream)
    got = out.numpy(stream)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _weights(gtype, N, K, rng):
    if gtype == pm.GGML_F32:
        w = rng.normal(0, 0.05, (N, K)).astype(np.float32)
        return w, w
    if gtype == pm.GGML_F16:
        h = rng.normal(0, 0.05, (N, K)).astype(np.float16)
        return h.view(np.uint16), h.astype(np.float32)
    raw = pm.synth_q8_0(rng, N * K) if gtype == pm.GGML_Q8_0 else pm.synth_q4_k(rng, N * K)
    return raw, oracle.dequantize(gtype, raw, N * K).reshape(N, K)


@pytest.mark.parametrize("prec", [0, 1])
@pytest.mark.parametrize("gtype", [pm.GGML_F32, pm.GGML_F16, pm.GGML_Q8_0, pm.GGML_Q4_K])
@pytest.mark.parametrize("M,N,K", [(77, 96, 256), (300, 200, 512), (1, 64, 256), (130, 1030, 768)])
def test_linear(gpu, stream, prec, gtype, M, N, K):
    rng = _rng(M + N + K)
    raw, wf = _weights(gtype, N, K, rng)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    b = rng.normal(0, 0.1, N).astype(np.float32)
    print(f"[linear] prec={prec} type={gtype} M={M} N={N} K={K}", flush=True)
    ref = oracle.linear(x, wf, b)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    db = gpu.DeviceArray.from_numpy(b, stream)
    dy = gpu.DeviceArray((M, N), np.float32)
    gpu.linear(prec, gtype, N, K, raw, dx, M, dy, db, stream)
    got = dy.numpy(stream)
    err = rel_l2(got, ref)
    tol = 1e-5 if prec == 0 else 2e-3
    assert err < tol, err


@pytest.mark.parametrize("M,D", [(1, 64), (257, 512), (2000, 1024), (33, 640)])
def test_layernorm(gpu, stream, M, D):
    rng = _rng(M * D)
    x = (rng.normal(0, 2, (M, D)) + rng.normal(0, 3, (M, 1))).astype(np.float32)
    g = (1 + rng.normal(0, 0.1, D)).astype(np.float32)
    b = rng.normal(0, 0.1, D).astype(np.float32)
    ref = oracle.layer_norm(x, g, b)
    dx, dg, db = (gpu.DeviceArray.from_numpy(a, stream) for a in (x, g, b))
    dy = gpu.DeviceArray((M, D), np.float32)
    gpu.layernorm(dx, dg, db, dy, M, D, 1e-5, stream)
    got = dy.numpy(stream)
    assert rel_l2(got, ref) < 1e-6
    assert np.abs(got - ref).max() < 1e-5


@pytest.mark.parametrize("T,D", [(1, 64), (125, 1024), (375, 512), (26, 512)])
def test_rel_pos_encoding(gpu, stream, T, D):
    ref = oracle.rel_pos_encoding(T, D)
    out = gpu.DeviceArray((2 * T - 1, D), np.float32)
    gpu.rel_pos_encoding(T, D, out, stream)
    got = out.numpy(stream)
    # f64 sin/cos then one rounding to f32: equal up to at most 1 f32 ulp
    ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1


@pytest.mark.parametrize("gtype", [pm.GGML_F16, pm.GGML_Q8_0, pm.GGML_Q4_K])
@pytest.mark.parametrize("M,N,K", [(1000, 3072, 512), (2000, 4096, 256), (333, 2048, 1024), (129, 320, 1280),
                                   (2000, 1024, 4096), (700, 1000, 2048), (2000, 3072, 1024), (1900, 2880, 512),
                                   (2000, 2832, 256)])
def test_linear_tile_shapes(gpu, stream, gtype, M, N, K):
    """f16 path at shapes that select each MFMA tile (64x64, 128x64, 128x128,
    and 128x64 with two K groups for long K; the register-B 128x256 tiles) and
    leave partial tiles on both edges (N = 2832: the last 256-column tile holds
    16 columns, one lane half's store group of one wave)."""
    rng = _rng(M * 7 + N + K)
    raw, wf = _weights(gtype, N, K, rng)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    b = rng.normal(0, 0.1, N).astype(np.float32)
    print(f"[linear-tiles] type={gtype} M={M} N={N} K={K}", flush=True)
    ref = oracle.linear(x, wf, b)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    db = gpu.DeviceArray.from_numpy(b, stream)
    dy = gpu.DeviceArray((M, N), np.float32)
    gpu.linear(1, gtype, N, K, raw, dx, M, dy, db, stream)
    err = rel_l2(dy.numpy(stream), ref)
    assert err < 2e-3, err


def _residual_calls(gpu, stream, gtype, K, shapes, rng, tag):
    """linear_residual (y += alpha (x W^T + b)) on fresh random inputs at each
    (M, N) of shapes.  Every element is checked against a float64 product of
    the exact f16 operands the kernel multiplies (activations rounded to f16;
    q8_0 weights f16(d q), f16 weights as stored), within the worst-case f32
    summation bound of its K terms, and the first element outside it fails
    the test."""
    alpha = 0.5
    for call, (M, N) in enumerate(shapes):
        raw, wf = _weights(gtype, N, K, rng)
        if gtype == pm.GGML_Q8_0:
            blk = raw.reshape(-1, 34)
            d = blk[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
            q = blk[:, 2:].view(np.int8).astype(np.float32)
            w16 = (d * q).astype(np.float16).astype(np.float64).reshape(N, K)
        else:
            w16 = wf.astype(np.float64)
        x = rng.normal(0, 1, (M, K)).astype(np.float32)
        b = rng.normal(0, 0.1, N).astype(np.float32)
        y0 = rng.normal(0, 1, (M, N)).astype(np.float32)
        x16 = x.astype(np.float16).astype(np.float64)
        acc = x16 @ w16.T
        ref = y0.astype(np.float64) + alpha * (acc + b)
        # |f32 sum - exact| <= K 2^-24 sum|x w| (+ the rounding of the last adds)
        bound = K * 2.0 ** -24 * (np.abs(x16) @ np.abs(w16).T) + 2.0 ** -22 * (np.abs(ref) + 1.0)
        print(f"[{tag}] call {call} type={gtype} M={M} N={N} K={K}", flush=True)
        dx = gpu.DeviceArray.from_numpy(x, stream)
        db = gpu.DeviceArray.from_numpy(b, stream)
        dy = gpu.DeviceArray.from_numpy(y0, stream)
        gpu.linear_residual(1, gtype, N, K, raw, dx, M, dy, alpha, db, stream)
        got = dy.numpy(stream).astype(np.float64)
        bad = np.abs(got - ref) > bound
        if bad.any():
            i, j = np.argwhere(bad)[0]
            raise AssertionError(f"call {call}: y[{i}][{j}] = {got[i, j]!r}, float64 {ref[i, j]!r}, "
                                 f"bound {bound[i, j]:.3g} ({int(bad.sum())} elements outside)")
        dx.free(), db.free(), dy.free()


@pytest.mark.parametrize("gtype", [pm.GGML_Q8_0, pm.GGML_F16])
def test_residual_split_k_fresh_inputs(gpu, stream, gtype):
    """The split-K residual product (M <= 512 rows, K >= 1024: S workgroups per
    tile hand partial tiles to the last arriver, which sums them in split order)
    on fresh random inputs at every call, the calls of different sizes (some
    with a tile's splits on two XCDs), so a stale or missing partial cannot
    repeat the previous result."""
    # (M, N): 128 64x64 tiles x 2 splits and 64 x 4 (32 positions per XCD, a
    # tile's splits on one XCD), then 10 tiles x 8 splits and 21 x 4, whose
    # per-XCD ranges (10, 10-11 positions) cut tiles' splits over two XCDs
    _residual_calls(gpu, stream, gtype, 2048, ((512, 1024), (200, 1024), (128, 320), (192, 448), (512, 1024)),
                    _rng(2048), "split-k")


@pytest.mark.parametrize("gtype", [pm.GGML_Q8_0, pm.GGML_F16])
@pytest.mark.parametrize("K", [4096, 1024, 512])
def test_residual_two_k_groups(gpu, stream, gtype, K):
    """The residual products at N = 1024, M = 2000 (FFN linear2 and attention
    output shapes): q8_0 weights on the register-B kernel with two K groups
    (64 x 128 tiles, one per CU), f16 weights on the LDS-B kernel with two K
    groups.  In the former group g sums the other group's partial into row
    block g; M = 2040 leaves the last tile's second row block 24 rows,
    M = 1990 leaves it none (the first 6), and N = 960 leaves the last column
    tile's two right waves no columns."""
    _residual_calls(gpu, stream, gtype, K, ((2000, 1024), (2040, 1024), (1990, 1024), (2000, 960)),
                    _rng(K + gtype), "two-k-groups")


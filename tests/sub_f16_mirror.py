"""Subsampling of the f16 product mode, restated in numpy with the GPU path's
f16 roundings (test infrastructure, used only by the GPU tests).

The f64 oracle (oracle/pk_oracle.c: orc_subsampling) keeps every
intermediate map exact; the f16 mode stores the mel tile, conv.0's weights,
the maps after conv.2, conv.3 and conv.5, the flattened rows and the
pointwise / out weights as f16.  Those storage roundings put its result about
2e-4 (relative L2) from the oracle, which hides kernel faults of the same
size (a wrong row in one frame of eight moves the whole output by 3e-4).
This restatement rounds at exactly those points and accumulates in f64, so
the GPU result differs from it only by f32 accumulation order (an
intermediate value that lands within ~1e-7 of an f16 rounding boundary can
round the other way): agreement to ~1e-5 is expected, and a tolerance there
catches one-row mistakes.

Algorithm and masking follow src/subsampling.cpp (conv.0 :143-157, depthwise
:168-184, pointwise :186-192, flatten :194-204, frame mask :206-231, out
:233-236) in the same form as pk_oracle.c, symmetric padding only.
"""
import numpy as np

import pk_model as pm


def f16(a):
    return np.asarray(a, dtype=np.float64).astype(np.float16).astype(np.float64)


def weight_values(t: pm.Tensor) -> np.ndarray:
    """The f16 values the GPU multiplies with for a weight tensor (f64 array,
    torch shape): f32 rounded to nearest f16, f16 as stored, q8_0 as
    f16(q * d) (the dequantisation computes the product in f16)."""
    if t.gtype == pm.GGML_F32:
        return f16(t.data.reshape(t.shape))
    if t.gtype == pm.GGML_F16:
        return t.data.view(np.float16).astype(np.float64).reshape(t.shape)
    if t.gtype == pm.GGML_Q8_0:
        blk = t.data.reshape(-1, 34)
        d = blk[:, :2].copy().view(np.float16)                 # [nb, 1]
        q = blk[:, 2:].copy().view(np.int8).astype(np.float16)  # [nb, 32]
        return (q * d).astype(np.float64).reshape(t.shape)     # f16 x f16 -> f16 (round to nearest)
    raise ValueError("weight type not covered by the f16 restatement")


def _s2(n):
    """k3 s2 output length, all_paddings 2 (subsampling.cpp:25-46), with C's
    truncating division (a valid length of 0 gives 1)."""
    return int((n - 1) / 2) + 1


def _conv3x3s2(x, To, Fo, taps):
    """sum over (kh, kw) of taps(kh, kw) * x[2 t + kh - 1, 2 f + kw - 1] (zero
    outside x); x [Ti][Fi] or [Ti][Fi][C]; taps returns a scalar or [C]."""
    Ti, Fi = x.shape[:2]
    xp = np.zeros((2 * To + 2, 2 * Fo + 2) + x.shape[2:])
    ti, fi = min(Ti, 2 * To + 1), min(Fi, 2 * Fo + 1)
    xp[1:1 + ti, 1:1 + fi] = x[:ti, :fi]
    acc = 0.0
    for kh in range(3):
        for kw in range(3):
            win = xp[kh:kh + 2 * To:2, kw:kw + 2 * Fo:2]
            acc = acc + (win[..., None] if win.ndim == 2 else win) * taps(kh, kw)
    return acc


def subsampling(m: pm.Model, mel, valid_in=None, stage_masks=True):
    """mel [B][F][T] f32 -> ([B][T3][D] f64, valid_out); valid_in as the
    oracle takes it (per item, or None for T - 1)."""
    w = m.tensors
    p = "encoder.pre_encode."
    C = m.cfg.sub_channels
    vals = lambda n: w[p + n].data.astype(np.float64).reshape(w[p + n].shape)
    w0 = f16(vals("conv.0.weight").reshape(C, 3, 3))
    b0, w2, b2 = vals("conv.0.bias"), vals("conv.2.weight").reshape(C, 3, 3), vals("conv.2.bias")
    w5, b5 = vals("conv.5.weight").reshape(C, 3, 3), vals("conv.5.bias")
    W3 = weight_values(w[p + "conv.3.weight"]).reshape(C, C)
    W6 = weight_values(w[p + "conv.6.weight"]).reshape(C, C)
    b3, b6 = vals("conv.3.bias"), vals("conv.6.bias")
    Wo, bo = weight_values(w[p + "out.weight"]), vals("out.bias")
    B, F, T = mel.shape
    T1, F1 = _s2(T), _s2(F)
    T2, F2 = _s2(T1), _s2(F1)
    T3, F3 = _s2(T2), _s2(F2)
    flat = np.zeros((B, T3, C * F3))
    vout = np.zeros(B, dtype=np.int32)
    for b in range(B):
        v0 = int(valid_in[b]) if valid_in is not None else T - 1
        v1 = _s2(v0)
        v2 = _s2(v1)
        vout[b] = min(_s2(v2), T3)
        m0, m1, m2 = (v0, v1, v2) if stage_masks else (T, T1, T2)
        x = f16(np.asarray(mel[b], dtype=np.float64).T)          # [T][F], the f16 mel tile
        x[m0:] = 0.0
        a1 = np.maximum(_conv3x3s2(x, T1, F1, lambda kh, kw: w0[:, kh, kw]) + b0, 0.0)
        a1[m1:] = 0.0
        a2 = f16(_conv3x3s2(a1, T2, F2, lambda kh, kw: w2[:, kh, kw]) + b2)
        a2p = f16(np.maximum(a2 @ W3.T + b3, 0.0))
        a2p[m2:] = 0.0
        a3 = f16(_conv3x3s2(a2p, T3, F3, lambda kh, kw: w5[:, kh, kw]) + b5)
        a3p = np.maximum(a3 @ W6.T + b6, 0.0)                    # [T3][F3][C]
        a3p[vout[b]:] = 0.0
        flat[b] = f16(a3p.transpose(0, 2, 1).reshape(T3, C * F3))
    return flat @ Wo.T + bo, vout   # (xscaling is the encoder's, encoder.cpp:122-124)

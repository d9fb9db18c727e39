"""The other benchmark shapes at production width, against the oracle.

* 0.6B shape with f16 weights on a ragged batch of 16 clips of 2-20 s
  (T_b = 200 + floor(U * 1801) mel frames, zero-padded to T_max), two
  conformer blocks checked per layer, then the TDT joint (640 hidden, 1025
  tokens + 5 durations) over the encoder output with per-frame argmax.
* 1.1B shape (q8_0, d = 1024, 8 heads, FFN 4096) at batch 8 x 30 s: one
  block at T' = 375, and the long-T stress shape T' = 3750 through the
  relative-position attention alone (batch 1) and through a whole block
  (batch 2, ragged).
Bars: relative L2 1e-2 over valid frames (F16 path); the joint (f32 for
every weight type) fed the same encoder output gives identical argmax ids on
every frame but exact f32 ties.
"""
import numpy as np
import pytest

import oracle
import pk_model as pm
from conftest import argmax_identical, rel_l2

pytestmark = pytest.mark.gpu


def _cfg06(n_layers, **kw):
    base = dict(d_model=1024, n_layers=n_layers, n_heads=8, ff_dim=4096, conv_kernel=9, n_mels=128,
                sub_channels=256, xscaling=False, vocab_size=1024, attn_bias=False, ff_bias=False,
                conv_bias=False, joint_hidden=640, pred_hidden=640)
    base.update(kw)
    return pm.Config(**base)


def test_f16_ragged_batch_with_tdt_joint(gpu, stream):
    cfg = _cfg06(2)
    m = pm.synthesize(cfg, "f16", bn_random=True)
    om = oracle.OracleModel(m)
    gm = gpu.Model.from_tensors(m, 1)
    rng = np.random.default_rng(7)
    B = 16
    lens = (200 + np.floor(rng.random(B) * 1801)).astype(np.int32)
    T = int(lens.max())
    mel = rng.normal(0, 1, (B, cfg.n_mels, T)).astype(np.float32)
    for b, v in enumerate(lens):
        mel[b, :, v:] = 0.0
    print(f"[c3] B={B} T_max={T} lens={lens.tolist()}", flush=True)
    ref, vo_ref, cap_ref = om.encoder(mel, lens - 1, capture=True)
    Tp = oracle.subsampled_len(T)
    dm = gpu.DeviceArray.from_numpy(mel, stream)
    dy = gpu.DeviceArray((B, Tp, cfg.d_model), np.float32)
    dc = gpu.DeviceArray((cfg.n_layers, B, Tp, cfg.d_model), np.float32)
    tp, vo = gm.encoder_forward(dm, lens, dy, capture=dc, stream=stream)
    assert tp == Tp and list(vo) == list(vo_ref)
    cap = dc.numpy(stream)
    mask = np.arange(Tp)[None, :] < np.asarray(vo)[:, None]
    for l in range(cfg.n_layers):
        err = rel_l2(cap[l][mask], cap_ref[l][mask])
        print(f"[c3] layer {l} rel_l2 {err:.2e}", flush=True)
        assert err < 1e-2
    # TDT joint argmax over every valid frame with one prediction-net output
    enc = dy.numpy(stream)[mask]
    g = rng.normal(0, 1, cfg.pred_hidden).astype(np.float32)
    lg_ref, tok_ref, dur_ref = om.tdt_joint(enc, g)
    de, dg = gpu.DeviceArray.from_numpy(enc, stream), gpu.DeviceArray.from_numpy(g, stream)
    Mv, V = lg_ref.shape
    dl = gpu.DeviceArray((Mv, V), np.float32)
    dt, dd = gpu.DeviceArray((Mv,), np.int32), gpu.DeviceArray((Mv,), np.int32)
    gm.tdt_joint(de, Mv, dg, dl, dt, dd, stream)
    tok, dur = dt.numpy(stream), dd.numpy(stream)
    n_tok = V - len(cfg.tdt_durations)
    argmax_identical(tok, tok_ref, lg_ref[:, :n_tok], "c3 joint tokens")
    argmax_identical(dur, dur_ref, lg_ref[:, n_tok:], "c3 joint durations")
    gm.close()


@pytest.fixture(scope="module")
def model11(gpu):
    cfg = _cfg06(1)
    m = pm.synthesize(cfg, "q8_0", heads=False, bn_random=True)
    om = oracle.OracleModel(m)
    gm = gpu.Model.from_tensors(m, 1)
    yield m, om, gm
    gm.close()


def test_long_utterance_block(gpu, stream, model11):
    """One 1.1B-shape block at batch 8 x 30 s (T' = 375), ragged."""
    m, om, gm = model11
    B, T, D = 8, 375, 1024
    rng = np.random.default_rng(375)
    valid = [375, 375, 300, 375, 17, 375, 250, 374]
    x = rng.normal(0, 1, (B, T, D)).astype(np.float32)
    print(f"[c5] B={B} T={T} valid={valid}", flush=True)
    ref = om.conformer_layer(0, x, oracle.rel_pos_encoding(T, D), valid)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dy = gpu.DeviceArray((B, T, D), np.float32)
    gm.conformer_layer(0, dx, valid, dy, None, stream)
    got = dy.numpy(stream)
    mask = np.arange(T)[None, :] < np.asarray(valid)[:, None]
    assert rel_l2(got[mask], ref[mask]) < 1e-2
    assert rel_l2(got[mask] - x[mask], ref[mask] - x[mask]) < 3e-2


def test_long_T_stress_attention(gpu, stream, model11):
    """Relative-position attention at T' = 3750 (300 s of audio), batch 1."""
    m, om, gm = model11
    T, D = 3750, 1024
    rng = np.random.default_rng(3750)
    x = rng.normal(0, 1, (1, T, D)).astype(np.float32)
    valid = [3749]
    print(f"[c5-stress] T={T} valid={valid}", flush=True)
    ref = om.relpos_attention(0, x, oracle.rel_pos_encoding(T, D), valid)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dy = gpu.DeviceArray((1, T, D), np.float32)
    gm.relpos_attention(0, dx, valid, dy, stream)
    got = dy.numpy(stream)
    assert rel_l2(got[0, :3749], ref[0, :3749]) < 1e-2
    assert rel_l2(got[0, 3749:], ref[0, 3749:]) < 1e-2      # padded query row -> linear_out bias


def test_long_T_stress_block(gpu, stream, model11):
    """One 1.1B-shape block at T' = 3750 (300 s of audio), batch 2, ragged: the
    O(T'^2) attention and its rel_shift inside the whole block
    (src/relpos_attention.cpp:252-278, src/conformer.cpp:285-353)."""
    m, om, gm = model11
    B, T, D = 2, 3750, 1024
    rng = np.random.default_rng(37502)
    valid = [3750, 2811]
    x = rng.normal(0, 1, (B, T, D)).astype(np.float32)
    print(f"[c5-stress] block B={B} T={T} valid={valid}", flush=True)
    ref = om.conformer_layer(0, x, oracle.rel_pos_encoding(T, D), valid)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dy = gpu.DeviceArray((B, T, D), np.float32)
    gm.conformer_layer(0, dx, valid, dy, None, stream)
    got = dy.numpy(stream)
    mask = np.arange(T)[None, :] < np.asarray(valid)[:, None]
    assert np.isfinite(got[mask]).all()
    assert rel_l2(got[mask], ref[mask]) < 1e-2
    assert rel_l2(got[mask] - x[mask], ref[mask] - x[mask]) < 3e-2

"""Every benchmark configuration at its own shape and full depth, against the
oracle, through the C ABI.

* 110M f32 block (d 512, 8 x 64 heads, FFN 2048, kernel 9) at B 1 x T' 125,
  valid 125 and 124 (the reference's padded-frame case,
  tests/test_conformer.cpp:16-73): layer output, the conv-module output and
  the attention and conv sublayers alone, each within 1e-4 relative L2.
* 110M f32 encoder (17 blocks) from N(0,1) 80-mel x 1000 frames, every layer
  within 1e-4 (tests/test_encoder.cpp:21-81), then the 1025-way CTC head:
  log-probabilities within 1e-4 and greedy ids identical on every frame except
  exact f32 ties (src/ctc_decoder.cpp:34-116, src/search.cpp:21-90).
* 0.6B q8_0 and q4_K encoders, 24 blocks, B 16 x 10 s, every layer within 1e-2.
* 0.6B f16 encoder, 24 blocks, 16 ragged clips of 2-20 s, every layer within
  1e-2, then the TDT joint (640 hidden, 1025 tokens + 5 durations) argmax.
* 1.1B-shape q8_0 encoder, 42 blocks, the configuration's 8 clips of 30 s
  (T' 375, one of them ragged), every layer within 1e-2.
* 0.6B shape, 3 blocks, at few rows (B 3 ragged and B 1): the split-K
  residual products, every layer within 1e-2 and bit-identical on a repeat.
Relative L2 is over each item's valid frames.
"""
import time

import numpy as np
import pytest

import oracle
import pk_model as pm
from conftest import argmax_identical, argmax_within_error, rel_l2

pytestmark = pytest.mark.gpu


def _cfg110(n_layers):
    return pm.Config(d_model=512, n_layers=n_layers, n_heads=8, ff_dim=2048, conv_kernel=9, n_mels=80,
                     sub_channels=256, xscaling=False, vocab_size=1024, joint_hidden=640, pred_hidden=640,
                     pred_rnn_layers=1)


def _cfg06(n_layers, **kw):
    base = dict(d_model=1024, n_layers=n_layers, n_heads=8, ff_dim=4096, conv_kernel=9, n_mels=128,
                sub_channels=256, xscaling=False, vocab_size=1024, attn_bias=False, ff_bias=False,
                conv_bias=False, joint_hidden=640, pred_hidden=640)
    base.update(kw)
    return pm.Config(**base)


def _mask(T, valid):
    return np.arange(T)[None, :] < np.asarray(valid)[:, None]


def _run_encoder(gpu, stream, gm, om, mel, lens, label, tol):
    """Encoder forward on both sides with per-layer capture; asserts every
    layer and the output within tol.  Returns (gpu out, oracle out, valid)."""
    B, F, T = mel.shape
    D, L = om.cfg.d_model, om.cfg.n_layers
    t0 = time.time()
    ref, vo_ref, cap_ref = om.encoder(mel, np.asarray(lens) - 1, capture=True)
    print(f"[{label}] oracle {time.time() - t0:.1f} s", flush=True)
    Tp = oracle.subsampled_len(T)
    dm = gpu.DeviceArray.from_numpy(mel, stream)
    dy = gpu.DeviceArray((B, Tp, D), np.float32)
    dc = gpu.DeviceArray((L, B, Tp, D), np.float32)
    tp, vo = gm.encoder_forward(dm, lens, dy, capture=dc, stream=stream)
    assert tp == Tp and list(vo) == list(vo_ref)
    cap = dc.numpy(stream)
    mask = _mask(Tp, vo)
    errs = [rel_l2(cap[l][mask], cap_ref[l][mask]) for l in range(L)]
    print(f"[{label}] per-layer rel_l2: " + " ".join(f"{e:.1e}" for e in errs), flush=True)
    for l, e in enumerate(errs):
        assert e < tol, (label, l, e)
    got = dy.numpy(stream)
    assert rel_l2(got[mask], ref[mask]) < tol
    dm.free(), dy.free(), dc.free()
    return got, ref, np.asarray(vo)


# ---------------------------------------------------------------------------
# 110M f32: one block (tests/test_conformer.cpp) and the 17-block encoder +
# CTC (tests/test_encoder.cpp, tests/test_ctc.cpp)
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def block110(gpu):
    m = pm.synthesize(_cfg110(1), "f32", bn_random=True, heads=False)
    gm = gpu.Model.from_tensors(m, gpu.PREC_F32)
    yield m, oracle.OracleModel(m), gm
    gm.close()


@pytest.mark.parametrize("valid", [125, 124])
def test_110m_block_f32(gpu, stream, block110, valid):
    m, om, gm = block110
    B, T, D = 1, 125, 512
    rng = np.random.default_rng(16 + valid)
    x = rng.normal(0, 1, (B, T, D)).astype(np.float32)
    pe = oracle.rel_pos_encoding(T, D)
    print(f"[c1] B={B} T'={T} valid={valid}", flush=True)
    ref, conv_ref = om.conformer_layer(0, x, pe, [valid], want_conv=True)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dy = gpu.DeviceArray((B, T, D), np.float32)
    dconv = gpu.DeviceArray((B, T, D), np.float32)
    gm.conformer_layer(0, dx, [valid], dy, dconv, stream)
    mask = _mask(T, [valid])
    e_layer = rel_l2(dy.numpy(stream)[mask], ref[mask])
    e_conv = rel_l2(dconv.numpy(stream)[mask], conv_ref[mask])
    # the attention and conv sublayers alone, on LayerNorm-ed inputs
    w = om.w
    xa = oracle.layer_norm(x, w["encoder.layers.0.norm_self_att.weight"], w["encoder.layers.0.norm_self_att.bias"])
    att_ref = om.relpos_attention(0, xa, pe, [valid])
    dxa = gpu.DeviceArray.from_numpy(np.ascontiguousarray(xa, dtype=np.float32), stream)
    gm.relpos_attention(0, dxa, [valid], dy, stream)
    e_att = rel_l2(dy.numpy(stream)[mask], att_ref[mask])
    xc = oracle.layer_norm(x, w["encoder.layers.0.norm_conv.weight"], w["encoder.layers.0.norm_conv.bias"])
    cm_ref = om.conv_module(0, xc, [valid])
    dxc = gpu.DeviceArray.from_numpy(np.ascontiguousarray(xc, dtype=np.float32), stream)
    gm.conv_module(0, dxc, [valid], dy, stream)
    e_cm = rel_l2(dy.numpy(stream)[mask], cm_ref[mask])
    print(f"[c1] rel_l2 layer {e_layer:.2e} conv-in-layer {e_conv:.2e} attention {e_att:.2e} "
          f"conv module {e_cm:.2e}", flush=True)
    for e in (e_layer, e_conv, e_att, e_cm):
        assert e < 1e-4


@pytest.fixture(scope="module")
def enc110(gpu):
    m = pm.synthesize(_cfg110(17), "f32", bn_random=True)
    gm = gpu.Model.from_tensors(m, gpu.PREC_F32)
    yield m, oracle.OracleModel(m), gm
    gm.close()


def test_110m_encoder_f32_ctc(gpu, stream, enc110):
    m, om, gm = enc110
    rng = np.random.default_rng(80)
    mel = rng.normal(0, 1, (1, 80, 1000)).astype(np.float32)
    got, ref, vo = _run_encoder(gpu, stream, gm, om, mel, [1000], "c2", 1e-4)
    assert list(vo) == [125]
    # CTC head end to end: oracle encoder -> oracle head vs device encoder -> device head
    V = m.cfg.vocab_size + 1
    enc = np.ascontiguousarray(got[0, :125])
    lp_ref, am_ref = om.ctc(ref[0, :125])
    de = gpu.DeviceArray.from_numpy(enc, stream)
    dlp = gpu.DeviceArray((125, V), np.float32)
    dam = gpu.DeviceArray((125,), np.int32)
    gm.ctc(de, 125, dlp, dam, stream)
    lp, am = dlp.numpy(stream), dam.numpy(stream)
    print(f"[c2] CTC log-prob max abs diff {np.abs(lp - lp_ref).max():.2e}", flush=True)
    assert np.abs(lp - lp_ref).max() < 1e-4
    argmax_identical(am, am_ref, lp_ref, "c2 ctc")
    ids, ids_ref = oracle.ctc_greedy(am, m.cfg.vocab_size), oracle.ctc_greedy(am_ref, m.cfg.vocab_size)
    print(f"[c2] greedy ids: {len(ids)} tokens", flush=True)
    assert list(ids) == list(ids_ref)


# ---------------------------------------------------------------------------
# 0.6B at full depth
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("wtype", ["q8_0", "q4_k"])
def test_06b_full_depth_quantised(gpu, stream, wtype):
    t0 = time.time()
    m = pm.synthesize(_cfg06(24), wtype, bn_random=True, heads=False)
    om = oracle.OracleModel(m)
    gm = gpu.Model.from_tensors(m, gpu.PREC_F16)
    print(f"[c4 {wtype}] models ready in {time.time() - t0:.1f} s", flush=True)
    rng = np.random.default_rng(1000)
    mel = rng.normal(0, 1, (16, 128, 1000)).astype(np.float32)
    _run_encoder(gpu, stream, gm, om, mel, [1000] * 16, f"c4 {wtype}", 1e-2)
    gm.close()


def test_06b_full_depth_f16_ragged_tdt(gpu, stream):
    t0 = time.time()
    cfg = _cfg06(24)
    m = pm.synthesize(cfg, "f16", bn_random=True)
    om = oracle.OracleModel(m)
    gm = gpu.Model.from_tensors(m, gpu.PREC_F16)
    print(f"[c3] models ready in {time.time() - t0:.1f} s", flush=True)
    rng = np.random.default_rng(7)
    B = 16
    lens = (200 + np.floor(rng.random(B) * 1801)).astype(np.int32)
    T = int(lens.max())
    mel = rng.normal(0, 1, (B, cfg.n_mels, T)).astype(np.float32)
    for b, v in enumerate(lens):
        mel[b, :, v:] = 0.0
    print(f"[c3] B={B} T_max={T} lens={lens.tolist()}", flush=True)
    got, ref, vo = _run_encoder(gpu, stream, gm, om, mel, lens, "c3", 1e-2)
    mask = _mask(got.shape[1], vo)
    g = rng.normal(0, 1, cfg.pred_hidden).astype(np.float32)
    n_tok = cfg.vocab_size + 1

    def joint(enc):
        Mv = enc.shape[0]
        V = n_tok + len(cfg.tdt_durations)
        de, dg = gpu.DeviceArray.from_numpy(np.ascontiguousarray(enc), stream), gpu.DeviceArray.from_numpy(g, stream)
        dl = gpu.DeviceArray((Mv, V), np.float32)
        dt, dd = gpu.DeviceArray((Mv,), np.int32), gpu.DeviceArray((Mv,), np.int32)
        gm.tdt_joint(de, Mv, dg, dl, dt, dd, stream)
        return dl.numpy(stream), dt.numpy(stream), dd.numpy(stream)

    # the joint itself (f32) on the same encoder output: identical but for f32 ties
    lg, tok, dur = joint(got[mask])
    lg_ref, tok_ref, dur_ref = om.tdt_joint(got[mask], g)
    assert rel_l2(lg, lg_ref) < 1e-5
    argmax_identical(tok, tok_ref, lg_ref[:, :n_tok], "c3 joint tokens")
    argmax_identical(dur, dur_ref, lg_ref[:, n_tok:], "c3 joint durations")
    # end to end: device encoder (f16 operands) + joint vs oracle encoder + joint
    lg_e2e, tok_e2e, dur_e2e = om.tdt_joint(ref[mask], g)
    argmax_within_error(tok, tok_e2e, lg_e2e[:, :n_tok], lg[:, :n_tok], "c3 end-to-end tokens")
    argmax_within_error(dur, dur_e2e, lg_e2e[:, n_tok:], lg[:, n_tok:], "c3 end-to-end durations")
    gm.close()


# ---------------------------------------------------------------------------
# Few rows (M = B*T' <= 512): the residual products of K >= 1024 (FFN linear2,
# attention out, pw2) split K over 2 (B 3, M 375) or 8 (B 1, M 125) workgroups
# per tile, partials summed in a fixed order
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("wtype,lens", [("q8_0", [1000, 737, 1000]), ("f16", [1000])])
def test_06b_few_rows_split_k(gpu, stream, wtype, lens):
    m = pm.synthesize(_cfg06(3), wtype, bn_random=True, heads=False)
    om = oracle.OracleModel(m)
    gm = gpu.Model.from_tensors(m, gpu.PREC_F16)
    rng = np.random.default_rng(4000)
    mel = rng.normal(0, 1, (len(lens), 128, 1000)).astype(np.float32)
    for b, v in enumerate(lens):
        mel[b, :, v:] = 0.0
    label = f"split-K {wtype} B={len(lens)}"
    print(f"[{label}] lens={lens}", flush=True)
    got, _, _ = _run_encoder(gpu, stream, gm, om, mel, lens, label, 1e-2)
    # deterministic: the same partials in the same order on a second call
    dm = gpu.DeviceArray.from_numpy(mel, stream)
    dy = gpu.DeviceArray(got.shape, np.float32)
    gm.encoder_forward(dm, lens, dy, stream=stream)
    assert np.array_equal(dy.numpy(stream), got)
    dm.free(), dy.free()
    gm.close()


# ---------------------------------------------------------------------------
# 1.1B shape (42 blocks) at 30 s
# ---------------------------------------------------------------------------
def test_11b_full_depth_q8_0(gpu, stream):
    t0 = time.time()
    m = pm.synthesize(_cfg06(42), "q8_0", bn_random=True, heads=False)
    om = oracle.OracleModel(m)
    gm = gpu.Model.from_tensors(m, gpu.PREC_F16)
    print(f"[c5] models ready in {time.time() - t0:.1f} s", flush=True)
    rng = np.random.default_rng(3000)
    lens = [3000, 3000, 3000, 2123, 3000, 3000, 3000, 3000]
    mel = rng.normal(0, 1, (8, 128, 3000)).astype(np.float32)
    mel[3, :, 2123:] = 0.0
    _run_encoder(gpu, stream, gm, om, mel, lens, "c5", 1e-2)
    gm.close()

"""Offline (whole-utterance) forward of a cache-aware streaming model through
the offline entry points, against the oracle: the shape of the reference's
tests/test_encoder_eou.cpp (full encoder with causal subsampling, LayerNorm
conv norm with causal depthwise padding, and the chunked-limited attention
mask, src/conformer.cpp:100-133, src/relpos_attention.cpp:245-275) and
tests/test_conv_eou.cpp (the conv module alone), plus the attention alone
and ragged batches.

Bars (relative L2 over valid frames): F32 path 1e-4, F16 path (f16 / q8_0)
1e-2.
"""
import numpy as np
import pytest

import oracle
import pk_model as pm
from conftest import rel_l2

pytestmark = pytest.mark.gpu

CASES = {
    "f32": (dict(d_model=128, n_heads=4, ff_dim=256), "f32", 0, 1e-4),
    "f16_dk128": (dict(d_model=256, n_heads=2, ff_dim=512), "f16", 1, 1e-2),
    "q8_0": (dict(d_model=256, n_heads=4, ff_dim=512), "q8_0", 1, 1e-2),
    # the BatchNorm conv norm with causal padding, and a window of two chunks
    "f32_bn_window": (dict(d_model=128, n_heads=4, ff_dim=256, conv_norm_type="batch_norm", att_context_left=6,
                           att_context_right=2), "f32", 0, 1e-4),
}
_CACHE = {}


def _models(gpu, name):
    if name not in _CACHE:
        kw, qt, prec, tol = CASES[name]
        base = dict(n_layers=3, conv_kernel=9, n_mels=64, sub_channels=64)
        base.update(kw)
        cfg = pm.eou_config(**base)
        m = pm.synthesize(cfg, qt, heads=False, std=0.05, bn_random=True)
        _CACHE[name] = (cfg, m, oracle.OracleModel(m), gpu.Model.from_tensors(m, precision=prec), tol)
    return _CACHE[name]


def _mask(T, valid):
    return np.arange(T)[None, :] < np.asarray(valid)[:, None]


@pytest.mark.parametrize("name", list(CASES))
def test_eou_encoder_offline_per_layer(gpu, stream, name):
    cfg, m, om, gm, tol = _models(gpu, name)
    rng = np.random.default_rng(71)
    lens = [161, 161, 97]
    B, T = len(lens), max(lens)
    mel = rng.normal(0, 1, (B, cfg.n_mels, T)).astype(np.float32)
    for b, v in enumerate(lens):
        mel[b, :, v:] = 0.0
    print(f"[eou-offline] {name} B={B} T={T} lens={lens}", flush=True)
    ref, vo_ref, cap_ref = om.encoder(mel, np.asarray(lens) - 1, capture=True)
    Tp = oracle.lib().orc_subsampled_len_c(T, 1)
    dm = gpu.DeviceArray.from_numpy(mel, stream)
    dy = gpu.DeviceArray((B, Tp, cfg.d_model), np.float32)
    dc = gpu.DeviceArray((cfg.n_layers, B, Tp, cfg.d_model), np.float32)
    tp, vo = gm.encoder_forward(dm, lens, dy, capture=dc, stream=stream)
    assert tp == Tp and list(vo) == list(vo_ref)
    cap = dc.numpy(stream)
    mask = _mask(Tp, vo)
    errs = [rel_l2(cap[l][mask], cap_ref[l][mask]) for l in range(cfg.n_layers)]
    print(f"[eou-offline]   per-layer rel_l2 " + " ".join(f"{e:.1e}" for e in errs), flush=True)
    for l, e in enumerate(errs):
        assert e < tol, (name, l, e)
    assert rel_l2(dy.numpy(stream)[mask], ref[mask]) < tol


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("valid", [[40], [40, 23]])
def test_eou_conv_module_and_attention(gpu, stream, name, valid):
    """The conv module alone (LayerNorm or BatchNorm conv norm, causal
    depthwise padding) and the attention alone (chunked-limited mask), ragged."""
    cfg, m, om, gm, tol = _models(gpu, name)
    rng = np.random.default_rng(40 + len(valid))
    B, T, D = len(valid), 40, cfg.d_model
    c = rng.normal(0, 1, (B, T, D)).astype(np.float32)
    print(f"[eou-offline] {name} conv module / attention B={B} T={T} valid={valid}", flush=True)
    mask = _mask(T, valid)
    ref = om.conv_module(0, c, valid)
    dx = gpu.DeviceArray.from_numpy(c, stream)
    dy = gpu.DeviceArray((B, T, D), np.float32)
    gm.conv_module(0, dx, valid, dy, stream)
    e_conv = rel_l2(dy.numpy(stream)[mask], ref[mask])
    pe = oracle.rel_pos_encoding(T, D)
    ref_a = om.relpos_attention(1, c, pe, valid)
    gm.relpos_attention(1, dx, valid, dy, stream)
    got_a = dy.numpy(stream)
    e_att = rel_l2(got_a[mask], ref_a[mask])
    print(f"[eou-offline]   conv module rel_l2 {e_conv:.2e}, attention rel_l2 {e_att:.2e}", flush=True)
    assert e_conv < tol and e_att < tol
    # padded query rows of the attention are linear_out.bias (src/relpos_attention.cpp:291-302)
    if not mask.all():
        assert rel_l2(got_a[~mask], ref_a[~mask]) < tol


def test_eou_layer_matches_streamed_frames(gpu, stream):
    """The conformer block entry point on a streaming model, with the
    conv-module capture, against the oracle's block."""
    cfg, m, om, gm, tol = _models(gpu, "f32")
    rng = np.random.default_rng(9)
    B, T, D = 2, 33, cfg.d_model
    valid = [33, 17]
    x = rng.normal(0, 1, (B, T, D)).astype(np.float32)
    pe = oracle.rel_pos_encoding(T, D)
    ref, conv_ref = om.conformer_layer(2, x, pe, valid, want_conv=True)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dy = gpu.DeviceArray((B, T, D), np.float32)
    dconv = gpu.DeviceArray((B, T, D), np.float32)
    gm.conformer_layer(2, dx, valid, dy, dconv, stream)
    mask = _mask(T, valid)
    e1 = rel_l2(dy.numpy(stream)[mask], ref[mask])
    e2 = rel_l2(dconv.numpy(stream)[mask], conv_ref[mask])
    print(f"[eou-offline] block rel_l2 {e1:.2e}, conv-in-block {e2:.2e}", flush=True)
    assert e1 < tol and e2 < tol

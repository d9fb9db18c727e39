"""Pins of the oracle's cache-aware streaming encoder and the streaming-model
variants it rests on (no GPU).

* causal subsampling (subsampling.cpp:81-99, pad 2 before / 1 after on both
  axes): against an independent scipy correlate2d + numpy restatement;
* causal depthwise conv + LayerNorm conv-norm (conformer.cpp:100-133): a
  depthwise kernel that is a delta at the last tap turns the conv into the
  identity only when the padding is K-1 on the left, which reduces the module
  to numpy LayerNorm / SiLU / products; and causality itself (future frames
  never change earlier outputs);
* chunked-limited attention (relpos_attention.cpp:245-275): a window wider than
  the clip reduces to full attention; frames outside a query's chunk window
  never change its output;
* StreamingEncoder::step (streaming_encoder.cpp:340-462): the concatenated
  chunk outputs equal the offline encoder with the same masks and causal
  convolutions (cache-aware equivalence, tests/test_streaming_encoder.cpp:127-
  155), chunk by chunk in the reference's schedule; reset() restarts the stream.
"""
import numpy as np
import pytest
from scipy.signal import correlate2d

import oracle
import pk_model as pm
from conftest import rel_l2


def eou_tiny(**kw):
    base = dict(d_model=64, n_layers=2, n_heads=4, ff_dim=128, conv_kernel=9, n_mels=32, sub_channels=16)
    base.update(kw)
    return pm.eou_config(**base)


@pytest.fixture(scope="module")
def eou():
    cfg = eou_tiny()
    m = pm.synthesize(cfg, "f32", heads=False, std=0.1)
    return cfg, oracle.OracleModel(m)


def _np_causal_subsampling(om, mel):
    """Independent restatement: explicit (2, 1) zero padding, scipy correlation,
    stride-2 slicing, numpy products; input [F][T] -> [T3][D] (float64)."""
    w = {k: om.w["encoder.pre_encode." + k].astype(np.float64) for k in
         ("conv.0.weight", "conv.0.bias", "conv.2.weight", "conv.2.bias", "conv.3.weight", "conv.3.bias",
          "conv.5.weight", "conv.5.bias", "conv.6.weight", "conv.6.bias", "out.weight", "out.bias")}
    x = mel.T.astype(np.float64)                            # [T][F], H = time, W = feature
    C = w["conv.0.weight"].shape[0]

    def pad(a):
        return np.pad(a, ((2, 1), (2, 1)))

    def conv_s2(img, k):
        return correlate2d(pad(img), k, mode="valid")[::2, ::2]

    a = np.stack([np.maximum(conv_s2(x, w["conv.0.weight"][c, 0]) + w["conv.0.bias"][c], 0) for c in range(C)])
    for dw, pw in (("conv.2", "conv.3"), ("conv.5", "conv.6")):
        d = np.stack([conv_s2(a[c], w[dw + ".weight"][c, 0]) + w[dw + ".bias"][c] for c in range(C)])
        a = np.maximum(np.einsum("oc,cij->oij", w[pw + ".weight"][:, :, 0, 0], d)
                       + w[pw + ".bias"][:, None, None], 0)
    T3 = a.shape[1]
    flat = a.transpose(1, 0, 2).reshape(T3, -1)             # per time: channel-major c*F' + f
    return flat @ w["out.weight"].T + w["out.bias"]


@pytest.mark.parametrize("T", [9, 25, 40, 57])
def test_causal_subsampling_matches_numpy(eou, T):
    cfg, om = eou
    rng = np.random.default_rng(T)
    mel = rng.normal(0, 1, (1, cfg.n_mels, T)).astype(np.float32)
    got, vo = om.subsampling(mel, valid_in=[T])
    ref = _np_causal_subsampling(om, mel[0])
    assert got.shape[1] == ref.shape[0] == oracle.lib().orc_subsampled_len_c(T, 1)
    assert vo[0] == got.shape[1]                           # every frame valid: no masking
    assert rel_l2(got[0], ref) < 1e-5


def test_causal_subsampling_lengths():
    # calc_length with all_paddings 3: floor(t/2) + 1 per stage
    for T in range(1, 200):
        t = T
        for _ in range(3):
            t = t // 2 + 1
        assert oracle.lib().orc_subsampled_len_c(T, 1) == t
        assert oracle.lib().orc_valid_out_len_c(T, T, 1) == t


def _layer_of(om, i):
    return {k: om.w[f"encoder.layers.{i}.{v}"].astype(np.float64)
            for k, v in oracle._LAYER_MAP.items() if f"encoder.layers.{i}.{v}" in om.w}


def _np_ln(x, g, b):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + 1e-5) * g + b


def test_causal_conv_layer_norm_closed_form(eou):
    """Delta at the last tap: causal depthwise conv == identity (+ bias)."""
    cfg, om = eou
    K, D = cfg.conv_kernel, cfg.d_model
    L = om.layers[0]
    dw = np.zeros((D, 1, K), np.float32)
    dw[:, 0, K - 1] = 1.0
    L.dw_w = oracle.fp(dw)
    try:
        rng = np.random.default_rng(5)
        c = rng.normal(0, 1, (2, 13, D)).astype(np.float32)
        got = om.conv_module(0, c, [13, 9])
    finally:   # a ctypes pointer field read shares the struct's storage: restore from the array
        L.dw_w = oracle.fp(om.w["encoder.layers.0.conv.depthwise_conv.weight"])
    w = _layer_of(om, 0)
    y = c.astype(np.float64) @ w["pw1_w"][:, :, 0].T + w["pw1_b"]
    glu = y[..., :D] / (1 + np.exp(-y[..., D:]))
    glu[1, 9:] = 0.0                                       # pad mask of the shorter item
    n = _np_ln(glu + w["dw_b"], w["bn_g"], w["bn_b"])
    n = n / (1 + np.exp(-n))
    ref = n @ w["pw2_w"][:, :, 0].T + w["pw2_b"]
    assert rel_l2(got, ref) < 1e-5


def test_causal_conv_ignores_future(eou):
    cfg, om = eou
    rng = np.random.default_rng(6)
    c = rng.normal(0, 1, (1, 20, cfg.d_model)).astype(np.float32)
    a = om.conv_module(0, c, [20])
    c2 = c.copy()
    c2[0, 12:] += rng.normal(0, 1, (8, cfg.d_model)).astype(np.float32)
    b = om.conv_module(0, c2, [20])
    assert np.array_equal(a[0, :12], b[0, :12])
    assert not np.allclose(a[0, 12:], b[0, 12:])


def test_chunked_limited_wide_window_is_full_attention():
    cfg_r = pm.Config(d_model=64, n_layers=1, n_heads=4, ff_dim=128, n_mels=32, sub_channels=16)
    cfg_c = eou_tiny(n_layers=1, att_context_left=1000, att_context_right=999)
    m = pm.synthesize(cfg_r, "f32", heads=False, std=0.1)
    om_r = oracle.OracleModel(m)
    om_c = oracle.OracleModel(pm.Model(cfg_c, dict(m.tensors)))
    rng = np.random.default_rng(7)
    T = 23
    x = rng.normal(0, 1, (2, T, 64)).astype(np.float32)
    pe = oracle.rel_pos_encoding(T, 64)
    assert np.array_equal(om_r.relpos_attention(0, x, pe, [T, 17]), om_c.relpos_attention(0, x, pe, [T, 17]))


def test_chunked_limited_window(eou):
    """att_context [6, 1]: chunks of 2, queries see 3 chunks back; frames outside
    the window leave a query's output unchanged, frames inside change it."""
    cfg = eou_tiny(n_layers=1, att_context_left=6, att_context_right=1)
    om = oracle.OracleModel(pm.synthesize(cfg, "f32", heads=False, std=0.1))
    rng = np.random.default_rng(8)
    T = 24
    x = rng.normal(0, 1, (1, T, 64)).astype(np.float32)
    pe = oracle.rel_pos_encoding(T, 64)
    base = om.relpos_attention(0, x, pe, [T])
    j = 11                                                  # chunk 5
    x2 = x.copy()
    x2[0, j] += 1.0
    out = om.relpos_attention(0, x2, pe, [T])
    for i in range(T):
        d = i // 2 - j // 2
        same = np.array_equal(out[0, i], base[0, i])
        assert same == (not (0 <= d <= 3)) or i == j, (i, d)


def _stream_all(om, cfg, mel):
    st = oracle.Stream(om)
    outs = []
    for lo, hi, last in oracle.stream_windows(mel.shape[1], st.chunk_first, st.chunk, st.pre_cache):
        outs.append(st.step(mel[:, lo:hi], is_last=last))
    return np.concatenate(outs), st


@pytest.mark.parametrize("T", [150, 121, 96])
def test_stream_equals_offline(eou, T):
    cfg, om = eou
    rng = np.random.default_rng(T)
    mel = rng.normal(0, 1, (cfg.n_mels, T)).astype(np.float32)
    got, st = _stream_all(om, cfg, mel)
    off, vo = om.encoder(mel[None], valid_in=[T])
    Tp = off.shape[1]
    assert got.shape == (Tp, cfg.d_model)
    # the last chunk's frames may see a different right edge; every earlier frame is
    # the offline frame
    lead = Tp - st.valid_out_len
    err = rel_l2(got[:lead], off[0, :lead])
    print(f"T={T} T'={Tp} lead={lead} rel_l2={err:.2e}")
    assert err < 1e-5
    # with every mel frame valid the last window ends where the clip ends, so
    # the tail matches too (the reference's offline baseline masks the last
    # mel frame, which is why its test leaves the tail out)
    assert rel_l2(got, off[0]) < 1e-5


def test_stream_reset_and_chunk_outputs(eou):
    cfg, om = eou
    rng = np.random.default_rng(3)
    mel = rng.normal(0, 1, (cfg.n_mels, 90)).astype(np.float32)
    a, st = _stream_all(om, cfg, mel)
    st.reset()
    outs = [st.step(mel[:, lo:hi], is_last=last)
            for lo, hi, last in oracle.stream_windows(90, st.chunk_first, st.chunk, st.pre_cache)]
    assert np.array_equal(np.concatenate(outs), a)
    assert [o.shape[0] for o in outs[:-1]] == [2] * (len(outs) - 1)
    # a window too short for an output frame after the drop yields nothing
    st.reset()
    st.step(mel[:, :9])
    assert st.step(mel[:, :7]).shape[0] == 0               # 7 frames -> 2 subsampled, both dropped


def test_stream_planted_mistake_detected(eou):
    """A stream that forgets the attention cache (clc never grows) differs from offline."""
    cfg, om = eou
    rng = np.random.default_rng(4)
    mel = rng.normal(0, 1, (cfg.n_mels, 80)).astype(np.float32)
    st = oracle.Stream(om)
    outs = []
    for lo, hi, last in oracle.stream_windows(80, st.chunk_first, st.chunk, st.pre_cache):
        outs.append(st.step(mel[:, lo:hi], is_last=last))
        st.reset()                                          # planted: caches dropped every chunk
        st.step(mel[:, :9])                                 # step counter past the first chunk
    off, _ = om.encoder(mel[None], valid_in=[80])
    got = np.concatenate(outs)
    assert rel_l2(got[:-2], off[0, :got.shape[0] - 2]) > 1e-2

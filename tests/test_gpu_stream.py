"""Cache-aware streaming encoder through the C ABI (pkx_streaming_*) vs the
oracle's restatement of pk::StreamingEncoder (streaming_encoder.cpp:340-462),
chunk by chunk in the reference's schedule (tests/test_streaming_encoder.cpp:
68-99), for several streams at once, plus the causal subsampling
(subsampling.cpp:81-147) on its own.

Bars (relative L2): F32 path 1e-4; F16 path (f16 / q8_0 weights) 1e-2.  The
oracle itself is pinned to the offline encoder (streaming == offline) on the
CPU, so these chunks are also the offline encoder's frames.
"""
import numpy as np
import pytest

import oracle
import pk_model as pm
from conftest import rel_l2

pytestmark = pytest.mark.gpu

CASES = {
    "f32": (dict(d_model=128, n_heads=4, ff_dim=256), "f32", 0, 1e-4),
    "f16": (dict(d_model=128, n_heads=2, ff_dim=256), "f16", 1, 1e-2),
    "q8_0": (dict(d_model=256, n_heads=4, ff_dim=512), "q8_0", 1, 1e-2),
    "f16_dk128": (dict(d_model=256, n_heads=2, ff_dim=512), "f16", 1, 1e-2),
    # K = 2048 in linear2: the two-K-group products at few rows
    "q8_0_ff2048": (dict(d_model=256, n_heads=4, ff_dim=2048), "q8_0", 1, 1e-2),
}


def _cfg(kw, n_layers=2):
    base = dict(n_layers=n_layers, conv_kernel=9, n_mels=32, sub_channels=64)
    base.update(kw)
    return pm.eou_config(**base)


_CACHE = {}


def _models(gpu, name):
    if name not in _CACHE:
        kw, qt, prec, tol = CASES[name]
        cfg = _cfg(kw)
        m = pm.synthesize(cfg, qt, heads=False, std=0.05)
        _CACHE[name] = (cfg, m, oracle.OracleModel(m), gpu.Model.from_tensors(m, precision=prec), tol)
    return _CACHE[name]


@pytest.mark.parametrize("name", list(CASES))
def test_causal_subsampling_ragged(gpu, stream, name):
    cfg, m, om, gm, tol = _models(gpu, name)
    rng = np.random.default_rng(11)
    B, T = 3, 57
    vt = np.array([57, 40, 25], np.int32)
    mel = rng.normal(0, 1, (B, cfg.n_mels, T)).astype(np.float32)
    print(f"[stream] causal subsampling {name} B={B} T={T}", flush=True)
    d_mel = gpu.DeviceArray.from_numpy(mel, stream)
    Tp = oracle.lib().orc_subsampled_len_c(T, 1)
    out = gpu.DeviceArray((B, Tp, cfg.d_model), np.float32)
    tout, vo = gm.subsampling_forward(d_mel, vt, out, stream=stream)
    ref, vref = om.subsampling(mel, valid_in=vt - 1)      # the C ABI's entry convention: valid_T - 1
    assert tout == Tp and np.array_equal(vo, vref)
    got = out.numpy(stream)
    for b in range(B):
        err = rel_l2(got[b, :vo[b]], ref[b, :vo[b]])
        print(f"[stream]   item {b}: rel_l2 {err:.2e}", flush=True)
        assert err < tol


@pytest.mark.parametrize("name", list(CASES))
def test_streaming_matches_oracle(gpu, stream, name):
    cfg, m, om, gm, tol = _models(gpu, name)
    S, T = 3, 121
    rng = np.random.default_rng(5)
    mels = rng.normal(0, 1, (S, cfg.n_mels, T)).astype(np.float32)
    st = gpu.Streaming(gm, n_streams=S, max_window=25, stream=stream)
    assert (st.chunk_first, st.chunk, st.pre_cache, st.valid_out_len) == (9, 16, 9, 2)
    refs = [oracle.Stream(om) for _ in range(S)]
    windows = oracle.stream_windows(T, st.chunk_first, st.chunk, st.pre_cache)
    print(f"[stream] {name}: {S} streams, {len(windows)} chunks", flush=True)
    worst = 0.0
    for k, (lo, hi, last) in enumerate(windows):
        n = hi - lo
        tc = st.chunk_len(n)
        d_mel = gpu.DeviceArray.from_numpy(np.ascontiguousarray(mels[:, :, lo:hi]), stream)
        out = gpu.DeviceArray((S, max(tc, 1), cfg.d_model), np.float32)
        nv = st.step(d_mel, out, is_last=last, stream=stream)
        got = out.numpy(stream)
        for s in range(S):
            ref = refs[s].step(mels[s, :, lo:hi], is_last=last)
            assert nv == ref.shape[0], (k, nv, ref.shape)
            if nv:
                err = rel_l2(got[s, :nv], ref)
                worst = max(worst, err)
                assert err < tol, (name, k, s, err)
    print(f"[stream]   worst chunk rel_l2 {worst:.2e}; step_num {st.step_num}", flush=True)
    assert st.step_num == len(windows)
    st.close()


def test_streaming_reset_and_short_window(gpu, stream):
    cfg, m, om, gm, tol = _models(gpu, "f32")
    rng = np.random.default_rng(9)
    mel = rng.normal(0, 1, (1, cfg.n_mels, 60)).astype(np.float32)
    st = gpu.Streaming(gm, n_streams=1, max_window=25, stream=stream)

    def run():
        outs = []
        for lo, hi, last in oracle.stream_windows(60, 9, 16, 9):
            d = gpu.DeviceArray.from_numpy(np.ascontiguousarray(mel[:, :, lo:hi]), stream)
            o = gpu.DeviceArray((1, max(st.chunk_len(hi - lo), 1), cfg.d_model), np.float32)
            nv = st.step(d, o, is_last=last, stream=stream)
            outs.append(o.numpy(stream)[0, :nv])
        return np.concatenate(outs)

    a = run()
    st.reset(stream)
    assert st.step_num == 0
    b = run()
    assert np.array_equal(a, b)
    # after the first chunk, a 7-frame window yields two subsampled frames, both dropped
    st.reset(stream)
    d = gpu.DeviceArray.from_numpy(np.ascontiguousarray(mel[:, :, :9]), stream)
    o = gpu.DeviceArray((1, 2, cfg.d_model), np.float32)
    assert st.step(d, o, stream=stream) == 2
    assert st.chunk_len(7) == 0
    d7 = gpu.DeviceArray.from_numpy(np.ascontiguousarray(mel[:, :, :7]), stream)
    assert st.step(d7, o, stream=stream) == 0
    with pytest.raises(gpu.PkxError):
        st.step(gpu.DeviceArray.from_numpy(np.zeros((1, cfg.n_mels, 26), np.float32), stream), o, stream=stream)
    st.close()


def test_streaming_needs_streaming_model(gpu, stream):
    cfg = pm.Config(d_model=128, n_layers=1, n_heads=2, ff_dim=256, n_mels=32, sub_channels=64)
    gm = gpu.Model.from_tensors(pm.synthesize(cfg, "f32", heads=False), precision=0)
    with pytest.raises(gpu.PkxError, match="streaming configuration"):
        gpu.Streaming(gm, 1, 25, stream=stream)


def test_streaming_model_from_gguf(gpu, stream, tmp_path):
    """The streaming KV (scripts/convert_parakeet_to_gguf.py:176-222) loads
    (src/model_loader.cpp:110-131) and the loaded model streams exactly like the
    same tensors uploaded directly."""
    cfg, m, om, gm, tol = _models(gpu, "q8_0")
    path = str(tmp_path / "eou.gguf")
    pm.write_gguf(m, path)
    g2 = gpu.Model.load_gguf(path)
    c = g2.cfg
    assert (c.conv_ln, c.causal_sub, c.conv_causal, c.att_limited, c.att_left, c.att_right) == (1, 1, 1, 1, 70, 1)
    assert (c.stream_chunk_first, c.stream_chunk, c.stream_pre_cache, c.stream_cache_len,
            c.stream_valid_out_len, c.stream_drop_extra) == (9, 16, 9, 70, 2, 2)
    rng = np.random.default_rng(2)
    mel = rng.normal(0, 1, (2, cfg.n_mels, 50)).astype(np.float32)
    outs = []
    for model in (gm, g2):
        st = gpu.Streaming(model, n_streams=2, max_window=25, stream=stream)
        res = []
        for lo, hi, last in oracle.stream_windows(50, 9, 16, 9):
            d = gpu.DeviceArray.from_numpy(np.ascontiguousarray(mel[:, :, lo:hi]), stream)
            o = gpu.DeviceArray((2, max(st.chunk_len(hi - lo), 1), cfg.d_model), np.float32)
            nv = st.step(d, o, is_last=last, stream=stream)
            res.append(o.numpy(stream)[:, :nv])
        outs.append(np.concatenate(res, axis=1))
        st.close()
    assert np.array_equal(outs[0], outs[1])


def test_streaming_binding_checks_shapes(gpu, stream):
    """The device buffers' sizes cannot cross the C ABI, so the binding checks
    them before the call: a window for the wrong number of streams or an output
    too short for the chunk is refused without a launch."""
    cfg, m, om, gm, tol = _models(gpu, "f32")
    st = gpu.Streaming(gm, n_streams=2, max_window=25, stream=stream)
    one = gpu.DeviceArray((1, cfg.n_mels, 9), np.float32)
    out = gpu.DeviceArray((2, 2, cfg.d_model), np.float32)
    with pytest.raises(gpu.PkxError, match="mel must be"):
        st.step(one, out, stream=stream)
    two = gpu.DeviceArray.from_numpy(np.zeros((2, cfg.n_mels, 9), np.float32), stream)
    short = gpu.DeviceArray((2, 1, cfg.d_model), np.float32)
    with pytest.raises(gpu.PkxError, match="out must be"):
        st.step(two, short, stream=stream)
    # an output with more rows than the chunk would put the second stream's
    # frames at the wrong offset (the device writes one packed [S][tc][D] block)
    long_out = gpu.DeviceArray((2, 5, cfg.d_model), np.float32)
    with pytest.raises(gpu.PkxError, match="out must be"):
        st.step(two, long_out, stream=stream)
    assert st.step_num == 0
    assert st.step(two, out, stream=stream) == 2
    st.close()


# Schedules and variants beyond the streaming model's own: chunks of 72 mel
# frames (9 encoder frames per step, more than the compile-time conv kernel's
# 8, so the generic causal conv and a 9-row attention chunk run), the
# BatchNorm conv norm, and a depthwise kernel of 5.
VARIANTS = {
    "f16_tc9_batchnorm": (dict(d_model=128, n_heads=2, ff_dim=256, conv_norm_type="batch_norm",
                               stream_chunk_size=(9, 72), stream_shift_size=(9, 72), stream_valid_out_len=9,
                               att_context_right=8), "f16", 1, 1e-2, 81),
    "f32_tc9": (dict(d_model=128, n_heads=4, ff_dim=256, stream_chunk_size=(9, 72), stream_shift_size=(9, 72),
                     stream_valid_out_len=9, att_context_right=8), "f32", 0, 1e-4, 81),
    "f32_k5": (dict(d_model=128, n_heads=4, ff_dim=256, conv_kernel=5), "f32", 0, 1e-4, 25),
    "q8_0_k5_batchnorm": (dict(d_model=256, n_heads=4, ff_dim=512, conv_kernel=5, conv_norm_type="batch_norm"),
                          "q8_0", 1, 1e-2, 25),
}


@pytest.mark.parametrize("name", list(VARIANTS))
def test_streaming_variants_match_oracle(gpu, stream, name):
    kw, qt, prec, tol, max_window = VARIANTS[name]
    cfg = _cfg(kw)
    m = pm.synthesize(cfg, qt, heads=False, std=0.05, bn_random=True)
    om = oracle.OracleModel(m)
    gm = gpu.Model.from_tensors(m, precision=prec)
    S, T = 2, 200
    rng = np.random.default_rng(21)
    mels = rng.normal(0, 1, (S, cfg.n_mels, T)).astype(np.float32)
    st = gpu.Streaming(gm, n_streams=S, max_window=max_window, stream=stream)
    refs = [oracle.Stream(om) for _ in range(S)]
    windows = oracle.stream_windows(T, st.chunk_first, st.chunk, st.pre_cache)
    tcs = sorted({st.chunk_len(hi - lo) for lo, hi, _ in windows})
    print(f"[stream] {name}: {S} streams, {len(windows)} chunks, chunk lengths {tcs}", flush=True)
    worst = 0.0
    for k, (lo, hi, last) in enumerate(windows):
        tc = st.chunk_len(hi - lo)
        d_mel = gpu.DeviceArray.from_numpy(np.ascontiguousarray(mels[:, :, lo:hi]), stream)
        out = gpu.DeviceArray((S, max(tc, 1), cfg.d_model), np.float32)
        nv = st.step(d_mel, out, is_last=last, stream=stream)
        got = out.numpy(stream)
        for s in range(S):
            ref = refs[s].step(mels[s, :, lo:hi], is_last=last)
            assert nv == ref.shape[0], (k, nv, ref.shape)
            if nv:
                err = rel_l2(got[s, :nv], ref)
                worst = max(worst, err)
                assert err < tol, (name, k, s, err)
    print(f"[stream]   worst chunk rel_l2 {worst:.2e}", flush=True)
    if "tc9" in name:
        assert max(tcs) > 8
    st.close()
    gm.close()

"""The C++ encoder-path tests (tests/cpp/, written against the host classes in
include/pk_encoder.hpp) run on the GPU against a synthetic model GGUF and a
baseline GGUF whose tensors come from the oracle, named as the reference's
parity baselines name them (tests/python/check_baseline.py:51-69):
mel, subsampling_out, pos_emb, enc_pre_layers, l0_attn_in/out, l0_conv_out,
enc_layer_{0,mid,last}, encoder_out.  The mel has 1001 frames, so T' = 126
with 125 valid frames: the last frame is padding, as in the reference's
fixtures (valid_len = T - 1 in its layer tests).  The baseline pos_emb is
rel_pos_encoding perturbed by up to 5e-4 (NeMo's table is computed in f32);
the layer baselines are computed with that table, which the host classes
must use as given; pos_emb_f64 is the exact table."""
import os
import subprocess

import numpy as np
import pytest

import oracle
import pk_model as pm

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "build")
TESTS = ["test_subsampling", "test_subsampling_batch", "test_relpos_attention", "test_relpos_attention_batch",
         "test_conformer", "test_conformer_batch", "test_encoder", "test_encoder_batch", "test_mel",
         "test_transducer_greedy_batch", "test_model_loader"]
_FILES = {}


def read_wav(path):
    """16-bit mono PCM -> f32 in [-1, 1) (x / 32768, as dr_wav converts s16)."""
    import wave
    with wave.open(path, "rb") as w:
        assert w.getsampwidth() == 2 and w.getnchannels() == 1 and w.getframerate() == 16000
        a = np.frombuffer(w.readframes(w.getnframes()), dtype="<i2")
    return (a.astype(np.float32) / np.float32(32768.0)).astype(np.float32)


def _files(tmp_path_factory, wtype):
    if wtype in _FILES:
        return _FILES[wtype]
    d = tmp_path_factory.mktemp(f"cpp_{wtype}")
    cfg = pm.Config(d_model=256, n_layers=4, n_heads=4, ff_dim=1024, conv_kernel=9, n_mels=80, sub_channels=64,
                    xscaling=True, vocab_size=127, joint_hidden=64, pred_hidden=64)
    m = pm.add_featurizer(pm.add_prediction(pm.synthesize(cfg, wtype, bn_random=True)))
    for n in ("joint.joint_net.2.weight", "joint.joint_net.2.bias"):   # decision margins far above f32 rounding
        t = m.tensors[n]
        m.tensors[n] = pm.Tensor(t.gtype, t.shape, (t.data * 60.0).astype(np.float32))
    om = oracle.OracleModel(m)
    rng = np.random.default_rng(42)
    F, T = cfg.n_mels, 1001
    mel = rng.standard_normal((F, T)).astype(np.float32)
    sub, vo = om.subsampling(mel[None], None, stage_masks=False)
    Tp, D = sub.shape[1], cfg.d_model
    assert Tp == 126 and vo[0] == Tp - 1
    # the whole-window convention (in_valid_frames = T, src/subsampling.hpp:53-61)
    sub_w, vo_w = om.subsampling(mel[None], [T], stage_masks=False)
    assert vo_w[0] == Tp
    pre = (sub[0] * np.float32(np.sqrt(D))).astype(np.float32)
    pe64 = oracle.rel_pos_encoding(Tp, D)
    # the layer-level baselines take a table perturbed by up to 5e-4 (a table
    # computed in f32 elsewhere, as NeMo's is): the host classes must use the
    # caller's table as given (the encoder computes its own)
    pe = (pe64 + rng.uniform(-5e-4, 5e-4, pe64.shape)).astype(np.float32)
    enc, vo2, cap = om.encoder(mel[None], None, stage_masks=False, capture=True)
    valid = [Tp - 1]
    y0, conv0 = om.conformer_layer(0, pre[None], pe, valid, want_conv=True)
    attn_in = rng.standard_normal((Tp, D)).astype(np.float32)
    conv_in = rng.standard_normal((Tp, D)).astype(np.float32)
    L = cfg.n_layers
    base = {
        "mel": mel, "subsampling_out": sub[0], "subsampling_out_whole": sub_w[0],
        "subsampling_valid_whole": np.array([vo_w[0]], np.int32), "pos_emb": pe, "pos_emb_f64": pe64, "enc_pre_layers": pre,
        "l0_attn_in": attn_in, "l0_attn_out": om.relpos_attention(0, attn_in[None], pe, valid)[0],
        "l0_conv_out": conv0[0], "l0_conv_in": conv_in,
        "l0_conv_module_out": om.conv_module(0, conv_in[None], valid)[0],
        "enc_layer_0": y0[0], "enc_layer_mid": cap[L // 2][0], "enc_layer_last": cap[L - 1][0],
        "encoder_out": np.ascontiguousarray(enc[0].T),
    }
    # log-mel of the speech fixture (the oracle's MelFrontend restatement)
    pcm = read_wav(os.path.join(ROOT, "tests", "golden", "speech.wav"))
    mcfg = oracle.mel_cfg(n_fft=cfg.n_fft, hop=cfg.hop_length, n_mels=cfg.n_mels, preemph=cfg.preemph,
                          mag_power=cfg.mag_power, log_guard=cfg.log_zero_guard)
    base["pcm"] = pcm
    # greedy TDT decode of a ragged batch of encoder outputs (the oracle's per-item loop)
    tr = oracle.Transducer(m)
    dT = np.array([40, 23, 9], np.int32)
    denc = rng.standard_normal((3, 40, cfg.d_model)).astype(np.float32)
    base["dec_enc"], base["dec_T"] = denc, dT
    base["dec_durations"] = np.array(cfg.tdt_durations, np.int32)
    for n in range(3):
        ids, fr, _, sp = tr.greedy(denc[n, :dT[n]], cfg.tdt_durations)
        base[f"dec_ids_{n}"], base[f"dec_frames_{n}"], base[f"dec_spans_{n}"] = ids, fr, sp
    base["cfg_expect"] = np.array([cfg.n_mels, cfg.d_model, cfg.n_layers, cfg.n_heads, cfg.ff_dim, cfg.conv_kernel,
                                   cfg.sub_channels, cfg.vocab_size, cfg.vocab_size, cfg.pred_hidden,
                                   cfg.pred_rnn_layers, cfg.joint_hidden, cfg.n_mels, cfg.n_fft, cfg.win_length,
                                   cfg.hop_length, cfg.sample_rate, len(cfg.tdt_durations)], np.int32)
    base["mel_pcm"] = oracle.mel(mcfg, oracle.mel_window(m.tensors["preprocessor.featurizer.window"].data, cfg.n_fft),
                                 m.tensors["preprocessor.featurizer.fb"].data.reshape(cfg.n_mels, -1), pcm)
    mp, bp = str(d / "model.gguf"), str(d / "baseline.gguf")
    pm.write_gguf(m, mp)
    pm.write_baseline_gguf(bp, base)
    _FILES[wtype] = (mp, bp)
    return _FILES[wtype]


def _files_eou(tmp_path_factory, wtype):
    """A cache-aware streaming model and its baselines: the mel, the oracle's
    streamed encoder output (stream_encoder_out) and its offline encoder output
    with every frame valid (encoder_out), both [d_model][T']."""
    key = "eou_" + wtype
    if key in _FILES:
        return _FILES[key]
    d = tmp_path_factory.mktemp(f"cpp_{key}")
    cfg = pm.eou_config(d_model=256, n_layers=3, n_heads=4, ff_dim=512, n_mels=64, sub_channels=64)
    m = pm.synthesize(cfg, wtype, heads=False, std=0.05)
    om = oracle.OracleModel(m)
    rng = np.random.default_rng(17)
    T = 137
    mel = rng.standard_normal((cfg.n_mels, T)).astype(np.float32)
    st = oracle.Stream(om)
    outs = [st.step(mel[:, lo:hi], is_last=last) for lo, hi, last in oracle.stream_windows(T, 9, 16, 9)]
    stream = np.concatenate(outs)
    off, _ = om.encoder(mel[None], valid_in=[T])
    mp, bp, sp = str(d / "eou.gguf"), str(d / "baseline_eou.gguf"), str(d / "baseline_eou_stream.gguf")
    pm.write_gguf(m, mp)
    pm.write_baseline_gguf(bp, {"mel": mel, "encoder_out": np.ascontiguousarray(off[0].T)})
    pm.write_baseline_gguf(sp, {"stream_encoder_out": np.ascontiguousarray(stream.T)})
    _FILES[key] = (mp, bp, sp)
    return _FILES[key]


def _files_eou_offline(tmp_path_factory, wtype):
    """The streaming model's offline baselines for Encoder::forward_capture:
    the mel, the oracle's whole-sequence encoder output [d_model][T'] and the
    layer 0 / mid / last captures [T'][d_model], at the forward path's entry
    valid length T - 1 (src/encoder.cpp:30-95)."""
    key = "eou_off_" + wtype
    if key in _FILES:
        return _FILES[key]
    mp, _, _ = _files_eou(tmp_path_factory, wtype)
    d = tmp_path_factory.mktemp(f"cpp_{key}")
    cfg = pm.eou_config(d_model=256, n_layers=3, n_heads=4, ff_dim=512, n_mels=64, sub_channels=64)
    m = pm.synthesize(cfg, wtype, heads=False, std=0.05)
    om = oracle.OracleModel(m)
    rng = np.random.default_rng(23)
    T = 161
    mel = rng.standard_normal((cfg.n_mels, T)).astype(np.float32)
    off, _, cap = om.encoder(mel[None], valid_in=[T - 1], capture=True)
    L = cfg.n_layers
    bp = str(d / "baseline_eou_offline.gguf")
    pm.write_baseline_gguf(bp, {"mel": mel, "encoder_out": np.ascontiguousarray(off[0].T),
                                "enc_layer_0": cap[0][0], "enc_layer_mid": cap[L // 2][0],
                                "enc_layer_last": cap[L - 1][0]})
    _FILES[key] = (mp, bp)
    return _FILES[key]


@pytest.mark.parametrize("wtype", ["f32", "q8_0"])
def test_cpp_encoder_eou(tmp_path_factory, wtype):
    exe = os.path.join(BIN, "test_encoder_eou")
    assert os.path.exists(exe), f"{exe} not built (make -C tests/cpp)"
    mp, bp = _files_eou_offline(tmp_path_factory, wtype)
    env = dict(os.environ, PARAKEET_TEST_GGUF_EOU=mp, PARAKEET_TEST_BASELINE_EOU=bp)
    print(f"[cpp] test_encoder_eou {wtype}", flush=True)
    r = subprocess.run([exe], env=env, capture_output=True, text=True, timeout=120)
    print(r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.parametrize("wtype", ["f32", "q8_0"])
def test_cpp_streaming_encoder(tmp_path_factory, wtype):
    exe = os.path.join(BIN, "test_streaming_encoder")
    assert os.path.exists(exe), f"{exe} not built (make -C tests/cpp)"
    mp, bp, sp = _files_eou(tmp_path_factory, wtype)
    env = dict(os.environ, PARAKEET_TEST_GGUF_EOU=mp, PARAKEET_TEST_BASELINE_EOU=bp,
               PARAKEET_TEST_BASELINE_EOU_STREAM=sp)
    print(f"[cpp] test_streaming_encoder {wtype}", flush=True)
    r = subprocess.run([exe], env=env, capture_output=True, text=True, timeout=120)
    print(r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.parametrize("wtype", ["f32", "q8_0"])
@pytest.mark.parametrize("name", TESTS)
def test_cpp(tmp_path_factory, wtype, name):
    exe = os.path.join(BIN, name)
    assert os.path.exists(exe), f"{exe} not built (make -C tests/cpp)"
    mp, bp = _files(tmp_path_factory, wtype)
    env = dict(os.environ, PARAKEET_TEST_GGUF=mp, PARAKEET_TEST_BASELINE=bp)
    print(f"[cpp] {name} {wtype}", flush=True)
    r = subprocess.run([exe], env=env, capture_output=True, text=True, timeout=120)
    print(r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr

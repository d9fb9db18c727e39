"""Device log-mel front end (pkx_mel_*) against the oracle's restatement of
pk::MelFrontend::compute + build_mel_batch (mel.cpp:99-185, model.cpp:114-146).

Both sides compute in f64 with the reference's f32 roundings and operation
order; they can differ only by the libm ulp of sqrt / pow / log and by the
summation order of the per-feature statistics (f64).  Bar: raw log-mel within
1e-5 absolute, normalised features within 1e-4 absolute (values ~N(0, 1)), and
most values bit-identical.
"""
import numpy as np
import pytest

import oracle
import pk_model as pm

pytestmark = pytest.mark.gpu

N_FFT, HOP, WIN, SR = 512, 160, 400, 16000


@pytest.fixture(scope="module")
def feat():
    return pm.hann_window(WIN), pm.mel_filterbank(SR, N_FFT, 128)


def _ragged(lens, seed=0):
    rng = np.random.default_rng(seed)
    pcm = np.zeros((len(lens), max(max(lens), 1)), np.float32)
    for b, n in enumerate(lens):
        pcm[b, :n] = (rng.standard_normal(n) * 0.1).astype(np.float32)
    return pcm


def _run(gpu, stream, mel, pcm, lens, T_max):
    d_pcm = gpu.DeviceArray.from_numpy(pcm, stream)
    d_out = gpu.DeviceArray((pcm.shape[0], mel.cfg.n_mels, T_max), np.float32)
    T = mel.forward(d_pcm, lens, d_out, T_max, stream=stream)
    out = d_out.numpy(stream)
    d_pcm.free()
    d_out.free()
    return out, T


@pytest.mark.parametrize("per_feature", [False, True])
def test_mel_batch_matches_oracle(gpu, stream, feat, per_feature):
    win, fb = feat
    lens = [16000 * 10, 1, 159, 160, 161, 16000 * 2 + 37, 16000 * 20, 5000, 0]
    print(f"[mel] per_feature={per_feature} lens={lens}", flush=True)
    pcm = _ragged(lens)
    mel = gpu.Mel.create(N_FFT, WIN, HOP, 128, win, fb, per_feature=per_feature)
    cfg = oracle.mel_cfg(per_feature=per_feature)
    T_max = max(oracle.mel_frames(cfg, n) for n in lens) + 3          # extra padding columns
    ref, T_ref = oracle.mel_batch(cfg, oracle.mel_window(win, N_FFT), fb, pcm, lens, T_max)
    got, T = _run(gpu, stream, mel, pcm, lens, T_max)
    assert list(T) == list(T_ref)
    assert np.isfinite(got).all()
    err = np.max(np.abs(got - ref))
    same = float(np.mean(got == ref))
    print(f"[mel] max abs {err:.3e}, bit-identical fraction {same:.4f}", flush=True)
    assert err <= (1e-4 if per_feature else 1e-5)
    assert same >= 0.99
    for b, t in enumerate(T):
        assert np.all(got[b, :, t:] == 0)                               # zero padding to T_max
    mel.close()


def test_mel_other_shapes(gpu, stream):
    """80-mel, no preemphasis, magnitude spectrum, n_fft 256 with a full window."""
    lens = [4000, 2570, 1]
    pcm = _ragged(lens, seed=5)
    win, fb = pm.hann_window(256), pm.mel_filterbank(8000, 256, 80)
    mel = gpu.Mel.create(256, 256, 80, 80, win, fb, preemph=0.0, mag_power=1.0, per_feature=True)
    cfg = oracle.mel_cfg(n_fft=256, hop=80, n_mels=80, per_feature=True, preemph=0.0, mag_power=1.0)
    T_max = max(oracle.mel_frames(cfg, n) for n in lens)
    ref, T_ref = oracle.mel_batch(cfg, oracle.mel_window(win, 256), fb, pcm, lens, T_max)
    got, T = _run(gpu, stream, mel, pcm, lens, T_max)
    assert list(T) == list(T_ref)
    assert np.max(np.abs(got - ref)) <= 1e-4
    mel.close()


def test_mel_from_gguf_equals_create(gpu, stream, tmp_path, feat):
    cfg = pm.Config(d_model=64, n_layers=1, n_heads=2, ff_dim=128, n_mels=128, sub_channels=16, vocab_size=16)
    m = pm.add_featurizer(pm.synthesize(cfg, "f32", heads=False))
    path = str(tmp_path / "mel.gguf")
    pm.write_gguf(m, path)
    a = gpu.Mel.load_gguf(path)
    b = gpu.Mel.from_model(m)
    assert (a.cfg.n_fft, a.cfg.win_length, a.cfg.hop_length, a.cfg.n_mels, a.cfg.per_feature) == \
        (512, 400, 160, 128, 1)
    assert abs(a.cfg.preemph - 0.97) < 1e-7 and abs(a.cfg.log_zero_guard - 2.0 ** -24) < 1e-12
    lens = [16000, 7000]
    pcm = _ragged(lens, seed=9)
    T_max = a.frames(16000)
    ga, _ = _run(gpu, stream, a, pcm, lens, T_max)
    gb, _ = _run(gpu, stream, b, pcm, lens, T_max)
    assert np.array_equal(ga, gb)
    a.close()
    b.close()


def test_mel_rejects_bad_arguments(gpu, stream, feat):
    win, fb = feat
    with pytest.raises(gpu.PkxError, match="n_fft"):
        gpu.Mel.create(1024, 400, 160, 128, win, np.zeros((128, 513), np.float32))
    mel = gpu.Mel.create(N_FFT, WIN, HOP, 128, win, fb)
    pcm = _ragged([16000])
    d_pcm = gpu.DeviceArray.from_numpy(pcm, stream)
    d_out = gpu.DeviceArray((1, 128, 50), np.float32)
    with pytest.raises(gpu.PkxError, match="T_max"):
        mel.forward(d_pcm, [16000], d_out, 50, stream=stream)      # needs 101 frames
    with pytest.raises(gpu.PkxError, match="S_stride"):
        mel.forward(d_pcm, [16001], d_out, 200, stream=stream)
    d_pcm.free()
    d_out.free()
    mel.close()


def test_mel_on_speech_fixtures(gpu, stream, feat):
    """The reference's own audio fixtures (tests/fixtures/clip.wav, speech.wav),
    batched: real speech through the device front end against the oracle."""
    import os
    from test_gpu_cpp import read_wav
    root = os.path.dirname(os.path.abspath(__file__))
    clips = [read_wav(os.path.join(root, "golden", n)) for n in ("clip.wav", "speech.wav")]
    lens = [len(c) for c in clips]
    print(f"[mel] speech fixtures lens={lens}", flush=True)
    pcm = np.zeros((2, max(lens)), np.float32)
    for b, c in enumerate(clips):
        pcm[b, :len(c)] = c
    win, fb = feat
    mel = gpu.Mel.create(N_FFT, WIN, HOP, 128, win, fb)
    cfg = oracle.mel_cfg()
    T_max = max(oracle.mel_frames(cfg, n) for n in lens)
    ref, _ = oracle.mel_batch(cfg, oracle.mel_window(win, N_FFT), fb, pcm, lens, T_max)
    got, T = _run(gpu, stream, mel, pcm, lens, T_max)
    err = np.max(np.abs(got - ref))
    print(f"[mel] speech max abs {err:.3e}, bit-identical {float(np.mean(got == ref)):.4f}", flush=True)
    assert err <= 1e-4
    mel.close()

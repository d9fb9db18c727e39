"""Pins of the oracle's log-mel front end (mel.cpp, fft.cpp, model.cpp:114-146).

The reference's front end is f64 arithmetic with f32 roundings at fixed
points; it is pinned here against numpy's float64 FFT of the same frames
(closed form: the DFT), Parseval, a pure tone's bin, the frame-count formula,
the window centring and the per-feature normalisation invariants.  No fixture
of the reference's own mel output exists (its baselines need NeMo).
"""
import numpy as np
import pytest

import oracle
import pk_model as pm


def numpy_logmel(samples, win_nfft, fb, n_fft=512, hop=160, preemph=0.97, guard=2.0 ** -24):
    """mel.cpp:99-150 restated with numpy's float64 rfft (not the oracle's FFT)."""
    S = len(samples)
    x = samples.astype(np.float64).copy()
    if preemph > 0 and S > 1:
        x[1:] = samples[1:].astype(np.float64) - np.float64(np.float32(preemph)) * samples[:-1].astype(np.float64)
    pad = n_fft // 2
    xp = np.zeros(S + 2 * pad)
    xp[pad:pad + S] = x
    T = 1 + (S + 2 * pad - n_fft) // hop
    frames = np.stack([(xp[t * hop:t * hop + n_fft] * win_nfft.astype(np.float64)).astype(np.float32)
                       for t in range(T)])
    spec = np.fft.rfft(frames.astype(np.float64), axis=1)
    re = spec.real.astype(np.float32).astype(np.float64)
    im = spec.imag.astype(np.float32).astype(np.float64)
    power = re * re + im * im
    return np.log(power @ fb.astype(np.float64).T + np.float64(np.float32(guard))).astype(np.float32).T


@pytest.fixture(scope="module")
def featurizer():
    win = oracle.mel_window(pm.hann_window(400), 512)
    fb = pm.mel_filterbank(16000, 512, 128)
    return win, fb


@pytest.mark.parametrize("n", [64, 256, 512])
def test_rfft_matches_numpy(n):
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    re, im = oracle.rfft(x)
    ref = np.fft.rfft(x.astype(np.float64))
    # only the final f32 rounding of re/im separates them
    assert np.max(np.abs(re - ref.real)) <= 2e-7 * np.max(np.abs(ref))
    assert np.max(np.abs(im - ref.imag)) <= 2e-7 * np.max(np.abs(ref))
    # Parseval on the full spectrum (unnormalised forward transform)
    full = np.fft.fft(x.astype(np.float64))
    assert np.isclose(np.sum(np.abs(full) ** 2), n * np.sum(x.astype(np.float64) ** 2), rtol=1e-10)


def test_window_centre_padding():
    w = np.arange(1, 401, dtype=np.float32)
    out = oracle.mel_window(w, 512)
    assert np.all(out[:56] == 0) and np.all(out[456:] == 0)
    assert np.array_equal(out[56:456], w)
    assert np.array_equal(oracle.mel_window(np.ones(512, np.float32), 512), np.ones(512, np.float32))


def test_frame_count():
    cfg = oracle.mel_cfg()
    for S in [0, 1, 159, 160, 161, 16000, 32037]:
        assert oracle.mel_frames(cfg, S) == (0 if S == 0 else 1 + S // 160)


def test_logmel_matches_numpy_pipeline(featurizer):
    win, fb = featurizer
    rng = np.random.default_rng(1)
    for S in [1, 161, 16000 * 2 + 37]:
        s = (rng.standard_normal(S) * 0.1).astype(np.float32)
        got = oracle.mel(oracle.mel_cfg(per_feature=False), win, fb, s)
        ref = numpy_logmel(s, win, fb)
        assert got.shape == ref.shape == (128, 1 + S // 160)
        assert np.max(np.abs(got - ref)) <= 1e-6


def test_pure_tone_lands_in_its_filter(featurizer):
    win, fb = featurizer
    t = np.arange(16000) / 16000.0
    s = (0.5 * np.sin(2 * np.pi * 1000.0 * t)).astype(np.float32)
    feats = oracle.mel(oracle.mel_cfg(per_feature=False, preemph=0.0), win, fb, s)
    k = int(round(1000.0 * 512 / 16000))                  # FFT bin of 1 kHz
    mid = feats[:, feats.shape[1] // 2]
    assert int(np.argmax(mid)) == int(np.argmax(fb[:, k]))


def test_per_feature_normalisation(featurizer):
    win, fb = featurizer
    S = 16000 * 3 + 100
    s = (np.random.default_rng(2).standard_normal(S) * 0.1).astype(np.float32)
    raw = oracle.mel(oracle.mel_cfg(per_feature=False), win, fb, s)
    nrm = oracle.mel(oracle.mel_cfg(per_feature=True), win, fb, s)
    valid = S // 160                                      # T = valid + 1: the last frame is zeroed
    assert nrm.shape[1] == valid + 1
    assert np.all(nrm[:, valid:] == 0)
    mean = raw[:, :valid].astype(np.float64).mean(1, keepdims=True)
    sd = raw[:, :valid].astype(np.float64).std(1, ddof=1, keepdims=True) + 1e-5
    assert np.max(np.abs(nrm[:, :valid] - (raw[:, :valid] - mean) / sd)) <= 1e-5
    # invariants: zero mean, unit unbiased std (up to the 1e-5 added to std)
    assert np.max(np.abs(nrm[:, :valid].mean(1))) <= 1e-5
    assert np.max(np.abs(nrm[:, :valid].std(1, ddof=1) - 1.0)) <= 1e-3


def test_batch_stacks_per_clip(featurizer):
    win, fb = featurizer
    rng = np.random.default_rng(3)
    lens = [16000, 500, 16000 * 2 + 3, 0]
    pcm = np.zeros((4, max(lens)), np.float32)
    for b, n in enumerate(lens):
        pcm[b, :n] = rng.standard_normal(n) * 0.1
    cfg = oracle.mel_cfg()
    out, T = oracle.mel_batch(cfg, win, fb, pcm, lens)
    assert list(T) == [0 if n == 0 else 1 + n // 160 for n in lens]
    assert out.shape == (4, 128, max(T))
    for b, n in enumerate(lens):
        if n:
            one = oracle.mel(cfg, win, fb, pcm[b, :n])
            assert np.array_equal(out[b, :, :T[b]], one)
        assert np.all(out[b, :, T[b]:] == 0)


def test_filterbank_shape_and_area():
    fb = pm.mel_filterbank(16000, 512, 128)
    assert fb.shape == (128, 257) and np.all(fb >= 0)
    # Slaney normalisation: each triangle has unit area in Hz (the discrete sum
    # approximates it once a filter spans several bins)
    df = 16000 / 512
    area = fb.sum(1) * df
    wide = fb.astype(bool).sum(1) >= 6
    assert np.allclose(area[wide], 1.0, rtol=0.1)
    # filter centres increase monotonically
    assert np.all(np.diff(np.argmax(fb, 1)) >= 0)


def test_pin_detects_planted_mistakes(featurizer):
    """A slip in the front end's arithmetic must fail the numpy pin."""
    win, fb = featurizer
    s = (np.random.default_rng(4).standard_normal(16000) * 0.1).astype(np.float32)
    ref = numpy_logmel(s, win, fb)
    # window not centred (left-aligned)
    bad_win = np.zeros(512, np.float32)
    bad_win[:400] = pm.hann_window(400)
    assert np.max(np.abs(oracle.mel(oracle.mel_cfg(per_feature=False), bad_win, fb, s) - ref)) > 1e-2
    # preemphasis dropped
    assert np.max(np.abs(oracle.mel(oracle.mel_cfg(per_feature=False, preemph=0.0), win, fb, s) - ref)) > 1e-2
    # magnitude instead of power
    assert np.max(np.abs(oracle.mel(oracle.mel_cfg(per_feature=False, mag_power=1.0), win, fb, s) - ref)) > 1e-2

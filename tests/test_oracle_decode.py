"""Pins of the oracle's greedy transducer decode (prediction.cpp, joint.cpp,
tdt.cpp, decode_common.hpp).

The LSTM step is pinned against a float64 numpy restatement of PyTorch's
nn.LSTM cell (gate order i, f, g, o).  The loop control is pinned with
joints whose decisions are fixed by their biases, where the token count,
frames and spans follow in closed form from the rules (duration-0 loops
capped by max_symbols, frame advance by the predicted duration, RNNT
advance on blank); the confidence against its closed form.  No reference
vectors exist for this path (its baselines need NeMo)."""
import numpy as np
import pytest

import oracle
import pk_model as pm


def _model(durations=(0, 1, 2, 3, 4), layers=2):
    cfg = pm.Config(d_model=32, n_layers=1, n_heads=2, ff_dim=64, n_mels=64, sub_channels=16, vocab_size=12,
                    joint_hidden=16, pred_hidden=24, pred_rnn_layers=layers, tdt_durations=tuple(durations))
    return cfg, pm.add_prediction(pm.synthesize(cfg, "f32", heads=True))


def test_lstm_step_matches_numpy():
    cfg, m = _model()
    tr = oracle.Transducer(m)
    H, L = cfg.pred_hidden, cfg.pred_rnn_layers
    rng = np.random.default_rng(0)
    h = rng.standard_normal((L, H)).astype(np.float32)
    c = rng.standard_normal((L, H)).astype(np.float32)
    for token, sos in ((5, False), (0, True)):
        g, ho, co = tr.lstm_step(token, sos, h, c)
        x = np.zeros(H) if sos else m.tensors["decoder.prediction.embed.weight"].data.reshape(-1, H)[token]
        x = x.astype(np.float64)
        sig = lambda v: 1.0 / (1.0 + np.exp(-v))
        for l in range(L):
            t = lambda n: m.tensors[f"decoder.prediction.dec_rnn.lstm.{n}_l{l}"].data.astype(np.float64)
            z = t("weight_ih").reshape(4 * H, H) @ x + t("bias_ih") + t("weight_hh").reshape(4 * H, H) @ h[l] + \
                t("bias_hh")
            i, f, gg, o = z[:H], z[H:2 * H], z[2 * H:3 * H], z[3 * H:]
            cn = sig(f) * c[l] + sig(i) * np.tanh(gg)
            hn = sig(o) * np.tanh(cn)
            assert np.max(np.abs(co[l] - cn)) <= 1e-5 and np.max(np.abs(ho[l] - hn)) <= 1e-5
            x = hn
        assert np.array_equal(g, ho[L - 1])


def _scripted(durations, tok, dur_idx, margin=8.0):
    """A joint whose output is its bias: token `tok` and duration index `dur_idx` win by `margin`."""
    cfg, m = _model(durations)
    Vp = cfg.vocab_size + 1 + len(durations)
    w = m.tensors["joint.joint_net.2.weight"]
    m.tensors["joint.joint_net.2.weight"] = pm.Tensor(w.gtype, w.shape, np.zeros_like(w.data))
    b = np.zeros(Vp, np.float32)
    b[tok] = margin
    if durations:
        b[cfg.vocab_size + 1 + dur_idx] = margin
    m.tensors["joint.joint_net.2.bias"] = pm.Tensor(0, (Vp,), b)
    return cfg, oracle.Transducer(m)


@pytest.mark.parametrize("max_symbols", [1, 3, 10])
def test_tdt_duration_zero_emits_max_symbols_per_frame(max_symbols):
    cfg, tr = _scripted((0, 1, 2, 3, 4), tok=3, dur_idx=0)
    T = 7
    ids, fr, cf, sp = tr.greedy(np.zeros((T, cfg.d_model), np.float32), (0, 1, 2, 3, 4), max_symbols=max_symbols)
    assert len(ids) == T * max_symbols and np.all(ids == 3) and np.all(sp == 0)
    assert np.array_equal(fr, np.repeat(np.arange(T), max_symbols))


def test_tdt_blank_advances_by_duration():
    cfg, tr = _scripted((0, 1, 2, 3, 4), tok=12, dur_idx=2)          # blank, duration 2
    ids, *_ = tr.greedy(np.zeros((9, cfg.d_model), np.float32), (0, 1, 2, 3, 4))
    assert len(ids) == 0
    cfg, tr = _scripted((0, 1, 2, 3, 4), tok=4, dur_idx=3)           # token 4, duration 3
    ids, fr, cf, sp = tr.greedy(np.zeros((10, cfg.d_model), np.float32), (0, 1, 2, 3, 4))
    assert list(fr) == [0, 3, 6, 9] and np.all(sp == 3) and np.all(ids == 4)
    # confidence closed form: p = 1 / (1 + (N-1) e^-margin), conf = (N p - 1) / (N - 1)
    N = cfg.vocab_size + 1
    p = 1.0 / (1.0 + (N - 1) * np.exp(-8.0))
    assert np.allclose(cf, (N * p - 1) / (N - 1), atol=1e-6)


@pytest.mark.parametrize("max_symbols", [1, 4])
def test_rnnt_rules(max_symbols):
    cfg, tr = _scripted((), tok=5, dur_idx=0)
    T = 6
    ids, fr, cf, sp = tr.greedy(np.zeros((T, cfg.d_model), np.float32), (), max_symbols=max_symbols)
    assert len(ids) == T * max_symbols and np.all(sp == 1)
    assert np.array_equal(fr, np.repeat(np.arange(T), max_symbols))
    cfg, tr = _scripted((), tok=12, dur_idx=0)                          # always blank
    assert len(tr.greedy(np.zeros((T, cfg.d_model), np.float32), ())[0]) == 0

"""Greedy transducer decode on the device (pkx_transducer_greedy) against the
oracle's restatement of the per-item loops (tdt.cpp / the RNNT loop, which
transducer_batch.cpp reproduces in lockstep).  Bar: identical token ids,
frames and spans per item (the argmax decisions), confidence within 1e-5.
The joint's output weights are scaled up so that the decisions have margins
far above f32 rounding (the device sums the products in another order)."""
import numpy as np
import pytest

import oracle
import pk_model as pm

pytestmark = pytest.mark.gpu


def _model(durations, seed=7, qtype="f32"):
    cfg = pm.Config(d_model=128, n_layers=1, n_heads=2, ff_dim=256, n_mels=64, sub_channels=16, vocab_size=40,
                    joint_hidden=128, pred_hidden=64, pred_rnn_layers=2, tdt_durations=tuple(durations))
    m = pm.add_prediction(pm.synthesize(cfg, qtype, heads=True, seed=seed), seed=seed)
    for n in ("joint.joint_net.2.weight", "joint.joint_net.2.bias"):
        t = m.tensors[n]
        m.tensors[n] = pm.Tensor(t.gtype, t.shape, (t.data * 60.0).astype(np.float32))
    return cfg, m


@pytest.mark.parametrize("kind,max_symbols,qtype", [("tdt", 10, "f32"), ("tdt", 2, "f32"), ("rnnt", 10, "f32"),
                                                     ("rnnt", 1, "f32"), ("tdt", 10, "q8_0")])
def test_greedy_decode_matches_oracle(gpu, stream, kind, max_symbols, qtype):
    durations = (0, 1, 2, 3, 4) if kind == "tdt" else ()
    cfg, m = _model(durations, qtype=qtype)
    gm = gpu.Model.from_tensors(m)
    tr = oracle.Transducer(m)
    rng = np.random.default_rng(11)
    T_valid = [60, 1, 37, 0, 59, 12]
    B, T_max = len(T_valid), 60
    enc = rng.standard_normal((B, T_max, cfg.d_model)).astype(np.float32)
    print(f"[decode] {kind} max_symbols={max_symbols} T={T_valid}", flush=True)
    d_enc = gpu.DeviceArray.from_numpy(enc, stream)
    got = gm.transducer_greedy(d_enc, T_valid, durations=durations, max_symbols=max_symbols, stream=stream)
    total = 0
    for b in range(B):
        ids, fr, cf, sp = tr.greedy(enc[b, :T_valid[b]], durations=durations, max_symbols=max_symbols)
        g_ids, g_fr, g_cf, g_sp = got[b]
        total += len(ids)
        assert np.array_equal(g_ids, ids), (b, g_ids[:20], ids[:20])
        assert np.array_equal(g_fr, fr) and np.array_equal(g_sp, sp)
        assert np.max(np.abs(g_cf - cf), initial=0.0) <= 1e-5
        assert np.all(ids < cfg.vocab_size)
    print(f"[decode] {total} tokens identical", flush=True)
    assert total > 20
    d_enc.free()


def test_decode_rejects_bad_arguments(gpu, stream):
    cfg, m = _model((0, 1, 2, 3, 4))
    gm = gpu.Model.from_tensors(m)
    enc = np.zeros((1, 4, cfg.d_model), np.float32)
    d_enc = gpu.DeviceArray.from_numpy(enc, stream)
    with pytest.raises(gpu.PkxError, match="durations"):
        gm.transducer_greedy(d_enc, [4], durations=(0, 1), stream=stream)
    with pytest.raises(gpu.PkxError, match="T_valid"):
        gm.transducer_greedy(d_enc, [5], durations=(0, 1, 2, 3, 4), stream=stream)
    d_enc.free()


def test_greedy_decode_more_items_than_one_pass(gpu, stream):
    """21 items: the matvec kernels take the items in passes of 16 through LDS
    (the second pass reuses the weight rows the wave holds in registers)."""
    durations = (0, 1, 2, 3, 4)
    cfg, m = _model(durations, seed=9)
    gm = gpu.Model.from_tensors(m)
    tr = oracle.Transducer(m)
    rng = np.random.default_rng(21)
    T_valid = [int(t) for t in rng.integers(0, 41, 21)]
    B, T_max = len(T_valid), 40
    enc = rng.standard_normal((B, T_max, cfg.d_model)).astype(np.float32)
    print(f"[decode] B={B} T={T_valid}", flush=True)
    d_enc = gpu.DeviceArray.from_numpy(enc, stream)
    got = gm.transducer_greedy(d_enc, T_valid, durations=durations, max_symbols=10, stream=stream)
    total = 0
    for b in range(B):
        ids, fr, cf, sp = tr.greedy(enc[b, :T_valid[b]], durations=durations, max_symbols=10)
        g_ids, g_fr, g_cf, g_sp = got[b]
        total += len(ids)
        assert np.array_equal(g_ids, ids), (b, g_ids[:20], ids[:20])
        assert np.array_equal(g_fr, fr) and np.array_equal(g_sp, sp)
        assert np.max(np.abs(g_cf - cf), initial=0.0) <= 1e-5
    print(f"[decode] {total} tokens identical over {B} items", flush=True)
    assert total > 20
    d_enc.free()


def test_greedy_decode_production_shape(gpu, stream):
    """The 0.6B decoder's shape: 2-layer LSTM of 640 (K = 1280 in the gate
    products, several register slabs per lane), joint 640, 1024 tokens + blank +
    5 durations (1030 outputs, not a multiple of 4), encoder width 1024, and 17
    ragged items (more than one LDS pass of 16)."""
    durations = (0, 1, 2, 3, 4)
    cfg = pm.Config(d_model=1024, n_layers=1, n_heads=8, ff_dim=256, n_mels=64, sub_channels=16, vocab_size=1024,
                    joint_hidden=640, pred_hidden=640, pred_rnn_layers=2, tdt_durations=durations)
    m = pm.add_prediction(pm.synthesize(cfg, "q8_0", heads=True, seed=640), seed=640)
    for n in ("joint.joint_net.2.weight", "joint.joint_net.2.bias"):
        t = m.tensors[n]
        m.tensors[n] = pm.Tensor(t.gtype, t.shape, (t.data * 60.0).astype(np.float32))
    gm = gpu.Model.from_tensors(m)
    tr = oracle.Transducer(m)
    rng = np.random.default_rng(17)
    T_valid = [125, 125, 3, 0, 64, 125, 99, 1, 125, 17, 80, 125, 42, 125, 7, 110, 125]
    B, T_max = len(T_valid), 125
    enc = rng.standard_normal((B, T_max, cfg.d_model)).astype(np.float32)
    print(f"[decode] production shape B={B} T={T_valid}", flush=True)
    d_enc = gpu.DeviceArray.from_numpy(enc, stream)
    got = gm.transducer_greedy(d_enc, T_valid, durations=durations, max_symbols=10, stream=stream)
    total = 0
    for b in range(B):
        ids, fr, cf, sp = tr.greedy(enc[b, :T_valid[b]], durations=durations, max_symbols=10)
        g_ids, g_fr, g_cf, g_sp = got[b]
        total += len(ids)
        assert np.array_equal(g_ids, ids), (b, g_ids[:20], ids[:20])
        assert np.array_equal(g_fr, fr) and np.array_equal(g_sp, sp)
        # The joint output is scaled x60 here, so logits reach a few hundred,
        # where one f32 ulp is 1.5e-5-3e-5; device and oracle sum the K = 640
        # products in different orders, so each logit may differ by a few ulps.
        # The confidence (N p - 1) / (N - 1), p = 1 / sum exp(l - l_max), moves
        # by at most ~2 max|dl| * p: 5e-5 covers two ulps at |l| ~ 256.
        assert np.max(np.abs(g_cf - cf), initial=0.0) <= 5e-5
    print(f"[decode] {total} tokens identical over {B} items", flush=True)
    assert total > 100
    d_enc.free()
    gm.close()

"""GGUF v3 loading (the on-disk contract) and per-item output compaction on the
GPU path: a model read from a GGUF file gives bit-identical encoder outputs to
the same tensors uploaded one by one."""
import numpy as np
import pytest

import pk_model as pm

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("wtype", ["q8_0", "f16", "q4_k", "f32"])
def test_gguf_roundtrip_encoder(gpu, stream, tmp_path, wtype):
    cfg = pm.Config(d_model=256, n_layers=2, n_heads=4, ff_dim=512, n_mels=64, sub_channels=32, vocab_size=63,
                    joint_hidden=64, pred_hidden=64)
    m = pm.synthesize(cfg, wtype, bn_random=True)
    path = tmp_path / f"m_{wtype}.gguf"
    pm.write_gguf(m, str(path))
    a = gpu.Model.from_tensors(m)
    b = gpu.Model.load_gguf(path)
    assert a.precision == b.precision == (0 if wtype == "f32" else 1)
    assert b.has_ctc and b.has_joint
    rng = np.random.default_rng(1)
    B, T = 2, 150
    mel = rng.normal(0, 1, (B, cfg.n_mels, T)).astype(np.float32)
    d_mel = gpu.DeviceArray.from_numpy(mel, stream)
    Tp = gpu.subsampled_len(T)
    ya = gpu.DeviceArray((B, Tp, cfg.d_model), np.float32)
    yb = gpu.DeviceArray((B, Tp, cfg.d_model), np.float32)
    a.encoder_forward(d_mel, [150, 90], ya, stream=stream)
    b.encoder_forward(d_mel, [150, 90], yb, stream=stream)
    assert np.array_equal(ya.numpy(stream), yb.numpy(stream))


def test_compact_channels_first(gpu, stream):
    rng = np.random.default_rng(2)
    B, T, D = 3, 37, 96
    x = rng.normal(0, 1, (B, T, D)).astype(np.float32)
    valid = np.array([37, 20, 1], dtype=np.int32)
    offs = np.concatenate([[0], np.cumsum(valid * D)[:-1]]).astype(np.int64)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dv = gpu.DeviceArray.from_numpy(valid, stream)
    do = gpu.DeviceArray.from_numpy(offs, stream)
    out = gpu.DeviceArray((int(valid.sum()) * D,), np.float32)
    gpu.check(gpu.lib().pkx_compact_channels_first(dx.ptr, B, T, D, dv.ptr, do.ptr, out.ptr, stream.handle))
    got = out.numpy(stream)
    for b in range(B):
        ref = x[b, :valid[b]].T.reshape(-1)                    # [D][valid] channels-first (encoder.cpp:158-166)
        assert np.array_equal(got[offs[b]:offs[b] + valid[b] * D], ref)

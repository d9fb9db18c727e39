"""pkx_tdt_joint_argmax_noalloc (the entry point that allocates nothing: its
scratch is a fixed per-GPU device array) against pkx_tdt_joint_argmax on the
same inputs: logits, token and duration argmaxes bit-identical, on two calls
in a row (the second with fewer frames, so it runs on the scratch the first
left behind), then a size beyond the array refused with a message.  On a
freshly built model the no-allocation call runs first, before any allocating
joint call has grown the model's workspace, and the device's free memory
(hipMemGetInfo) is the same before and after it."""
import numpy as np
import pytest

import pk_model as pm

pytestmark = pytest.mark.gpu


def test_noalloc_joint_matches_allocating_joint(gpu, stream):
    cfg = pm.Config(d_model=512, n_layers=1, n_heads=8, ff_dim=256, n_mels=64, sub_channels=16, vocab_size=1024,
                    joint_hidden=640, pred_hidden=640, pred_rnn_layers=1, tdt_durations=(0, 1, 2, 3, 4))
    gm = gpu.Model.from_tensors(pm.synthesize(cfg, "q8_0", heads=True, seed=5), gpu.PREC_F16)
    V = cfg.vocab_size + 1 + len(cfg.tdt_durations)
    rng = np.random.default_rng(6)
    g = gpu.DeviceArray.from_numpy(rng.normal(0, 1, cfg.pred_hidden).astype(np.float32), stream)
    for M in (1500, 77):
        enc = rng.normal(0, 1, (M, cfg.d_model)).astype(np.float32)
        de = gpu.DeviceArray.from_numpy(enc, stream)
        bufs = [(gpu.DeviceArray((M, V), np.float32), gpu.DeviceArray((M,), np.int32),
                 gpu.DeviceArray((M,), np.int32)) for _ in range(2)]
        stream.sync()
        outs = []
        for noalloc, (dl, dt, dd) in zip((True, False), bufs):
            print(f"[noalloc] M={M} noalloc={noalloc}", flush=True)
            if noalloc:
                free0, _ = gpu.mem_info()
                gm.tdt_joint_noalloc(de, M, g, dl, dt, dd, stream)
                stream.sync()
                free1, _ = gpu.mem_info()
                assert free1 == free0, f"device free memory changed across the call: {free0} -> {free1}"
            else:
                gm.tdt_joint(de, M, g, dl, dt, dd, stream)
            outs.append((dl.numpy(stream), dt.numpy(stream), dd.numpy(stream)))
        for a, b in zip(outs[0], outs[1]):
            assert np.array_equal(a, b)
        print(f"[noalloc] M={M}: logits, tokens and durations bit-identical; no device memory taken", flush=True)
    # beyond the fixed array: refused before any launch
    big = (4 << 20) // cfg.joint_hidden
    dummy = gpu.DeviceArray((1, cfg.d_model), np.float32)
    with pytest.raises(gpu.PkxError, match="fixed scratch array"):
        gm.tdt_joint_noalloc(dummy, big, g, dummy, dummy, dummy, stream)
    gm.close()

"""Device quantisers (pkx_quantize) and the GGUF quantiser (pkx_quantize_gguf,
the parakeet-cli quantize command, examples/cli/main.cpp:322-426) against the
oracle's restatements of ggml's quantize_row_q8_0_ref / quantize_row_q4_K_ref.
Bar: identical bytes (both compute the same f32 operations in the same order,
without contraction); the quantised GGUF loads and runs bit-identically to the
same tensors quantised by the oracle and uploaded directly."""
import os
import struct
import subprocess

import numpy as np
import pytest

import oracle
import pk_model as pm

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def oracle_quant(gtype, x):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.zeros(oracle.lib().orc_row_bytes(gtype, x.size), np.uint8)
    assert oracle.lib().orc_quantize(gtype, oracle.fp(x), out.ctypes.data, x.size) == 0
    return out


@pytest.mark.parametrize("gtype,rows,per_row", [(8, 64, 1024), (8, 3, 96), (12, 48, 1024), (12, 5, 256)])
def test_quantize_matches_oracle_bytes(gpu, stream, gtype, rows, per_row):
    rng = np.random.default_rng(rows * 7 + gtype)
    x = (rng.standard_normal((rows, per_row)) * rng.uniform(0.001, 0.1, (rows, 1))).astype(np.float32)
    x[0, :256] = 0.0                                        # zero blocks
    x[1, :32] = 0.125                                       # a constant block
    if gtype == 8:
        x[2, :32] = 0.0
        x[2, 0], x[2, 1], x[2, 2] = 127.0, 2.5, -2.5       # ties of roundf
    print(f"[quant] gtype={gtype} rows={rows} per_row={per_row}", flush=True)
    bpr = (per_row // 32) * 34 if gtype == 8 else (per_row // 256) * 144
    d_x = gpu.DeviceArray.from_numpy(x, stream)
    d_y = gpu.DeviceArray((rows * bpr,), np.uint8)
    gpu.quantize(gtype, d_x, d_y, rows, per_row, stream=stream)
    got = d_y.numpy(stream)
    ref = oracle_quant(gtype, x)
    assert got.shape == ref.shape
    diff = np.count_nonzero(got != ref)
    print(f"[quant] differing bytes {diff} of {ref.size}", flush=True)
    assert diff == 0


def _kv_section(path):
    """Raw bytes of a GGUF's KV section (from the header to the tensor infos)."""
    with open(path, "rb") as f:
        data = f.read()
    _, _, n_t, n_kv = struct.unpack_from("<IIQQ", data, 0)
    pos = 24

    def skip_val(t, pos):
        sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}
        if t == 8:
            n, = struct.unpack_from("<Q", data, pos)
            return pos + 8 + n
        if t == 9:
            et, n = struct.unpack_from("<IQ", data, pos)
            pos += 12
            for _ in range(n):
                pos = skip_val(et, pos)
            return pos
        return pos + sizes[t]

    for _ in range(n_kv):
        n, = struct.unpack_from("<Q", data, pos)
        pos += 8 + n
        t, = struct.unpack_from("<I", data, pos)
        pos = skip_val(t, pos + 4)
    return data[24:pos], n_t


@pytest.mark.parametrize("qtype,gtype", [("q8_0", 8), ("q4_k", 12)])
def test_quantize_gguf_roundtrip(gpu, stream, tmp_path, qtype, gtype):
    cfg = pm.Config(d_model=256, n_layers=2, n_heads=4, ff_dim=512, n_mels=64, sub_channels=32, vocab_size=63,
                    joint_hidden=64, pred_hidden=64)
    m = pm.add_featurizer(pm.synthesize(cfg, "f32", bn_random=True))
    src, dst = str(tmp_path / "f32.gguf"), str(tmp_path / f"{qtype}.gguf")
    pm.write_gguf(m, src)
    nq, nk, ns = gpu.quantize_gguf(src, dst, qtype)
    # the oracle's expectation: allowlisted 2-D f32 tensors with ne0 % block == 0
    block = 32 if gtype == 8 else 256
    want = {}
    skipped = 0
    for name, t in m.tensors.items():
        if pm.quantizable(name) and t.gtype == 0 and len(t.shape) == 2 and min(t.shape) >= 32:
            if t.shape[-1] % block == 0:
                want[name] = pm.Tensor(gtype, t.shape, oracle_quant(gtype, t.data))
            else:
                skipped += 1
    print(f"[quant] {qtype}: quantized {nq} kept {nk} skipped {ns} (expected {len(want)} / {skipped})", flush=True)
    assert (nq, nk, ns) == (len(want), len(m.tensors) - len(want), skipped)
    assert _kv_section(src)[0] == _kv_section(dst)[0]       # every KV pair verbatim
    # the quantised file loads and runs exactly like the oracle-quantised tensors uploaded directly
    m2 = pm.Model(cfg, {n: want.get(n, t) for n, t in m.tensors.items()})
    a = gpu.Model.load_gguf(dst)
    b = gpu.Model.from_tensors(m2)
    assert a.precision == b.precision == 1
    rng = np.random.default_rng(3)
    B, T = 2, 150
    mel = rng.normal(0, 1, (B, cfg.n_mels, T)).astype(np.float32)
    d_mel = gpu.DeviceArray.from_numpy(mel, stream)
    Tp = gpu.subsampled_len(T)
    ya = gpu.DeviceArray((B, Tp, cfg.d_model), np.float32)
    yb = gpu.DeviceArray((B, Tp, cfg.d_model), np.float32)
    a.encoder_forward(d_mel, [150, 90], ya, stream=stream)
    b.encoder_forward(d_mel, [150, 90], yb, stream=stream)
    assert np.array_equal(ya.numpy(stream), yb.numpy(stream))
    # the front end tensors and keys survive too
    mel_a = gpu.Mel.load_gguf(dst)
    assert mel_a.cfg.n_mels == cfg.n_mels
    mel_a.close()


def test_quantize_cli(gpu, tmp_path):
    cfg = pm.Config(d_model=128, n_layers=1, n_heads=2, ff_dim=256, n_mels=64, sub_channels=16, vocab_size=31)
    m = pm.synthesize(cfg, "f32", heads=False)
    src, dst = str(tmp_path / "in.gguf"), str(tmp_path / "out.gguf")
    pm.write_gguf(m, src)
    exe = os.path.join(ROOT, "parakeet.cpp_amd", "build", "pkx-quantize")
    r = subprocess.run([exe, src, dst, "Q8_0"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "quantized" in r.stdout and os.path.exists(dst)
    r = subprocess.run([exe, src, dst, "q6_k"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "unsupported type" in r.stderr

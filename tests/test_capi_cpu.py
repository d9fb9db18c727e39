"""C-ABI surface checks that need no GPU: every declaration in include/pkx.h is
exported by libpkx.so, the host-side length arithmetic matches the oracle,
and invalid arguments come back as error codes with a message (no exception
crosses the boundary).  The library is exercised in a subprocess so this
process never loads a HIP runtime."""
import os
import re
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import oracle
import pk_model as pm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "parakeet.cpp_amd", "build", "libpkx.so")
HDR = os.path.join(ROOT, "include", "pkx.h")


def declared():
    txt = open(HDR).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(pkx_[a-z0-9_]+)\s*\(", txt)))


def test_header_declarations_are_exported():
    if not os.path.exists(LIB):
        pytest.skip("libpkx.so not built")
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (pkx_[a-z0-9_]+)$", out, flags=re.M))
    decl = declared()
    assert len(decl) >= 30
    missing = [d for d in decl if d not in exported]
    assert not missing, missing


def _run(code):
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([os.path.join(ROOT, "parakeet.cpp_amd", "python"),
                                         os.path.join(ROOT, "oracle"), env.get("PYTHONPATH", "")])
    r = subprocess.run([sys.executable, "-c", textwrap.dedent(code)], capture_output=True, text=True, env=env,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def test_length_arithmetic_matches_oracle():
    if not os.path.exists(LIB):
        pytest.skip("libpkx.so not built")
    out = _run("""
        import pkx
        L = pkx.lib()
        print(L.pkx_abi_version())
        print(' '.join(str(L.pkx_subsampled_len(t)) for t in range(1, 3001)))
        print(' '.join(str(L.pkx_valid_out_len(t, -1)) for t in range(1, 3001)))
        print(' '.join(str(L.pkx_valid_out_len(3000, v)) for v in range(0, 3001, 7)))
    """).split("\n")
    assert out[0] == "3"
    assert [int(x) for x in out[1].split()] == [oracle.subsampled_len(t) for t in range(1, 3001)]
    assert [int(x) for x in out[2].split()] == [oracle.valid_out_len(t) for t in range(1, 3001)]
    assert [int(x) for x in out[3].split()] == [oracle.valid_out_len(3000, v) for v in range(0, 3001, 7)]


def test_invalid_arguments_return_errors():
    if not os.path.exists(LIB):
        pytest.skip("libpkx.so not built")
    out = _run("""
        import ctypes as C, pkx
        L = pkx.lib()
        h = C.c_void_p()
        bad = pkx.Config(100, 2, 3, 64, 9, 80, 16, 0, 10, 0)        # d_model % n_heads != 0
        print(L.pkx_model_create(C.byref(bad), 0, C.byref(h)), L.pkx_last_error().decode())
        bad2 = pkx.Config(64, 2, 4, 64, 8, 80, 16, 0, 10, 0)         # even conv kernel
        print(L.pkx_model_create(C.byref(bad2), 0, C.byref(h)), L.pkx_last_error().decode())
        ok = pkx.Config(64, 1, 4, 128, 9, 24, 16, 0, 31, 5)
        print(L.pkx_model_create(C.byref(ok), 0, C.byref(h)), repr(L.pkx_last_error().decode()))
        ne = (C.c_int64 * 2)(64, 64)
        buf = (C.c_uint8 * 100)()
        print(L.pkx_model_set_tensor(h, b"x.weight", 0, 2, ne, buf, 100), L.pkx_last_error().decode())
        print(L.pkx_model_set_tensor(h, b"x.weight", 77, 2, ne, buf, 100), L.pkx_last_error().decode())
        print(L.pkx_model_create(None, 0, C.byref(h)), L.pkx_last_error().decode())
        print(L.pkx_model_free(h))
    """).strip().split("\n")
    assert out[0].startswith("1 ") and "n_heads" in out[0]
    assert out[1].startswith("1 ") and "odd" in out[1]
    assert out[2] == "0 ''"
    assert out[3].startswith("1 ") and "expected 16384 bytes" in out[3]
    assert out[4].startswith("1 ") and "unsupported" in out[4]
    assert out[5].startswith("1 ") and "null" in out[5]
    assert out[6] == "0"


def _read_gguf(path):
    """Minimal independent GGUF v3 reader (test side) for the writer's output."""
    import struct
    f = open(path, "rb")
    rd = lambda fmt: struct.unpack("<" + fmt, f.read(struct.calcsize("<" + fmt)))
    magic, ver, nt, nkv = rd("IIQQ")
    assert magic == 0x46554747 and ver == 3

    def rstr():
        (n,) = rd("Q")
        return f.read(n).decode()

    def rval(t):
        if t == 4: return rd("I")[0]
        if t == 5: return rd("i")[0]
        if t == 6: return rd("f")[0]
        if t == 7: return bool(rd("B")[0])
        if t == 8: return rstr()
        if t == 9:
            et, n = rd("IQ")
            return [rval(et) for _ in range(n)]
        raise ValueError(t)
    kv = {}
    for _ in range(nkv):
        k = rstr()
        (t,) = rd("I")
        kv[k] = rval(t)
    infos = []
    for _ in range(nt):
        name = rstr()
        (nd,) = rd("I")
        ne = rd("Q" * nd)
        gt, off = rd("IQ")
        infos.append((name, ne, gt, off))
    base = (f.tell() + 31) // 32 * 32
    return kv, infos, base, f


def test_gguf_writer_layout(tmp_path):
    cfg = pm.Config(d_model=64, n_layers=1, n_heads=4, ff_dim=128, n_mels=24, sub_channels=16, vocab_size=31,
                    joint_hidden=32, pred_hidden=32)
    m = pm.synthesize(cfg, "q8_0")
    path = tmp_path / "m.gguf"
    pm.write_gguf(m, str(path))
    kv, infos, base, f = _read_gguf(path)
    assert kv["general.architecture"] == "parakeet"
    assert kv["parakeet.encoder.d_model"] == 64 and kv["parakeet.encoder.n_layers"] == 1
    assert kv["parakeet.tdt.durations"] == [0, 1, 2, 3, 4]
    names = {i[0]: i for i in infos}
    assert set(names) == set(m.tensors)
    for name, t in m.tensors.items():
        _, ne, gt, off = names[name]
        assert tuple(ne) == t.ne and gt == t.gtype and off % 32 == 0
        f.seek(base + off)
        assert f.read(t.nbytes()) == np.ascontiguousarray(t.data).tobytes()


def test_gguf_loader_rejects_unknown_conv_norm(tmp_path):
    """conv_norm_type other than batch_norm / layer_norm (conformer.cpp:279-280)
    is refused from the KV block, before any device allocation."""
    if not os.path.exists(LIB):
        pytest.skip("libpkx.so not built")
    cfg = pm.Config(d_model=64, n_layers=1, n_heads=4, ff_dim=128, n_mels=24, sub_channels=16, vocab_size=31,
                    joint_hidden=32, pred_hidden=32)
    m = pm.synthesize(cfg, "f32")
    path = tmp_path / "s.gguf"
    # later duplicate keys overwrite earlier ones in the reader's map
    pm.write_gguf(m, str(path), extra_kv=[("parakeet.encoder.conv_norm_type", 8, "group_norm")])
    out = _run(f"""
        import ctypes as C, pkx
        L = pkx.lib()
        h = C.c_void_p()
        print(L.pkx_model_load_gguf({str(path)!r}.encode(), -1, C.byref(h)), L.pkx_last_error().decode())
    """).strip()
    assert out.startswith("1 ") and "conv_norm_type" in out


def test_gguf_kv_reader(tmp_path):
    """pkx_gguf_read_kv hands every KV pair of a GGUF header to the visitor in
    file order with the GGUF type codes and raw values (the KV half of
    gguf_init_from_file that ModelLoader::load reads, src/model_loader.cpp:99-156);
    host-only, no device call."""
    if not os.path.exists(LIB):
        pytest.skip("libpkx.so not built")
    cfg = pm.Config(d_model=64, n_layers=1, n_heads=2, ff_dim=128, n_mels=16, sub_channels=8, vocab_size=7,
                    joint_hidden=16, pred_hidden=16)
    path = str(tmp_path / "kv.gguf")
    pm.write_gguf(pm.synthesize(cfg, "f32"), path)
    out = _run(f"""
        import ctypes as C, pkx
        L = pkx.lib()
        class S(C.Structure):
            _fields_ = [("s", C.c_char_p), ("n", C.c_size_t)]
        FN = C.CFUNCTYPE(None, C.c_void_p, C.c_char_p, C.c_int, C.c_int, C.c_uint64, C.c_void_p)
        L.pkx_gguf_read_kv.argtypes = [C.c_char_p, FN, C.c_void_p]
        seen = []
        def visit(user, key, t, et, n, data):
            if et == 8:
                arr = C.cast(data, C.POINTER(S))
                val = [arr[i].s[:arr[i].n].decode() for i in range(n)]
            elif et == 4:
                val = list(C.cast(data, C.POINTER(C.c_uint32))[:n])
            elif et == 5:
                val = list(C.cast(data, C.POINTER(C.c_int32))[:n])
            elif et == 6:
                val = list(C.cast(data, C.POINTER(C.c_float))[:n])
            elif et == 7:
                val = [bool(b) for b in C.cast(data, C.POINTER(C.c_uint8))[:n]]
            else:
                val = None
            seen.append((key.decode(), t, et, n, val))
        cb = FN(visit)
        assert L.pkx_gguf_read_kv({path!r}.encode(), cb, None) == 0
        for k, t, et, n, v in seen:
            print(repr((k, t, et, n, v if n < 20 else (v[:3], len(v)))))
        assert L.pkx_gguf_read_kv(b"/nonexistent.gguf", cb, None) != 0
        print("ERR", L.pkx_last_error().decode())
    """)
    rows = [eval(l) for l in out.splitlines() if l.startswith("(")]
    kv = {r[0]: r for r in rows}
    assert [r[0] for r in rows][:2] == ["general.architecture", "parakeet.arch"]
    assert kv["parakeet.arch"][4] == ["hybrid_tdt_ctc"] and kv["parakeet.arch"][1] == 8
    assert kv["parakeet.encoder.d_model"][1:] == (4, 4, 1, [64])
    assert kv["parakeet.encoder.xscaling"][4] == [False]
    assert kv["parakeet.tdt.durations"][1:] == (9, 5, 5, [0, 1, 2, 3, 4])
    assert abs(kv["parakeet.preprocessor.preemph"][4][0] - 0.97) < 1e-7
    assert kv["parakeet.tokenizer.pieces"][1:4] == (9, 8, 7)
    assert kv["parakeet.tokenizer.pieces"][4] == ["<unk>", "\u2581t1", "\u2581t2", "\u2581t3", "\u2581t4",
                                                  "\u2581t5", "\u2581t6"]
    assert "cannot open" in out.splitlines()[-1]

"""ctypes binding of libpkx.so (include/pkx.h) for tests, smoke and bench.

The native library owns device memory and streams through its own HIP
runtime, so no other GPU framework needs to be loaded in the same process.
Importing this module never falls back to anything: if libpkx.so is missing
or fails to load, it raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG, "build", "libpkx.so")

PREC_AUTO, PREC_F32, PREC_F16 = -1, 0, 1
MASK_BATCHED, MASK_SCALAR = 0, 1
PROF_FAMILIES = ["subsampling", "layernorm", "gemm_ffn", "gemm_qkv", "gemm_pos", "attention",
                 "gemm_out", "gemm_pw1_glu", "dwconv", "gemm_pw2", "pos_enc"]

_vp = C.c_void_p
_f = C.POINTER(C.c_float)
_ip = C.POINTER(C.c_int)


class PkxError(RuntimeError):
    pass


class MelConfig(C.Structure):
    _fields_ = [("n_fft", C.c_int), ("win_length", C.c_int), ("hop_length", C.c_int), ("n_mels", C.c_int),
                ("per_feature", C.c_int), ("preemph", C.c_float), ("mag_power", C.c_float),
                ("log_zero_guard", C.c_float)]


class Config(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("d_model", "n_layers", "n_heads", "ff_dim", "conv_kernel",
                                        "n_mels", "sub_channels", "xscaling", "vocab_size",
                                        "n_durations", "conv_ln", "causal_sub", "conv_causal",
                                        "att_limited", "att_left", "att_right", "stream_chunk_first",
                                        "stream_chunk", "stream_pre_cache", "stream_cache_len",
                                        "stream_valid_out_len", "stream_drop_extra")]


SIGS = {
    "pkx_abi_version": ([], C.c_int),
    "pkx_last_error": ([], C.c_char_p),
    "pkx_device_count": ([_ip], C.c_int),
    "pkx_malloc": ([C.POINTER(_vp), C.c_size_t], C.c_int),
    "pkx_free": ([_vp], C.c_int),
    "pkx_memcpy_h2d": ([_vp, _vp, C.c_size_t, _vp], C.c_int),
    "pkx_memcpy_d2h": ([_vp, _vp, C.c_size_t, _vp], C.c_int),
    "pkx_memcpy_d2d": ([_vp, _vp, C.c_size_t, _vp], C.c_int),
    "pkx_stream_create": ([C.POINTER(_vp)], C.c_int),
    "pkx_stream_destroy": ([_vp], C.c_int),
    "pkx_stream_synchronize": ([_vp], C.c_int),
    "pkx_event_create": ([C.POINTER(_vp)], C.c_int),
    "pkx_event_destroy": ([_vp], C.c_int),
    "pkx_event_record": ([_vp, _vp], C.c_int),
    "pkx_event_elapsed_ms": ([_f, _vp, _vp], C.c_int),
    "pkx_model_load_gguf": ([C.c_char_p, C.c_int, C.POINTER(_vp)], C.c_int),
    "pkx_model_create": ([C.POINTER(Config), C.c_int, C.POINTER(_vp)], C.c_int),
    "pkx_model_set_tensor": ([_vp, C.c_char_p, C.c_int, C.c_int, C.POINTER(C.c_int64), _vp,
                              C.c_size_t], C.c_int),
    "pkx_model_finalize": ([_vp], C.c_int),
    "pkx_model_free": ([_vp], C.c_int),
    "pkx_model_info": ([_vp, C.POINTER(Config), _ip, _ip, _ip], C.c_int),
    "pkx_subsampled_len": ([C.c_int], C.c_int),
    "pkx_valid_out_len": ([C.c_int, C.c_int], C.c_int),
    "pkx_encoder_forward": ([_vp, _vp, C.c_int, C.c_int, _ip, C.c_int, _vp, _ip, _ip, _vp, _vp],
                            C.c_int),
    "pkx_compact_channels_first": ([_vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp], C.c_int),
    "pkx_subsampling_forward": ([_vp, _vp, C.c_int, C.c_int, _ip, C.c_int, _vp, _ip, _ip, _vp],
                                C.c_int),
    "pkx_conformer_layer_forward": ([_vp, C.c_int, _vp, C.c_int, C.c_int, _ip, _vp, _vp, _vp, _vp],
                                    C.c_int),
    "pkx_relpos_attention_forward": ([_vp, C.c_int, _vp, C.c_int, C.c_int, _ip, _vp, _vp, _vp], C.c_int),
    "pkx_conv_module_forward": ([_vp, C.c_int, _vp, C.c_int, C.c_int, _ip, _vp, _vp], C.c_int),
    "pkx_ctc_forward": ([_vp, _vp, C.c_int64, _vp, _vp, _vp], C.c_int),
    "pkx_tdt_joint_argmax": ([_vp, _vp, C.c_int64, _vp, _vp, _vp, _vp, _vp], C.c_int),
    "pkx_tdt_joint_argmax_noalloc": ([_vp, _vp, C.c_int64, _vp, _vp, _vp, _vp, _vp], C.c_int),
    "pkx_dequantize": ([C.c_int, _vp, _vp, C.c_int64, _vp], C.c_int),
    "pkx_linear": ([C.c_int, C.c_int, C.c_int, C.c_int, _vp, C.c_size_t, _vp, _vp, C.c_int64, _vp,
                    _vp], C.c_int),
    "pkx_linear_residual": ([C.c_int, C.c_int, C.c_int, C.c_int, _vp, C.c_size_t, _vp, _vp, C.c_int64,
                             C.c_float, _vp, _vp], C.c_int),
    "pkx_mem_info": ([C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)], C.c_int),
    "pkx_layernorm": ([_vp, _vp, _vp, _vp, C.c_int64, C.c_int, C.c_float, _vp], C.c_int),
    "pkx_rel_pos_encoding": ([C.c_int, C.c_int, _vp, _vp], C.c_int),
    "pkx_mel_create": ([C.POINTER(MelConfig), _vp, C.c_int, _vp, C.POINTER(_vp)], C.c_int),
    "pkx_mel_load_gguf": ([C.c_char_p, C.POINTER(_vp)], C.c_int),
    "pkx_mel_free": ([_vp], C.c_int),
    "pkx_mel_info": ([_vp, C.POINTER(MelConfig)], C.c_int),
    "pkx_mel_frames": ([_vp, C.c_int], C.c_int),
    "pkx_mel_forward": ([_vp, _vp, C.c_int, C.c_int64, _ip, _vp, C.c_int, _ip, _vp], C.c_int),
    "pkx_quantize": ([C.c_int, _vp, _vp, C.c_int64, C.c_int64, _vp], C.c_int),
    "pkx_transducer_greedy": ([_vp, _vp, C.c_int, C.c_int, _ip, C.POINTER(C.c_int32), C.c_int, C.c_int, C.c_int,
                               C.c_int, C.POINTER(C.c_int32), C.POINTER(C.c_int32), _f, C.POINTER(C.c_int32), _ip,
                               _vp], C.c_int),
    "pkx_quantize_gguf": ([C.c_char_p, C.c_char_p, C.c_int, _ip, _ip, _ip], C.c_int),
    "pkx_streaming_create": ([_vp, C.c_int, C.c_int, _vp, C.POINTER(_vp)], C.c_int),
    "pkx_streaming_free": ([_vp], C.c_int),
    "pkx_streaming_reset": ([_vp, _vp], C.c_int),
    "pkx_streaming_info": ([_vp, _ip, _ip, _ip, _ip, _ip], C.c_int),
    "pkx_streaming_chunk_len": ([_vp, C.c_int], C.c_int),
    "pkx_streaming_step": ([_vp, _vp, C.c_int, C.c_int, _vp, _ip, _vp], C.c_int),
    "pkx_model_set_profiling": ([_vp, C.c_uint, C.c_int], C.c_int),
    "pkx_model_profile_read": ([_vp, C.POINTER(C.c_double), C.POINTER(C.c_int64)], C.c_int),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise PkxError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise PkxError(lib().pkx_last_error().decode())


def device_count() -> int:
    n = C.c_int(0)
    check(lib().pkx_device_count(C.byref(n)))
    return n.value


def _sh(stream):
    return stream.handle if stream is not None else None


def _iptr(a):
    if a is None:
        return None
    return a.ctypes.data_as(_ip)


class DeviceArray:
    """A device allocation with a numpy-like shape/dtype (no arithmetic)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = _vp()
        check(lib().pkx_malloc(C.byref(p), max(self.nbytes, 16)))
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a, stream=None):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a, stream)
        return d

    def upload(self, a, stream=None):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        check(lib().pkx_memcpy_h2d(self.ptr, a.ctypes.data, self.nbytes, _sh(stream)))

    def numpy(self, stream=None):
        out = np.empty(self.shape, dtype=self.dtype)
        check(lib().pkx_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes, _sh(stream)))
        return out

    def free(self):
        if self.ptr:
            lib().pkx_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = _vp()
        check(lib().pkx_stream_create(C.byref(p)))
        self.handle = p.value

    def sync(self):
        check(lib().pkx_stream_synchronize(self.handle))

    def __del__(self):
        try:
            if self.handle:
                lib().pkx_stream_destroy(self.handle)
        except Exception:
            pass


class Event:
    def __init__(self):
        p = _vp()
        check(lib().pkx_event_create(C.byref(p)))
        self.handle = p.value

    def record(self, stream):
        check(lib().pkx_event_record(self.handle, stream.handle if stream else None))

    def elapsed_ms(self, stop) -> float:
        ms = C.c_float(0)
        check(lib().pkx_event_elapsed_ms(C.byref(ms), self.handle, stop.handle))
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                lib().pkx_event_destroy(self.handle)
        except Exception:
            pass


def dequantize(gtype, raw_dev: DeviceArray, n, out: DeviceArray, stream=None):
    check(lib().pkx_dequantize(gtype, raw_dev.ptr, out.ptr, n, _sh(stream)))


def linear(precision, gtype, N, K, w_raw: np.ndarray, x: DeviceArray, M, y: DeviceArray,
           bias: DeviceArray = None, stream=None):
    w_raw = np.ascontiguousarray(w_raw)
    check(lib().pkx_linear(precision, gtype, N, K, w_raw.ctypes.data, w_raw.nbytes,
                           bias.ptr if bias is not None else None, x.ptr, M, y.ptr, _sh(stream)))


def linear_residual(precision, gtype, N, K, w_raw: np.ndarray, x: DeviceArray, M, y: DeviceArray, alpha=1.0,
                    bias: DeviceArray = None, stream=None):
    """y += alpha * (x . W^T + bias) on the encoder's residual-product kernels."""
    w_raw = np.ascontiguousarray(w_raw)
    check(lib().pkx_linear_residual(precision, gtype, N, K, w_raw.ctypes.data, w_raw.nbytes,
                                    bias.ptr if bias is not None else None, x.ptr, M, alpha, y.ptr, _sh(stream)))


def mem_info():
    """(free, total) device memory in bytes."""
    f, t = C.c_size_t(0), C.c_size_t(0)
    check(lib().pkx_mem_info(C.byref(f), C.byref(t)))
    return f.value, t.value


def layernorm(x: DeviceArray, g: DeviceArray, b: DeviceArray, y: DeviceArray, M, D, eps=1e-5,
              stream=None):
    check(lib().pkx_layernorm(x.ptr, g.ptr, b.ptr, y.ptr, M, D, eps, _sh(stream)))


def rel_pos_encoding(T, D, out: DeviceArray, stream=None):
    check(lib().pkx_rel_pos_encoding(T, D, out.ptr, _sh(stream)))


def subsampled_len(T):
    return lib().pkx_subsampled_len(T)


class Model:
    """A device-resident encoder (pkx_model handle)."""

    def __init__(self, handle):
        self.handle = handle
        cfg = Config()
        prec, hc, hj = C.c_int(), C.c_int(), C.c_int()
        check(lib().pkx_model_info(handle, C.byref(cfg), C.byref(prec), C.byref(hc), C.byref(hj)))
        self.cfg = cfg
        self.precision = prec.value
        self.has_ctc = bool(hc.value)
        self.has_joint = bool(hj.value)

    @classmethod
    def from_tensors(cls, model, precision=PREC_AUTO):
        """Upload a pk_model.Model (verbatim names, GGUF byte layout)."""
        c = model.cfg
        cfg = Config(c.d_model, c.n_layers, c.n_heads, c.ff_dim, c.conv_kernel, c.n_mels,
                     c.sub_channels, int(c.xscaling), c.vocab_size, len(c.tdt_durations))
        cfg.att_left, cfg.att_right = -1, -1
        if getattr(c, "streaming", False):
            cfg.conv_ln = int(c.conv_norm_type == "layer_norm")
            cfg.causal_sub = int(bool(c.causal_downsampling))
            cfg.conv_causal = int(bool(c.conv_causal))
            cfg.att_limited = int(c.att_context_style == "chunked_limited" and c.att_context_right >= 0)
            cfg.att_left, cfg.att_right = c.att_context_left, c.att_context_right
            cfg.stream_chunk_first, cfg.stream_chunk = c.stream_chunk_size[0], c.stream_chunk_size[-1]
            cfg.stream_pre_cache = c.stream_pre_encode_cache_size[-1]
            cfg.stream_cache_len = c.stream_last_channel_cache_size
            cfg.stream_valid_out_len = c.stream_valid_out_len
            cfg.stream_drop_extra = c.stream_drop_extra_pre_encoded
        h = _vp()
        check(lib().pkx_model_create(C.byref(cfg), precision, C.byref(h)))
        try:
            for name, t in model.tensors.items():
                ne = (C.c_int64 * len(t.ne))(*t.ne)
                data = np.ascontiguousarray(t.data)
                check(lib().pkx_model_set_tensor(h, name.encode(), t.gtype, len(t.ne), ne,
                                                 data.ctypes.data, data.nbytes))
            check(lib().pkx_model_finalize(h))
        except Exception:
            lib().pkx_model_free(h)
            raise
        return cls(h.value)

    @classmethod
    def load_gguf(cls, path, precision=PREC_AUTO):
        h = _vp()
        check(lib().pkx_model_load_gguf(str(path).encode(), precision, C.byref(h)))
        return cls(h.value)

    def close(self):
        if self.handle:
            lib().pkx_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- hot path ---------------------------------------------------------------
    def encoder_forward(self, mel: DeviceArray, valid_T, out: DeviceArray, mask_mode=MASK_BATCHED,
                        capture: DeviceArray = None, stream=None):
        B, F, T = mel.shape
        vt = None if valid_T is None else np.ascontiguousarray(valid_T, dtype=np.int32)
        tout = C.c_int(0)
        vo = np.zeros(B, dtype=np.int32)
        check(lib().pkx_encoder_forward(self.handle, mel.ptr, B, T, _iptr(vt), mask_mode, out.ptr,
                                        C.byref(tout), _iptr(vo),
                                        capture.ptr if capture is not None else None, _sh(stream)))
        return tout.value, vo

    def transducer_greedy(self, enc: DeviceArray, T_valid, durations=(), blank_id=None, max_symbols=10,
                          cap=None, stream=None):
        """enc [B][T_max][D] f32 on the device -> per item (ids, frames, conf, span)."""
        B, T_max, _ = enc.shape
        cap = cap or T_max * max_symbols
        blank = self.cfg.vocab_size if blank_id is None else blank_id
        tv = np.ascontiguousarray(T_valid, dtype=np.int32)
        du = np.ascontiguousarray(durations, dtype=np.int32)
        ids, fr, sp = (np.zeros((B, cap), np.int32) for _ in range(3))
        cf = np.zeros((B, cap), np.float32)
        cnt = np.zeros(B, np.int32)
        i32 = C.POINTER(C.c_int32)
        check(lib().pkx_transducer_greedy(self.handle, enc.ptr, B, T_max, _iptr(tv), du.ctypes.data_as(i32),
                                          len(du), blank, max_symbols, cap, ids.ctypes.data_as(i32),
                                          fr.ctypes.data_as(i32), cf.ctypes.data_as(_f), sp.ctypes.data_as(i32),
                                          _iptr(cnt), _sh(stream)))
        return [(ids[b, :cnt[b]], fr[b, :cnt[b]], cf[b, :cnt[b]], sp[b, :cnt[b]]) for b in range(B)]

    def subsampling_forward(self, mel: DeviceArray, valid_T, out: DeviceArray,
                            mask_mode=MASK_BATCHED, stream=None):
        B, F, T = mel.shape
        vt = None if valid_T is None else np.ascontiguousarray(valid_T, dtype=np.int32)
        tout = C.c_int(0)
        vo = np.zeros(B, dtype=np.int32)
        check(lib().pkx_subsampling_forward(self.handle, mel.ptr, B, T, _iptr(vt), mask_mode, out.ptr,
                                            C.byref(tout), _iptr(vo), _sh(stream)))
        return tout.value, vo

    def conformer_layer(self, layer, x: DeviceArray, valid, out: DeviceArray,
                        conv_out: DeviceArray = None, stream=None, pos_emb: DeviceArray = None):
        """pos_emb: the caller's [2T-1][d_model] f32 table, or None for rel_pos_encoding(T, d_model)."""
        B, T, D = x.shape
        v = None if valid is None else np.ascontiguousarray(valid, dtype=np.int32)
        check(lib().pkx_conformer_layer_forward(self.handle, layer, x.ptr, B, T, _iptr(v),
                                                pos_emb.ptr if pos_emb is not None else None, out.ptr,
                                                conv_out.ptr if conv_out is not None else None,
                                                _sh(stream)))

    def relpos_attention(self, layer, x: DeviceArray, valid, out: DeviceArray, stream=None,
                         pos_emb: DeviceArray = None):
        B, T, D = x.shape
        v = None if valid is None else np.ascontiguousarray(valid, dtype=np.int32)
        check(lib().pkx_relpos_attention_forward(self.handle, layer, x.ptr, B, T, _iptr(v),
                                                 pos_emb.ptr if pos_emb is not None else None, out.ptr,
                                                 _sh(stream)))

    def conv_module(self, layer, c: DeviceArray, valid, out: DeviceArray, stream=None):
        B, T, D = c.shape
        v = None if valid is None else np.ascontiguousarray(valid, dtype=np.int32)
        check(lib().pkx_conv_module_forward(self.handle, layer, c.ptr, B, T, _iptr(v), out.ptr,
                                            _sh(stream)))

    def ctc(self, enc: DeviceArray, M, logprobs: DeviceArray, argmax: DeviceArray, stream=None):
        check(lib().pkx_ctc_forward(self.handle, enc.ptr, M, logprobs.ptr, argmax.ptr, _sh(stream)))

    def tdt_joint(self, enc: DeviceArray, M, g: DeviceArray, logits: DeviceArray, tok: DeviceArray,
                  dur: DeviceArray, stream=None):
        check(lib().pkx_tdt_joint_argmax(self.handle, enc.ptr, M, g.ptr, logits.ptr, tok.ptr, dur.ptr,
                                         _sh(stream)))

    def tdt_joint_noalloc(self, enc: DeviceArray, M, g: DeviceArray, logits: DeviceArray, tok: DeviceArray,
                          dur: DeviceArray, stream=None):
        """pkx_tdt_joint_argmax_noalloc: the same joint on the library's fixed per-GPU scratch."""
        check(lib().pkx_tdt_joint_argmax_noalloc(self.handle, enc.ptr, M, g.ptr, logits.ptr, tok.ptr, dur.ptr,
                                                 _sh(stream)))

    def set_profiling(self, families=True, stride=1):
        """families: True (all), False/None (off), or an iterable of PROF_FAMILIES names;
        stride: time every stride-th launch of those families."""
        if families is True:
            mask = (1 << len(PROF_FAMILIES)) - 1
        elif not families:
            mask = 0
        else:
            mask = 0
            for f in families:
                mask |= 1 << PROF_FAMILIES.index(f)
        check(lib().pkx_model_set_profiling(self.handle, mask, int(stride)))

    def profile(self):
        ms = (C.c_double * len(PROF_FAMILIES))()
        n = (C.c_int64 * len(PROF_FAMILIES))()
        check(lib().pkx_model_profile_read(self.handle, ms, n))
        return {f: (ms[i], n[i]) for i, f in enumerate(PROF_FAMILIES)}


class Streaming:
    """Cache-aware streaming encoder (pkx_streaming handle): pk::StreamingEncoder
    for n_streams streams advanced together."""

    def __init__(self, model: "Model", n_streams=1, max_window=25, stream=None):
        self.model = model                     # kept alive: the handle points into it
        h = _vp()
        check(lib().pkx_streaming_create(model.handle, int(n_streams), int(max_window), _sh(stream), C.byref(h)))
        self.handle = h.value
        self.n_streams = int(n_streams)
        v = [C.c_int() for _ in range(5)]
        check(lib().pkx_streaming_info(self.handle, *[C.byref(x) for x in v]))
        self.chunk_first, self.chunk, self.pre_cache, self.valid_out_len, _ = (x.value for x in v)

    @property
    def step_num(self):
        v = C.c_int()
        check(lib().pkx_streaming_info(self.handle, None, None, None, None, C.byref(v)))
        return v.value

    def reset(self, stream=None):
        check(lib().pkx_streaming_reset(self.handle, _sh(stream)))

    def chunk_len(self, n):
        return lib().pkx_streaming_chunk_len(self.handle, int(n))

    def step(self, mel: DeviceArray, out: DeviceArray, is_last=False, stream=None):
        """mel [S][n_mels][n] -> out [S][chunk_len][D] (device); returns the kept frame count."""
        S, F, n = mel.shape
        if S != self.n_streams or F != self.model.cfg.n_mels or np.dtype(mel.dtype) != np.float32:
            raise PkxError(f"streaming step: mel must be [{self.n_streams}][{self.model.cfg.n_mels}][n], got {mel.shape}")
        tc = self.chunk_len(n)
        # the device writes one packed [S][tc][D] block, so the row count must be tc exactly
        if tc > 0 and (tuple(out.shape) != (S, tc, self.model.cfg.d_model) or np.dtype(out.dtype) != np.float32):
            raise PkxError(f"streaming step: out must be f32 [{S}][{tc}][{self.model.cfg.d_model}], got {out.shape}")
        nv = C.c_int()
        check(lib().pkx_streaming_step(self.handle, mel.ptr, int(n), 1 if is_last else 0, out.ptr, C.byref(nv),
                                       _sh(stream)))
        return nv.value

    def close(self):
        if self.handle:
            lib().pkx_streaming_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Mel:
    """A device log-mel front end (pkx_mel handle): pk::MelFrontend for a batch."""

    def __init__(self, handle):
        self.handle = handle
        cfg = MelConfig()
        check(lib().pkx_mel_info(handle, C.byref(cfg)))
        self.cfg = cfg

    @classmethod
    def create(cls, n_fft, win_length, hop_length, n_mels, window, fb, preemph=0.97, mag_power=2.0,
               log_zero_guard=2.0 ** -24, per_feature=True):
        window = np.ascontiguousarray(window, dtype=np.float32)
        fb = np.ascontiguousarray(fb, dtype=np.float32)
        cfg = MelConfig(n_fft, win_length, hop_length, n_mels, int(bool(per_feature)), preemph, mag_power,
                        log_zero_guard)
        h = _vp()
        check(lib().pkx_mel_create(C.byref(cfg), window.ctypes.data, len(window), fb.ctypes.data, C.byref(h)))
        return cls(h.value)

    @classmethod
    def from_model(cls, model):
        """From a pk_model.Model carrying the preprocessor config and featurizer tensors."""
        c = model.cfg
        return cls.create(c.n_fft, c.win_length, c.hop_length, c.n_mels,
                          model.tensors["preprocessor.featurizer.window"].data,
                          model.tensors["preprocessor.featurizer.fb"].data.reshape(c.n_mels, -1),
                          c.preemph, c.mag_power, c.log_zero_guard, c.normalize == "per_feature")

    @classmethod
    def load_gguf(cls, path):
        h = _vp()
        check(lib().pkx_mel_load_gguf(str(path).encode(), C.byref(h)))
        return cls(h.value)

    def frames(self, n_samples: int) -> int:
        return lib().pkx_mel_frames(self.handle, int(n_samples))

    def forward(self, pcm: DeviceArray, n_samples, out: DeviceArray, T_max: int, stream=None):
        """pcm [B][S_stride] f32 on the device -> out [B][n_mels][T_max]; returns frames per clip."""
        B, S_stride = pcm.shape
        ns = np.ascontiguousarray(n_samples, dtype=np.int32)
        T_out = np.zeros(B, np.int32)
        check(lib().pkx_mel_forward(self.handle, pcm.ptr, B, S_stride, _iptr(ns), out.ptr, int(T_max),
                                    _iptr(T_out), _sh(stream)))
        return T_out

    def close(self):
        if self.handle:
            lib().pkx_mel_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def quantize(gtype, src: DeviceArray, dst: DeviceArray, n_rows, n_per_row, stream=None):
    """ggml_quantize_chunk on the device: src [n_rows][n_per_row] f32 -> dst (raw blocks)."""
    check(lib().pkx_quantize(int(gtype), src.ptr, dst.ptr, int(n_rows), int(n_per_row), _sh(stream)))


def quantize_gguf(in_path, out_path, qtype: str):
    """parakeet-cli quantize: returns (quantized, kept, skipped) tensor counts."""
    gt = {"q8_0": 8, "q4_k": 12}[qtype.lower()]
    nq, nk, ns = C.c_int(), C.c_int(), C.c_int()
    check(lib().pkx_quantize_gguf(str(in_path).encode(), str(out_path).encode(), gt, C.byref(nq), C.byref(nk),
                                  C.byref(ns)))
    return nq.value, nk.value, ns.value

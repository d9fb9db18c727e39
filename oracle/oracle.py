"""ctypes binding of the CPU restatement (libpk_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the parity checker; the product never uses it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libpk_oracle.so")

_f = C.POINTER(C.c_float)
_i = C.POINTER(C.c_int)
_i32 = C.POINTER(C.c_int32)


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_row_bytes.restype = C.c_int64
        L.orc_row_bytes.argtypes = [C.c_int, C.c_int64]
        L.orc_dequantize.argtypes = [C.c_int, C.c_void_p, _f, C.c_int64]
        L.orc_quantize.argtypes = [C.c_int, _f, C.c_void_p, C.c_int64]
        L.orc_rel_pos_encoding.argtypes = [C.c_int, C.c_int, _f]
        L.orc_layer_norm.argtypes = [_f, C.c_int64, C.c_int, _f, _f, C.c_float, _f]
        L.orc_linear.argtypes = [_f, C.c_int64, C.c_int, _f, C.c_int, _f, _f]
        L.orc_relpos_attention.argtypes = [C.c_void_p, _f, C.c_int, C.c_int, _f, _i, _f]
        L.orc_conv_module.argtypes = [C.c_void_p, _f, C.c_int, C.c_int, _i, _f]
        L.orc_conformer_layer.argtypes = [C.c_void_p, _f, C.c_int, C.c_int, _f, _i, _f, _f]
        L.orc_valid_out_len.argtypes = [C.c_int, C.c_int]
        L.orc_subsampled_len.argtypes = [C.c_int]
        L.orc_valid_out_len_c.argtypes = [C.c_int, C.c_int, C.c_int]
        L.orc_subsampled_len_c.argtypes = [C.c_int, C.c_int]
        L.orc_stream_new.restype = C.c_void_p
        L.orc_stream_new.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                     C.c_int]
        L.orc_stream_free.argtypes = [C.c_void_p]
        L.orc_stream_reset.argtypes = [C.c_void_p]
        L.orc_stream_step.argtypes = [C.c_void_p, _f, C.c_int, C.c_int, _f]
        L.orc_stream_chunk_len.argtypes = [C.c_void_p, C.c_int]
        L.orc_subsampling.argtypes = [C.c_void_p, _f, C.c_int, C.c_int, C.c_int, _i, C.c_int, _f, _i]
        L.orc_encoder_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, _f, C.c_int,
                                          C.c_int, C.c_int, _i, C.c_int, _f, _i, _f]
        L.orc_ctc_head.argtypes = [_f, C.c_int, C.c_int, _f, _f, C.c_int, _f, _i32]
        L.orc_ctc_greedy.argtypes = [_i32, C.c_int, C.c_int, _i32]
        L.orc_tdt_joint_argmax.argtypes = [_f, C.c_int, C.c_int, _f, _f, C.c_int, _f, C.c_int,
                                           _f, _f, _f, _f, C.c_int, C.c_int, _f, _i32, _i32]
        L.orc_lstm_step.argtypes = [C.c_void_p, C.c_int32, C.c_int, _f, _f, _f, _f, _f]
        L.orc_transducer_greedy.argtypes = [C.c_void_p, _f, C.c_int, _i32, C.c_int, C.c_int, C.c_int, _i32,
                                            _i32, _f, _i32, C.c_int]
        L.orc_mel_window.argtypes = [_f, C.c_int, C.c_int, _f]
        L.orc_mel_frames.argtypes = [C.c_void_p, C.c_int]
        L.orc_rfft.argtypes = [_f, C.c_int, _f, _f]
        L.orc_mel.argtypes = [C.c_void_p, _f, _f, _f, C.c_int, _f]
        L.orc_mel_batch.argtypes = [C.c_void_p, _f, _f, _f, C.c_int, C.c_int, _i, C.c_int, _f, _i]
        _lib = L
    return _lib


def set_threads(n: int):
    lib().orc_set_threads(int(n))


def get_threads() -> int:
    return lib().orc_get_threads()


def fp(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f)


def ip(a):
    if a is None:
        return None
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a.ctypes.data_as(_i)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# --------------------------------------------------------------------------
# Elementary ops
# --------------------------------------------------------------------------

def dequantize(gtype: int, raw: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    raw = np.ascontiguousarray(raw)
    rc = lib().orc_dequantize(gtype, raw.ctypes.data_as(C.c_void_p), fp(out), n)
    if rc:
        raise ValueError(f"orc_dequantize rc={rc}")
    return out


def quantize(gtype: int, x: np.ndarray) -> np.ndarray:
    x = f32(x).reshape(-1)
    nbytes = lib().orc_row_bytes(gtype, x.size)
    out = np.empty(nbytes, dtype=np.uint8)
    rc = lib().orc_quantize(gtype, fp(x), out.ctypes.data_as(C.c_void_p), x.size)
    if rc:
        raise ValueError(f"orc_quantize rc={rc}")
    return out


def rel_pos_encoding(T: int, d: int) -> np.ndarray:
    out = np.empty((2 * T - 1, d), dtype=np.float32)
    lib().orc_rel_pos_encoding(T, d, fp(out))
    return out


def layer_norm(x, g, b, eps=1e-5):
    x = f32(x)
    D = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_layer_norm(fp(x), x.size // D, D, fp(f32(g)), fp(f32(b)), eps, fp(y))
    return y


def linear(x, W, b=None):
    x = f32(x)
    W = f32(W)
    K = x.shape[-1]
    N = W.shape[0]
    M = x.size // K
    y = np.empty(x.shape[:-1] + (N,), dtype=np.float32)
    lib().orc_linear(fp(x), M, K, fp(W), N, fp(f32(b)) if b is not None else None, fp(y))
    return y


# --------------------------------------------------------------------------
# Model-level ops (weights dequantised to f32 once per model)
# --------------------------------------------------------------------------

class OrcLayer(C.Structure):
    _fields_ = [("D", C.c_int), ("H", C.c_int), ("FF", C.c_int), ("K", C.c_int)] + [
        (n, _f) for n in (
            "ff1_ln_g", "ff1_ln_b", "ff1_w1", "ff1_b1", "ff1_w2", "ff1_b2",
            "att_ln_g", "att_ln_b",
            "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "wpos",
            "pos_bias_u", "pos_bias_v",
            "conv_ln_g", "conv_ln_b", "pw1_w", "pw1_b", "dw_w", "dw_b",
            "bn_g", "bn_b", "bn_mean", "bn_var", "pw2_w", "pw2_b",
            "ff2_ln_g", "ff2_ln_b", "ff2_w1", "ff2_b1", "ff2_w2", "ff2_b2",
            "out_ln_g", "out_ln_b")] + [
        (n, C.c_int) for n in ("conv_causal", "conv_ln", "att_limited", "att_left", "att_right")]


class OrcSub(C.Structure):
    _fields_ = [("C", C.c_int), ("D", C.c_int)] + [
        (n, _f) for n in ("w0", "b0", "w2", "b2", "w3", "b3", "w5", "b5", "w6", "b6", "wout", "bout")] + [
        ("causal", C.c_int)]


_LAYER_MAP = {
    "ff1_ln_g": "norm_feed_forward1.weight", "ff1_ln_b": "norm_feed_forward1.bias",
    "ff1_w1": "feed_forward1.linear1.weight", "ff1_b1": "feed_forward1.linear1.bias",
    "ff1_w2": "feed_forward1.linear2.weight", "ff1_b2": "feed_forward1.linear2.bias",
    "att_ln_g": "norm_self_att.weight", "att_ln_b": "norm_self_att.bias",
    "wq": "self_attn.linear_q.weight", "bq": "self_attn.linear_q.bias",
    "wk": "self_attn.linear_k.weight", "bk": "self_attn.linear_k.bias",
    "wv": "self_attn.linear_v.weight", "bv": "self_attn.linear_v.bias",
    "wo": "self_attn.linear_out.weight", "bo": "self_attn.linear_out.bias",
    "wpos": "self_attn.linear_pos.weight",
    "pos_bias_u": "self_attn.pos_bias_u", "pos_bias_v": "self_attn.pos_bias_v",
    "conv_ln_g": "norm_conv.weight", "conv_ln_b": "norm_conv.bias",
    "pw1_w": "conv.pointwise_conv1.weight", "pw1_b": "conv.pointwise_conv1.bias",
    "dw_w": "conv.depthwise_conv.weight", "dw_b": "conv.depthwise_conv.bias",
    "bn_g": "conv.batch_norm.weight", "bn_b": "conv.batch_norm.bias",
    "bn_mean": "conv.batch_norm.running_mean", "bn_var": "conv.batch_norm.running_var",
    "pw2_w": "conv.pointwise_conv2.weight", "pw2_b": "conv.pointwise_conv2.bias",
    "ff2_ln_g": "norm_feed_forward2.weight", "ff2_ln_b": "norm_feed_forward2.bias",
    "ff2_w1": "feed_forward2.linear1.weight", "ff2_b1": "feed_forward2.linear1.bias",
    "ff2_w2": "feed_forward2.linear2.weight", "ff2_b2": "feed_forward2.linear2.bias",
    "out_ln_g": "norm_out.weight", "out_ln_b": "norm_out.bias",
}

_SUB_MAP = {"w0": "conv.0.weight", "b0": "conv.0.bias", "w2": "conv.2.weight", "b2": "conv.2.bias",
            "w3": "conv.3.weight", "b3": "conv.3.bias", "w5": "conv.5.weight", "b5": "conv.5.bias",
            "w6": "conv.6.weight", "b6": "conv.6.bias", "wout": "out.weight", "bout": "out.bias"}


class OracleModel:
    """All tensors of a pk_model.Model dequantised to f32 (numpy, torch shapes)."""

    def __init__(self, model):
        self.cfg = model.cfg
        self.w = {}
        for name, t in model.tensors.items():
            n = int(np.prod(t.shape))
            if t.gtype == 0:
                a = f32(t.data)
            else:
                a = dequantize(t.gtype, t.data, n)
            self.w[name] = a.reshape(t.shape)
        cfg = self.cfg
        self.layers = (OrcLayer * cfg.n_layers)()
        for i in range(cfg.n_layers):
            L = self.layers[i]
            L.D, L.H, L.FF, L.K = cfg.d_model, cfg.n_heads, cfg.ff_dim, cfg.conv_kernel
            for field_name, suffix in _LAYER_MAP.items():
                a = self.w.get(f"encoder.layers.{i}.{suffix}")
                setattr(L, field_name, fp(a) if a is not None else None)
            L.conv_causal = int(bool(getattr(cfg, "conv_causal", False)))
            L.conv_ln = int(getattr(cfg, "conv_norm_type", "batch_norm") == "layer_norm")
            L.att_limited = int(getattr(cfg, "att_context_style", "regular") == "chunked_limited"
                                and getattr(cfg, "att_context_right", -1) >= 0)
            L.att_left = int(getattr(cfg, "att_context_left", -1))
            L.att_right = int(getattr(cfg, "att_context_right", -1))
        self.sub = OrcSub()
        self.sub.C, self.sub.D = cfg.sub_channels, cfg.d_model
        self.sub.causal = int(bool(getattr(cfg, "causal_downsampling", False)))
        for field_name, suffix in _SUB_MAP.items():
            setattr(self.sub, field_name, fp(self.w["encoder.pre_encode." + suffix]))

    def layer_ptr(self, i):
        return C.cast(C.pointer(self.layers[i]), C.c_void_p)

    def relpos_attention(self, i, x, pe, valid):
        x = f32(x)
        B, T, D = x.shape
        out = np.empty_like(x)
        lib().orc_relpos_attention(self.layer_ptr(i), fp(x), B, T, fp(f32(pe)), ip(valid), fp(out))
        return out

    def conv_module(self, i, c, valid):
        c = f32(c)
        B, T, D = c.shape
        out = np.empty_like(c)
        lib().orc_conv_module(self.layer_ptr(i), fp(c), B, T, ip(valid), fp(out))
        return out

    def conformer_layer(self, i, x, pe, valid, want_conv=False):
        x = f32(x)
        B, T, D = x.shape
        out = np.empty_like(x)
        conv = np.empty_like(x) if want_conv else None
        lib().orc_conformer_layer(self.layer_ptr(i), fp(x), B, T, fp(f32(pe)), ip(valid), fp(out),
                                  fp(conv) if want_conv else None)
        return (out, conv) if want_conv else out

    def subsampling(self, mel, valid_in=None, stage_masks=True):
        mel = f32(mel)
        B, F, T = mel.shape
        Tp = lib().orc_subsampled_len_c(T, self.sub.causal)
        out = np.empty((B, Tp, self.cfg.d_model), dtype=np.float32)
        vo = np.zeros(B, dtype=np.int32)
        lib().orc_subsampling(C.cast(C.pointer(self.sub), C.c_void_p), fp(mel), B, F, T,
                              ip(valid_in) if valid_in is not None else None,
                              1 if stage_masks else 0, fp(out), vo.ctypes.data_as(_i))
        return out, vo

    def encoder(self, mel, valid_in=None, stage_masks=True, capture=False):
        mel = f32(mel)
        B, F, T = mel.shape
        Tp = lib().orc_subsampled_len_c(T, self.sub.causal)
        D = self.cfg.d_model
        out = np.empty((B, Tp, D), dtype=np.float32)
        vo = np.zeros(B, dtype=np.int32)
        cap = np.empty((self.cfg.n_layers, B, Tp, D), dtype=np.float32) if capture else None
        lib().orc_encoder_forward(C.cast(C.pointer(self.sub), C.c_void_p),
                                  C.cast(self.layers, C.c_void_p), self.cfg.n_layers,
                                  1 if self.cfg.xscaling else 0, fp(mel), B, F, T,
                                  ip(valid_in) if valid_in is not None else None,
                                  1 if stage_masks else 0, fp(out), vo.ctypes.data_as(_i),
                                  fp(cap) if capture else None)
        return (out, vo, cap) if capture else (out, vo)

    def ctc(self, enc):
        enc = f32(enc)
        T, D = enc.shape
        W = self.w["ctc_decoder.decoder_layers.0.weight"].reshape(-1, D)
        b = self.w["ctc_decoder.decoder_layers.0.bias"]
        V = W.shape[0]
        lp = np.empty((T, V), dtype=np.float32)
        am = np.empty(T, dtype=np.int32)
        lib().orc_ctc_head(fp(enc), T, D, fp(f32(W)), fp(f32(b)), V, fp(lp), am.ctypes.data_as(_i32))
        return lp, am

    def tdt_joint(self, enc, g):
        enc = f32(enc)
        T, D = enc.shape
        We, be = self.w["joint.enc.weight"], self.w["joint.enc.bias"]
        Wp, bp = self.w["joint.pred.weight"], self.w["joint.pred.bias"]
        Wo, bo = self.w["joint.joint_net.2.weight"], self.w["joint.joint_net.2.bias"]
        Hj, P = We.shape[0], Wp.shape[1]
        n_dur = len(self.cfg.tdt_durations)
        n_tok = Wo.shape[0] - n_dur
        logits = np.empty((T, n_tok + n_dur), dtype=np.float32)
        tok = np.empty(T, dtype=np.int32)
        dur = np.empty(T, dtype=np.int32)
        lib().orc_tdt_joint_argmax(fp(enc), T, D, fp(f32(We)), fp(f32(be)), Hj, fp(f32(g)), P,
                                   fp(f32(Wp)), fp(f32(bp)), fp(f32(Wo)), fp(f32(bo)), n_tok, n_dur,
                                   fp(logits), tok.ctypes.data_as(_i32), dur.ctypes.data_as(_i32))
        return logits, tok, dur


class Stream:
    """StreamingEncoder (streaming_encoder.hpp:33-95) over an OracleModel of a
    streaming configuration: step() takes one mel window [n_mels][n] and
    returns the kept frames [n_valid][D]."""

    def __init__(self, om: OracleModel):
        cfg = om.cfg
        self.om = om
        self.cfg = cfg
        self.chunk_first = int(cfg.stream_chunk_size[0])
        self.chunk = int(cfg.stream_chunk_size[1] if len(cfg.stream_chunk_size) > 1 else 16)
        self.pre_cache = int(cfg.stream_pre_encode_cache_size[1]
                             if len(cfg.stream_pre_encode_cache_size) > 1 else 9)
        self.valid_out_len = int(cfg.stream_valid_out_len)
        self.cache_len = int(cfg.stream_last_channel_cache_size)
        self.h = lib().orc_stream_new(C.cast(C.pointer(om.sub), C.c_void_p), C.cast(om.layers, C.c_void_p),
                                      cfg.n_layers, 1 if cfg.xscaling else 0, cfg.n_mels, self.cache_len,
                                      int(cfg.stream_drop_extra_pre_encoded), self.valid_out_len)

    def reset(self):
        lib().orc_stream_reset(self.h)

    def step(self, mel_window, is_last=False):
        w = f32(mel_window)
        F, n = w.shape
        tc = lib().orc_stream_chunk_len(self.h, n)
        out = np.empty((max(tc, 1), self.cfg.d_model), dtype=np.float32)
        nv = lib().orc_stream_step(self.h, fp(w), n, 1 if is_last else 0, fp(out))
        return out[:nv].copy()

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_stream_free(self.h)
            self.h = None


def stream_windows(T, chunk_first, chunk, pre_cache):
    """The CacheAwareStreamingAudioBuffer chunk schedule (tests/test_streaming_encoder.cpp:68-99):
    (lo, hi, is_last) mel windows, the first without overlap, later ones with
    pre_cache frames of the previous window in front."""
    out = []
    idx, first = 0, True
    while idx < T:
        size = chunk_first if first else chunk
        hi = min(idx + size, T)
        if hi - idx <= 0:
            break
        lo = idx if first else max(0, idx - pre_cache)
        out.append((lo, hi, hi >= T))
        idx += size
        first = False
    return out


def ctc_greedy(argmax, blank_id):
    am = np.ascontiguousarray(argmax, dtype=np.int32)
    out = np.empty(max(1, am.size), dtype=np.int32)
    n = lib().orc_ctc_greedy(am.ctypes.data_as(_i32), am.size, blank_id, out.ctypes.data_as(_i32))
    return out[:n].copy()


def valid_out_len(T, in_valid=-1):
    return lib().orc_valid_out_len(T, in_valid)


def subsampled_len(T):
    return lib().orc_subsampled_len(T)


# ---- log-mel front end (mel.cpp, fft.cpp, model.cpp:114-146) ----------------

class MelCfg(C.Structure):
    _fields_ = [("n_fft", C.c_int), ("hop", C.c_int), ("n_mels", C.c_int), ("per_feature", C.c_int),
                ("preemph", C.c_float), ("mag_power", C.c_float), ("log_guard", C.c_float)]


def mel_cfg(n_fft=512, hop=160, n_mels=128, per_feature=True, preemph=0.97, mag_power=2.0,
            log_guard=2.0 ** -24) -> MelCfg:
    return MelCfg(n_fft, hop, n_mels, int(bool(per_feature)), preemph, mag_power, log_guard)


def mel_window(win: np.ndarray, n_fft: int) -> np.ndarray:
    win = np.ascontiguousarray(win, dtype=np.float32)
    out = np.zeros(n_fft, np.float32)
    lib().orc_mel_window(fp(win), len(win), n_fft, fp(out))
    return out


def mel_frames(cfg: MelCfg, S: int) -> int:
    return lib().orc_mel_frames(C.byref(cfg), int(S))


def rfft(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = len(x)
    re, im = np.zeros(n // 2 + 1, np.float32), np.zeros(n // 2 + 1, np.float32)
    lib().orc_rfft(fp(x), n, fp(re), fp(im))
    return re, im


def mel(cfg: MelCfg, window: np.ndarray, fb: np.ndarray, samples: np.ndarray) -> np.ndarray:
    """MelFrontend::compute for one clip -> feats [n_mels][T] (window: n_fft values)."""
    samples = np.ascontiguousarray(samples, dtype=np.float32)
    T = mel_frames(cfg, len(samples))
    out = np.zeros((cfg.n_mels, T), np.float32)
    if T:
        lib().orc_mel(C.byref(cfg), fp(np.ascontiguousarray(window, np.float32)),
                      fp(np.ascontiguousarray(fb, np.float32)), fp(samples), len(samples), fp(out))
    return out


def mel_batch(cfg: MelCfg, window: np.ndarray, fb: np.ndarray, pcm: np.ndarray, n_samples, T_max=None):
    """build_mel_batch -> ([B][n_mels][T_max] zero-padded, T per clip)."""
    pcm = np.ascontiguousarray(pcm, dtype=np.float32)
    ns = np.ascontiguousarray(n_samples, dtype=np.int32)
    B, S_stride = pcm.shape
    Ts = [mel_frames(cfg, int(s)) for s in ns]
    if T_max is None:
        T_max = max(Ts) if Ts else 0
    out = np.zeros((B, cfg.n_mels, T_max), np.float32)
    T_out = np.zeros(B, np.int32)
    lib().orc_mel_batch(C.byref(cfg), fp(np.ascontiguousarray(window, np.float32)),
                        fp(np.ascontiguousarray(fb, np.float32)), fp(pcm), B, S_stride, ip(ns), T_max,
                        fp(out), T_out.ctypes.data_as(_i))
    return out, T_out


# ---- greedy transducer decode (prediction.cpp, joint.cpp, tdt.cpp) ------------

class TransducerW(C.Structure):
    _fields_ = [("H", C.c_int), ("L", C.c_int), ("V1", C.c_int), ("embed", _f),
                ("w_ih", _f * 4), ("w_hh", _f * 4), ("b_ih", _f * 4), ("b_hh", _f * 4),
                ("Hj", C.c_int), ("D", C.c_int), ("Vp", C.c_int),
                ("jenc_w", _f), ("jenc_b", _f), ("jpred_w", _f), ("jpred_b", _f), ("jout_w", _f), ("jout_b", _f)]


class Transducer:
    """Prediction net + joint of a pk_model.Model (dequantised to f32)."""

    def __init__(self, model):
        c = model.cfg
        t = model.tensors

        def f32(name):
            tt = t[name]
            if tt.gtype == 0:
                return np.ascontiguousarray(tt.data, dtype=np.float32).reshape(-1)
            n = int(np.prod(tt.shape))
            out = np.zeros(n, np.float32)
            assert lib().orc_dequantize(tt.gtype, np.ascontiguousarray(tt.data).ctypes.data, fp(out), n) == 0
            return out

        self._keep = []

        def keep(a):
            self._keep.append(a)
            return fp(a)

        w = TransducerW()
        w.H, w.L, w.V1 = c.pred_hidden, c.pred_rnn_layers, c.vocab_size + 1
        w.embed = keep(f32("decoder.prediction.embed.weight"))
        for l in range(c.pred_rnn_layers):
            s = "decoder.prediction.dec_rnn.lstm.%s_l" + str(l)
            w.w_ih[l] = keep(f32(s % "weight_ih"))
            w.w_hh[l] = keep(f32(s % "weight_hh"))
            w.b_ih[l] = keep(f32(s % "bias_ih"))
            w.b_hh[l] = keep(f32(s % "bias_hh"))
        w.Hj, w.D = c.joint_hidden, c.d_model
        w.Vp = c.vocab_size + 1 + len(c.tdt_durations)
        w.jenc_w, w.jenc_b = keep(f32("joint.enc.weight")), keep(f32("joint.enc.bias"))
        w.jpred_w, w.jpred_b = keep(f32("joint.pred.weight")), keep(f32("joint.pred.bias"))
        w.jout_w, w.jout_b = keep(f32("joint.joint_net.2.weight")), keep(f32("joint.joint_net.2.bias"))
        self.w = w
        self.cfg = c

    def lstm_step(self, token, is_sos, h, c):
        H, L = self.w.H, self.w.L
        h = np.ascontiguousarray(h, np.float32).reshape(L, H)
        c = np.ascontiguousarray(c, np.float32).reshape(L, H)
        ho, co, g = np.zeros((L, H), np.float32), np.zeros((L, H), np.float32), np.zeros(H, np.float32)
        lib().orc_lstm_step(C.byref(self.w), int(token), int(bool(is_sos)), fp(h), fp(c), fp(ho), fp(co), fp(g))
        return g, ho, co

    def greedy(self, enc, durations=None, blank_id=None, max_symbols=10):
        """enc [T][D] -> (ids, frames, conf, span); durations None/() = RNNT (then the joint's
        output has no duration logits: build the model with tdt_durations=())."""
        enc = np.ascontiguousarray(enc, np.float32)
        T = enc.shape[0]
        durations = np.ascontiguousarray([] if durations is None else durations, np.int32)
        blank = self.cfg.vocab_size if blank_id is None else blank_id
        cap = max(1, T * max_symbols)
        ids, fr, sp = (np.zeros(cap, np.int32) for _ in range(3))
        cf = np.zeros(cap, np.float32)
        n = lib().orc_transducer_greedy(C.byref(self.w), fp(enc), T, durations.ctypes.data_as(_i32),
                                        len(durations), blank, max_symbols, ids.ctypes.data_as(_i32),
                                        fr.ctypes.data_as(_i32), fp(cf), sp.ctypes.data_as(_i32), cap)
        assert n >= 0
        return ids[:n].copy(), fr[:n].copy(), cf[:n].copy(), sp[:n].copy()

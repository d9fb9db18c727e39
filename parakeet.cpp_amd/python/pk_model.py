"""Model container for the FastConformer encoder path: config, tensors under
their verbatim NeMo names, seeded synthetic weights, and GGUF v3 I/O.

The GGUF schema follows the reference converter (docs/conversion.md:21-128):
``parakeet.*`` KV keys and state-dict tensor names, GGUF dims reversed versus
the torch shape.  Quantisation follows the converter allowlist
(docs/quantization.md:93-99): only the encoder FFN/attention linears, the
subsampling output projection and the joint enc/pred projections may be
f16 / q8_0 / q4_K; everything else stays f32.
"""
from __future__ import annotations

import re
import struct
from dataclasses import dataclass, field

import numpy as np

GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K = 0, 1, 8, 12
TYPE_NAMES = {"f32": GGML_F32, "f16": GGML_F16, "q8_0": GGML_Q8_0, "q4_k": GGML_Q4_K}
BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q8_0: (32, 34), GGML_Q4_K: (256, 144)}

QUANT_PATTERNS = [re.compile(p) for p in (
    r"^encoder\.layers\.\d+\.feed_forward[12]\.linear[12]\.weight$",
    r"^encoder\.layers\.\d+\.self_attn\.linear_(q|k|v|out|pos)\.weight$",
    r"^encoder\.pre_encode\.out\.weight$",
    r"^joint\.enc\.weight$",
    r"^joint\.pred\.weight$",
)]


def quantizable(name: str) -> bool:
    return any(p.match(name) for p in QUANT_PATTERNS)


def row_bytes(gtype: int, ne0: int) -> int:
    blk, nb = BLOCK[gtype]
    if ne0 % blk:
        raise ValueError(f"row of {ne0} not a multiple of block {blk}")
    return ne0 // blk * nb


def fnv1a64(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


@dataclass
class Config:
    """Mirror of the encoder-relevant ParakeetConfig fields (src/model_loader.hpp:27-52)."""
    d_model: int = 512
    n_layers: int = 1
    n_heads: int = 8
    ff_dim: int = 2048
    conv_kernel: int = 9
    n_mels: int = 80
    sub_channels: int = 256
    xscaling: bool = False
    vocab_size: int = 1024
    tdt_durations: tuple = (0, 1, 2, 3, 4)
    joint_hidden: int = 640
    pred_hidden: int = 640
    pred_rnn_layers: int = 2
    arch: str = "hybrid_tdt_ctc"
    attn_bias: bool = True          # linear_q/k/v/out biases (110m: yes, 0.6b-v2: no)
    conv_bias: bool = True
    ff_bias: bool = True
    # parakeet.preprocessor.* (src/model_loader.cpp:133-141; NeMo featurizer defaults)
    sample_rate: int = 16000
    n_fft: int = 512
    win_length: int = 400
    hop_length: int = 160
    preemph: float = 0.97
    mag_power: float = 2.0
    normalize: str = "per_feature"
    log_zero_guard: float = 2.0 ** -24
    # cache-aware streaming models (src/model_loader.cpp:110-131; the
    # parakeet_realtime_eou_120m-v1 values are conv_norm_type "layer_norm",
    # causal subsampling and conv, att_context [70, 1] "chunked_limited",
    # chunk [9, 16], pre-encode cache [0, 9], cache 70, valid_out_len 2, drop 2)
    conv_norm_type: str = "batch_norm"
    causal_downsampling: bool = False
    conv_causal: bool = False
    att_context_style: str = "regular"
    att_context_left: int = -1
    att_context_right: int = -1
    stream_chunk_size: tuple = (9, 16)
    stream_shift_size: tuple = (9, 16)
    stream_pre_encode_cache_size: tuple = (0, 9)
    stream_last_channel_cache_size: int = 70
    stream_valid_out_len: int = 2
    stream_drop_extra_pre_encoded: int = 2

    @property
    def d_head(self):
        return self.d_model // self.n_heads

    @property
    def streaming(self):
        return self.att_context_style != "regular"

    def sub_feat(self):
        f = self.n_mels
        ap = 3 if self.causal_downsampling else 2
        for _ in range(3):
            f = (f + ap - 3) // 2 + 1
        return f


def eou_config(**kw) -> "Config":
    """The cache-aware streaming model's architecture (parakeet_realtime_eou_120m-v1:
    512 / 17 layers / 8 heads, ff 2048, conv 9, 256 subsampling channels, 128 mel)."""
    base = dict(d_model=512, n_layers=17, n_heads=8, ff_dim=2048, conv_kernel=9, n_mels=128,
                sub_channels=256, xscaling=False, vocab_size=1026, tdt_durations=(), arch="rnnt",
                conv_norm_type="layer_norm", causal_downsampling=True, conv_causal=True,
                att_context_style="chunked_limited", att_context_left=70, att_context_right=1)
    base.update(kw)
    return Config(**base)


@dataclass
class Tensor:
    gtype: int
    shape: tuple          # torch order (outermost first)
    data: np.ndarray      # f32 -> float32 array; f16 -> uint16; quant -> uint8 raw blocks

    @property
    def ne(self):
        return tuple(reversed(self.shape))

    def nbytes(self):
        return self.data.nbytes


@dataclass
class Model:
    cfg: Config
    tensors: dict = field(default_factory=dict)

    def names(self):
        return list(self.tensors)


def _layer_names(cfg: Config, i: int):
    D, FF, H, K = cfg.d_model, cfg.ff_dim, cfg.n_heads, cfg.conv_kernel
    dk = D // H
    p = f"encoder.layers.{i}."
    out = []
    for nm in ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out"):
        out += [(p + nm + ".weight", (D,), "ln_g"), (p + nm + ".bias", (D,), "ln_b")]
    for ff in ("feed_forward1", "feed_forward2"):
        out += [(p + ff + ".linear1.weight", (FF, D), "w"), (p + ff + ".linear2.weight", (D, FF), "w")]
        if cfg.ff_bias:
            out += [(p + ff + ".linear1.bias", (FF,), "b"), (p + ff + ".linear2.bias", (D,), "b")]
    for lin in ("linear_q", "linear_k", "linear_v", "linear_out"):
        out.append((p + f"self_attn.{lin}.weight", (D, D), "w"))
        if cfg.attn_bias:
            out.append((p + f"self_attn.{lin}.bias", (D,), "b"))
    out += [(p + "self_attn.linear_pos.weight", (D, D), "w"),
            (p + "self_attn.pos_bias_u", (H, dk), "b"),
            (p + "self_attn.pos_bias_v", (H, dk), "b")]
    out += [(p + "conv.pointwise_conv1.weight", (2 * D, D, 1), "w"),
            (p + "conv.depthwise_conv.weight", (D, 1, K), "w"),
            (p + "conv.pointwise_conv2.weight", (D, D, 1), "w"),
            (p + "conv.batch_norm.weight", (D,), "ln_g"),
            (p + "conv.batch_norm.bias", (D,), "ln_b")]
    if cfg.conv_norm_type != "layer_norm":
        out += [(p + "conv.batch_norm.running_mean", (D,), "bn_mean"),
                (p + "conv.batch_norm.running_var", (D,), "bn_var")]
    if cfg.conv_bias:
        out += [(p + "conv.pointwise_conv1.bias", (2 * D,), "b"),
                (p + "conv.depthwise_conv.bias", (D,), "b"),
                (p + "conv.pointwise_conv2.bias", (D,), "b")]
    return out


def tensor_specs(cfg: Config, heads=True):
    """(name, torch shape, role) for every encoder (+ optional head) tensor."""
    C, D = cfg.sub_channels, cfg.d_model
    Fp = cfg.sub_feat()
    pre = "encoder.pre_encode."
    specs = [(pre + "conv.0.weight", (C, 1, 3, 3), "w"), (pre + "conv.0.bias", (C,), "b"),
             (pre + "conv.2.weight", (C, 1, 3, 3), "w"), (pre + "conv.2.bias", (C,), "b"),
             (pre + "conv.3.weight", (C, C, 1, 1), "w"), (pre + "conv.3.bias", (C,), "b"),
             (pre + "conv.5.weight", (C, 1, 3, 3), "w"), (pre + "conv.5.bias", (C,), "b"),
             (pre + "conv.6.weight", (C, C, 1, 1), "w"), (pre + "conv.6.bias", (C,), "b"),
             (pre + "out.weight", (D, C * Fp), "w"), (pre + "out.bias", (D,), "b")]
    for i in range(cfg.n_layers):
        specs += _layer_names(cfg, i)
    if heads:
        V1 = cfg.vocab_size + 1
        Hj, P, ND = cfg.joint_hidden, cfg.pred_hidden, len(cfg.tdt_durations)
        specs += [("ctc_decoder.decoder_layers.0.weight", (V1, D, 1), "w"),
                  ("ctc_decoder.decoder_layers.0.bias", (V1,), "b"),
                  ("joint.enc.weight", (Hj, D), "w"), ("joint.enc.bias", (Hj,), "b"),
                  ("joint.pred.weight", (Hj, P), "w"), ("joint.pred.bias", (Hj,), "b"),
                  ("joint.joint_net.2.weight", (V1 + ND, Hj), "w"),
                  ("joint.joint_net.2.bias", (V1 + ND,), "b")]
    return specs


def _f16_bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def synth_q8_0(rng: np.random.Generator, n: int) -> np.ndarray:
    """q8_0 blocks with d = f16(2.73e-4*(0.5+U)) and q ~ U{-127..127} (weight std ~0.02)."""
    nb = n // 32
    blk = np.empty((nb, 34), dtype=np.uint8)
    d = (2.73e-4 * (0.5 + rng.random(nb))).astype(np.float16).view(np.uint16)
    blk[:, 0] = (d & 0xFF).astype(np.uint8)
    blk[:, 1] = (d >> 8).astype(np.uint8)
    blk[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    return blk.reshape(-1)


def synth_q4_k(rng: np.random.Generator, n: int) -> np.ndarray:
    """q4_K super-blocks with random scale/qs bytes and small finite f16 d, dmin."""
    nb = n // 256
    blk = np.empty((nb, 144), dtype=np.uint8)
    d = (8.2e-5 * (0.75 + 0.5 * rng.random(nb))).astype(np.float16).view(np.uint16)
    dm = (6.1e-4 * (0.75 + 0.5 * rng.random(nb))).astype(np.float16).view(np.uint16)
    blk[:, 0] = (d & 0xFF).astype(np.uint8)
    blk[:, 1] = (d >> 8).astype(np.uint8)
    blk[:, 2] = (dm & 0xFF).astype(np.uint8)
    blk[:, 3] = (dm >> 8).astype(np.uint8)
    blk[:, 4:] = rng.integers(0, 256, size=(nb, 140), dtype=np.uint8)
    return blk.reshape(-1)


def hann_window(n: int) -> np.ndarray:
    """torch.hann_window(n, periodic=False): 0.5 - 0.5 cos(2 pi k / (n - 1))."""
    k = np.arange(n, dtype=np.float64)
    return (0.5 - 0.5 * np.cos(2.0 * np.pi * k / (n - 1))).astype(np.float32)


def _hz_to_mel(f):
    """Slaney's mel scale: linear below 1 kHz (200/3 Hz per mel), logarithmic above."""
    f = np.asarray(f, dtype=np.float64)
    f_sp, min_log_hz = 200.0 / 3, 1000.0
    min_log_mel, logstep = min_log_hz / f_sp, np.log(6.4) / 27.0
    return np.where(f >= min_log_hz, min_log_mel + np.log(np.maximum(f, 1e-10) / min_log_hz) / logstep, f / f_sp)


def _mel_to_hz(m):
    m = np.asarray(m, dtype=np.float64)
    f_sp, min_log_hz = 200.0 / 3, 1000.0
    min_log_mel, logstep = min_log_hz / f_sp, np.log(6.4) / 27.0
    return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), f_sp * m)


def mel_filterbank(sr: int, n_fft: int, n_mels: int, fmin: float = 0.0, fmax=None) -> np.ndarray:
    """Triangular filters on the Slaney mel scale with Slaney area normalisation
    ([n_mels][n_fft/2+1] f32), the featurizer's filterbank (preprocessor.featurizer.fb)."""
    fmax = sr / 2.0 if fmax is None else fmax
    fft_f = np.linspace(0.0, sr / 2.0, n_fft // 2 + 1)
    mel_f = _mel_to_hz(np.linspace(_hz_to_mel(fmin), _hz_to_mel(fmax), n_mels + 2))
    fdiff = np.diff(mel_f)
    ramps = mel_f[:, None] - fft_f[None, :]
    lower = -ramps[:-2] / fdiff[:-1, None]
    upper = ramps[2:] / fdiff[1:, None]
    w = np.maximum(0.0, np.minimum(lower, upper))
    w *= (2.0 / (mel_f[2:n_mels + 2] - mel_f[:n_mels]))[:, None]
    return w.astype(np.float32)


def add_prediction(m: "Model", seed: int = 20261201, std: float = 0.1):
    """The RNNT/TDT prediction network (NeMo RNNTDecoder: Embedding(vocab+1,
    pred_hidden) + stacked LSTM, prediction.hpp:27-50), seeded like synthesize()."""
    c = m.cfg
    P, V1 = c.pred_hidden, c.vocab_size + 1
    specs = [("decoder.prediction.embed.weight", (V1, P))]
    for l in range(c.pred_rnn_layers):
        s = f"decoder.prediction.dec_rnn.lstm.%s_l{l}"
        specs += [(s % "weight_ih", (4 * P, P)), (s % "weight_hh", (4 * P, P)),
                  (s % "bias_ih", (4 * P,)), (s % "bias_hh", (4 * P,))]
    for name, shape in specs:
        rng = np.random.default_rng(seed ^ fnv1a64(name))
        a = rng.normal(0, std if "embed" not in name else 1.0, int(np.prod(shape)))
        m.tensors[name] = Tensor(GGML_F32, shape, np.ascontiguousarray(a, dtype=np.float32).reshape(shape))
    return m


def add_featurizer(m: "Model"):
    """preprocessor.featurizer.window / .fb of the config (the two buffers the
    converter keeps from the checkpoint, docs/conversion.md:110-136)."""
    c = m.cfg
    m.tensors["preprocessor.featurizer.window"] = Tensor(GGML_F32, (c.win_length,), hann_window(c.win_length))
    m.tensors["preprocessor.featurizer.fb"] = Tensor(
        GGML_F32, (1, c.n_mels, c.n_fft // 2 + 1), mel_filterbank(c.sample_rate, c.n_fft, c.n_mels))
    return m


def synthesize(cfg: Config, qtype: str = "f32", seed: int = 20261201, heads: bool = True,
               bn_random: bool = False, std: float = 0.02) -> Model:
    """Seeded random-init weights of the given architecture.

    Linear/conv weights, biases and pos_bias_u/v ~ N(0, std); LayerNorm and
    BatchNorm gains 1 + N(0, std), shifts N(0, std); BatchNorm running stats
    mean 0 / var 1 unless ``bn_random`` (then N(0,0.1) / U(0.5,1.5) to exercise
    the fold).  Allowlisted linears are stored in ``qtype``; q8_0/q4_K draw the
    block fields directly (no f32 master), f16 rounds an f32 draw.
    """
    gq = TYPE_NAMES[qtype]
    m = Model(cfg)
    for name, shape, role in tensor_specs(cfg, heads):
        rng = np.random.default_rng(seed ^ fnv1a64(name))
        n = int(np.prod(shape))
        ne0 = shape[-1] if len(shape) > 1 else n
        if role == "w" and gq != GGML_F32 and quantizable(name) and len(shape) >= 2 \
                and min(shape) >= 32 and ne0 % BLOCK[gq][0] == 0:
            if gq == GGML_F16:
                m.tensors[name] = Tensor(GGML_F16, shape, _f16_bits(rng.normal(0, std, n)))
            elif gq == GGML_Q8_0:
                m.tensors[name] = Tensor(GGML_Q8_0, shape, synth_q8_0(rng, n))
            else:
                m.tensors[name] = Tensor(GGML_Q4_K, shape, synth_q4_k(rng, n))
            continue
        if role == "ln_g":
            a = 1.0 + rng.normal(0, std, n)
        elif role == "bn_mean":
            a = rng.normal(0, 0.1, n) if bn_random else np.zeros(n)
        elif role == "bn_var":
            a = rng.uniform(0.5, 1.5, n) if bn_random else np.ones(n)
        else:
            a = rng.normal(0, std, n)
        m.tensors[name] = Tensor(GGML_F32, shape, np.ascontiguousarray(a, dtype=np.float32))
    return m


# ---------------------------------------------------------------------------
# GGUF v3 (public format): little-endian, KV section then tensor infos, data
# aligned to general.alignment (default 32).
# ---------------------------------------------------------------------------
_GT_U32, _GT_I32, _GT_F32, _GT_BOOL, _GT_STR, _GT_ARR = 4, 5, 6, 7, 8, 9
_GT_U64 = 10


def _kv_items(cfg: Config):
    e = "parakeet.encoder."
    kv = [("general.architecture", _GT_STR, "parakeet"),
          ("parakeet.arch", _GT_STR, cfg.arch),
          (e + "feat_in", _GT_U32, cfg.n_mels), (e + "d_model", _GT_U32, cfg.d_model),
          (e + "n_layers", _GT_U32, cfg.n_layers), (e + "n_heads", _GT_U32, cfg.n_heads),
          (e + "ff_dim", _GT_U32, cfg.ff_dim), (e + "conv_kernel", _GT_U32, cfg.conv_kernel),
          (e + "conv_norm_type", _GT_STR, cfg.conv_norm_type),
          (e + "subsampling_factor", _GT_U32, 8),
          (e + "subsampling_conv_channels", _GT_U32, cfg.sub_channels),
          (e + "xscaling", _GT_BOOL, bool(cfg.xscaling)),
          (e + "pos_emb_max_len", _GT_U32, 5000),
          ("parakeet.preprocessor.n_mels", _GT_U32, cfg.n_mels),
          ("parakeet.preprocessor.sample_rate", _GT_U32, cfg.sample_rate),
          ("parakeet.preprocessor.n_fft", _GT_U32, cfg.n_fft),
          ("parakeet.preprocessor.win_length", _GT_U32, cfg.win_length),
          ("parakeet.preprocessor.hop_length", _GT_U32, cfg.hop_length),
          ("parakeet.preprocessor.preemph", _GT_F32, cfg.preemph),
          ("parakeet.preprocessor.mag_power", _GT_F32, cfg.mag_power),
          ("parakeet.preprocessor.normalize", _GT_STR, cfg.normalize),
          ("parakeet.preprocessor.log_zero_guard", _GT_F32, cfg.log_zero_guard),
          ("parakeet.vocab_size", _GT_U32, cfg.vocab_size),
          ("parakeet.blank_id", _GT_U32, cfg.vocab_size),
          ("parakeet.joint.joint_hidden", _GT_U32, cfg.joint_hidden),
          ("parakeet.decoder.pred_hidden", _GT_U32, cfg.pred_hidden),
          ("parakeet.decoder.pred_rnn_layers", _GT_U32, cfg.pred_rnn_layers),
          ("parakeet.joint.activation", _GT_STR, "relu"),
          ("parakeet.decoding.max_symbols", _GT_U32, 10),
          ("parakeet.tdt.durations", _GT_ARR, (_GT_I32, list(cfg.tdt_durations))),
          # SentencePiece pieces: synthetic ones, one per token id (blank excluded)
          ("parakeet.tokenizer.pieces", _GT_ARR, (_GT_STR, ["<unk>"] + [f"▁t{i}" for i in range(1, cfg.vocab_size)]))]
    if cfg.streaming:       # scripts/convert_parakeet_to_gguf.py:176-222
        st = "parakeet.streaming."
        kv += [(e + "att_context_left", _GT_I32, cfg.att_context_left),
               (e + "att_context_right", _GT_I32, cfg.att_context_right),
               (e + "att_context_style", _GT_STR, cfg.att_context_style),
               (e + "causal_downsampling", _GT_BOOL, bool(cfg.causal_downsampling)),
               (e + "conv_causal", _GT_BOOL, bool(cfg.conv_causal)),
               (st + "chunk_size", _GT_ARR, (_GT_I32, list(cfg.stream_chunk_size))),
               (st + "shift_size", _GT_ARR, (_GT_I32, list(cfg.stream_shift_size))),
               (st + "cache_drop_size", _GT_I32, 0),
               (st + "last_channel_cache_size", _GT_I32, cfg.stream_last_channel_cache_size),
               (st + "valid_out_len", _GT_I32, cfg.stream_valid_out_len),
               (st + "pre_encode_cache_size", _GT_ARR, (_GT_I32, list(cfg.stream_pre_encode_cache_size))),
               (st + "drop_extra_pre_encoded", _GT_I32, cfg.stream_drop_extra_pre_encoded)]
    return kv


def _wstr(f, s: str):
    b = s.encode()
    f.write(struct.pack("<Q", len(b)))
    f.write(b)


def _wval(f, t, v):
    if t == _GT_U32:
        f.write(struct.pack("<I", v))
    elif t == _GT_I32:
        f.write(struct.pack("<i", v))
    elif t == _GT_F32:
        f.write(struct.pack("<f", v))
    elif t == _GT_BOOL:
        f.write(struct.pack("<B", 1 if v else 0))
    elif t == _GT_STR:
        _wstr(f, v)
    elif t == _GT_ARR:
        et, items = v
        f.write(struct.pack("<IQ", et, len(items)))
        for it in items:
            _wval(f, et, it)
    else:
        raise ValueError(t)


def write_gguf_tensors(path: str, kv, tensors: dict, align: int = 32):
    """GGUF v3: kv is a list of (key, gguf type id, value); tensors maps
    name -> Tensor (ggml ne order taken from the torch-order shape)."""
    names = list(tensors)
    offs, off = [], 0
    for n in names:
        offs.append(off)
        off += tensors[n].nbytes()
        off = (off + align - 1) // align * align
    with open(path, "wb") as f:
        f.write(struct.pack("<IIQQ", 0x46554747, 3, len(names), len(kv)))
        for k, t, v in kv:
            _wstr(f, k)
            f.write(struct.pack("<I", t))
            _wval(f, t, v)
        for n, o in zip(names, offs):
            t = tensors[n]
            _wstr(f, n)
            f.write(struct.pack("<I", len(t.ne)))
            for d in t.ne:
                f.write(struct.pack("<Q", d))
            f.write(struct.pack("<IQ", t.gtype, o))
        pos = f.tell()
        f.write(b"\0" * ((pos + align - 1) // align * align - pos))
        base = f.tell()
        for n, o in zip(names, offs):
            cur = f.tell() - base
            f.write(b"\0" * (o - cur))
            f.write(np.ascontiguousarray(tensors[n].data).tobytes())


def write_gguf(model: Model, path: str, align: int = 32, extra_kv=()):
    """extra_kv: additional (key, gguf type id, value) items, e.g. streaming keys."""
    write_gguf_tensors(path, _kv_items(model.cfg) + list(extra_kv), model.tensors, align)


GT_I32 = 26   # ggml's int32 tensor type


def write_baseline_gguf(path: str, arrays: dict):
    """Named f32 / int32 arrays (shape outermost first) in a GGUF, the layout of
    the reference's parity baselines (tests/parity.hpp:12-41)."""
    tensors = {}
    for name, a in arrays.items():
        a = np.asarray(a)
        if a.dtype == np.int32:
            tensors[name] = Tensor(GT_I32, tuple(a.shape), np.ascontiguousarray(a))
        else:
            tensors[name] = Tensor(0, tuple(a.shape), np.ascontiguousarray(a, dtype=np.float32))
    write_gguf_tensors(path, [("general.architecture", 8, "parakeet-baseline")], tensors)

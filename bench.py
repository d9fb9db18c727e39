#!/usr/bin/env python3
"""Encoder throughput on one MI355X: the 0.6B FastConformer encoder with q8_0
linears, batch 16 x 10 s of synthetic 128-bin log-mel (1000 frames -> T'=125).

One step = one encoder forward (subsampling + 24 conformer blocks) over the
batch, inputs already resident in HBM.  Prints ONE JSON line with encoder RTFx
(audio seconds per wall second), the dominant kernel's roofline position
(measured with HIP events on the launch stream), and the CPU baseline (the
oracle restatement timed on this host's cores on a bounded sample).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "parakeet.cpp_amd", "python"), os.path.join(ROOT, "oracle")]

import pk_model as pm  # noqa: E402
import pkx  # noqa: E402

PEAK_F16_TFLOPS = 2500.0   # MI355X dense f16/bf16 MFMA
PEAK_F32_TFLOPS = 157.3    # MI355X dense f32 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E

# 0.6B shape (parakeet-tdt-0.6b-v2: no linear/conv biases)
CFG = dict(d_model=1024, n_layers=24, n_heads=8, ff_dim=4096, conv_kernel=9, n_mels=128,
           sub_channels=256, xscaling=False, vocab_size=1024, attn_bias=False, ff_bias=False,
           conv_bias=False)
# 110M shape (parakeet-tdt_ctc-110m: linear and conv biases present)
CFG110 = dict(d_model=512, n_layers=17, n_heads=8, ff_dim=2048, conv_kernel=9, n_mels=80,
              sub_channels=256, xscaling=False, vocab_size=1024)
B, T_MEL, HOP_S = 16, 1000, 0.01


def family_work(cfg, B, Tp):
    """Algorithmic FLOPs (GEMM/attention) or HBM bytes (memory-bound) per launch."""
    D, FF, H = cfg.d_model, cfg.ff_dim, cfg.n_heads
    dk, M, P = D // H, B * Tp, 2 * Tp - 1
    return {
        "gemm_ffn": ("TFLOP/s", 2.0 * M * D * FF),
        "gemm_qkv": ("TFLOP/s", 2.0 * M * D * 3 * D),
        # one launch projects the positional table for all L layers ([L*D][D] weight)
        "gemm_pos": ("TFLOP/s", 2.0 * P * D * (cfg.n_layers * D)),
        "gemm_out": ("TFLOP/s", 2.0 * M * D * D),
        # pointwise_conv1 (+ GLU, and with kernel 9 the depthwise conv + BN + SiLU in its epilogue)
        "gemm_pw1_glu": ("TFLOP/s", 2.0 * M * D * 2 * D),
        "gemm_pw2": ("TFLOP/s", 2.0 * M * D * D),
        "attention": ("TFLOP/s", 6.0 * B * H * Tp * Tp * dk),
        # f16 write of the normalised rows + f32 read of the residual stream (single LN);
        # the fused norm_out/next-LN pass also writes the f32 stream back.
        "layernorm": ("GB/s", None),
        "dwconv": ("GB/s", 2.0 * M * D * 2 + D * (cfg.conv_kernel + 3) * 4),
    }


def layernorm_bytes(cfg, B, Tp, launches):
    """HBM bytes per LayerNorm launch.  Unfolded (4 L + 1 launches): norm_self_att,
    norm_conv, norm_feed_forward2 and layer 0's norm_feed_forward1 read the f32
    stream and write f16; norm_out is fused with the next layer's
    norm_feed_forward1 (and also writes the f32 stream back), the last one f32
    only.  Folded (L + 1 launches): only layer 0's norm_feed_forward1 and the
    norm_out passes remain, and a norm_out fused with the next
    norm_feed_forward1 reads the f32 stream and writes the f16 operand and the
    per-row statistics (the next block's FFN1 linear2 applies norm_out)."""
    D, L, M = cfg.d_model, cfg.n_layers, B * Tp
    single = M * D * (4 + 2)
    last = M * D * (4 + 4)
    if launches == L + 1:
        fused = M * D * (4 + 2) + M * 8
        return (single + (L - 1) * fused + last) / launches
    fused = M * D * (4 + 4 + 2)
    return ((3 * L + 1) * single + (L - 1) * fused + last) / launches


def step_stats(events):
    """Median and p90 of the per-step times between consecutive events (ms)."""
    per = np.array([events[i].elapsed_ms(events[i + 1]) for i in range(len(events) - 1)])
    return round(float(np.median(per)), 4), round(float(np.percentile(per, 90)), 4)


def other_config(name, qtype, cfg_kw, lens, T_max, steps, warmup, stream, base=None, gm=None):
    """The other benchmark shapes, same measurement (one GPU, inputs resident,
    FFN GEMM sampled with per-dispatch events inside the timed region).  gm: a
    model handle to reuse (kept open); otherwise one is synthesised and closed."""
    kw = dict(CFG if base is None else base)
    kw.update(cfg_kw)
    cfg = pm.Config(**kw)
    own = gm is None
    if own:
        model = pm.synthesize(cfg, qtype, heads=False)
        gm = pkx.Model.from_tensors(model, pkx.PREC_AUTO)
        del model
    Bc = len(lens)
    rng = np.random.default_rng(42)
    mel = rng.standard_normal((Bc, cfg.n_mels, T_max)).astype(np.float32)
    for b, v in enumerate(lens):
        mel[b, :, v:] = 0.0
    d_mel = pkx.DeviceArray.from_numpy(mel, stream)
    Tp = pkx.subsampled_len(T_max)
    d_out = pkx.DeviceArray((Bc, Tp, cfg.d_model), np.float32)
    valid = np.asarray(lens, dtype=np.int32)
    for _ in range(warmup):
        gm.encoder_forward(d_mel, valid, d_out, stream=stream)
    stream.sync()
    gm.set_profiling(["gemm_ffn"], stride=25)
    ev = [pkx.Event() for _ in range(steps + 1)]
    ev[0].record(stream)
    vo = None
    for i in range(steps):
        _, vo = gm.encoder_forward(d_mel, valid, d_out, stream=stream)
        ev[i + 1].record(stream)
    ms = ev[0].elapsed_ms(ev[-1]) / steps
    stream.sync()
    med, p90 = step_stats(ev)
    ffn_ms, ffn_n = gm.profile()["gemm_ffn"]
    gm.set_profiling(False)
    res = d_out.numpy(stream)
    finite = bool(all(np.isfinite(res[b, :vo[b]]).all() for b in range(Bc)))
    if not finite:
        raise RuntimeError("%s: non-finite encoder output" % name)
    M = Bc * Tp
    ffn_flop = 2.0 * M * cfg.d_model * cfg.ff_dim
    ffn_tf = ffn_flop / (ffn_ms / 1e3 / ffn_n) / 1e12
    f32 = gm.precision == pkx.PREC_F32
    peak = PEAK_F32_TFLOPS if f32 else PEAK_F16_TFLOPS
    audio_s = float(np.sum(lens)) * HOP_S
    out = {"workload": name, "dtype": "f32" if f32 else "f16", "ms_per_step": round(ms, 4),
           "ms_per_step_median": med, "ms_per_step_p90": p90, "outputs_finite": finite,
           "rtfx": round(audio_s / (ms / 1e3), 1),
           "frames_per_s": round(float(np.sum(vo)) / (ms / 1e3), 1),
           "gemm_ffn": {"avg_us": round(ffn_ms / ffn_n * 1e3, 2), "achieved": round(ffn_tf, 2),
                        "unit": "TFLOP/s", "peak": peak, "frac": round(ffn_tf / peak, 4)},
           "steps": steps}
    d_mel.free()
    d_out.free()
    if own:
        gm.close()
    return out


def pcm_in(gm, cfg, stream, steps, warmup=2):
    """PCM-in path: the device log-mel front end (pkx_mel_forward, 16 clips of
    10 s of 16 kHz audio -> [16][n_mels][1001]) followed by the same encoder
    forward.  Reports the front end alone (time, RTFx, algorithmic bytes
    against HBM) and the two together."""
    mel = pkx.Mel.create(cfg.n_fft, cfg.win_length, cfg.hop_length, cfg.n_mels, pm.hann_window(cfg.win_length),
                         pm.mel_filterbank(cfg.sample_rate, cfg.n_fft, cfg.n_mels))
    S = 10 * cfg.sample_rate
    pcm = (np.random.default_rng(11).standard_normal((B, S)) * 0.1).astype(np.float32)
    lens = np.full(B, S, np.int32)
    T = mel.frames(S)
    d_pcm = pkx.DeviceArray.from_numpy(pcm, stream)
    d_mel = pkx.DeviceArray((B, cfg.n_mels, T), np.float32)
    d_out = pkx.DeviceArray((B, pkx.subsampled_len(T), cfg.d_model), np.float32)
    for _ in range(warmup):
        Tv = mel.forward(d_pcm, lens, d_mel, T, stream=stream)
        gm.encoder_forward(d_mel, Tv, d_out, stream=stream)
    stream.sync()
    e0, e1 = pkx.Event(), pkx.Event()
    e0.record(stream)
    for _ in range(steps):
        mel.forward(d_pcm, lens, d_mel, T, stream=stream)
    e1.record(stream)
    mel_ms = e0.elapsed_ms(e1) / steps
    e0.record(stream)
    for _ in range(steps):
        Tv = mel.forward(d_pcm, lens, d_mel, T, stream=stream)
        gm.encoder_forward(d_mel, Tv, d_out, stream=stream)
    e1.record(stream)
    both_ms = e0.elapsed_ms(e1) / steps
    stream.sync()
    assert np.isfinite(d_out.numpy(stream)).all()
    for a in (d_pcm, d_mel, d_out):
        a.free()
    mel.close()
    audio_s = B * S / cfg.sample_rate
    mel_bytes = B * S * 4 + B * cfg.n_mels * T * 4            # PCM in, log-mel out (f32)
    return {"workload": "log-mel front end + encoder, batch 16 x 10 s of 16 kHz PCM (-> %d mel frames)" % T,
            "mel_ms": round(mel_ms, 4), "mel_rtfx": round(audio_s / (mel_ms / 1e3), 1),
            "mel_hbm": {"achieved": round(mel_bytes / (mel_ms / 1e3) / 1e9, 1), "unit": "GB/s",
                        "frac": round(mel_bytes / (mel_ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
                        "bytes": mel_bytes, "note": "call time incl. its host sync; f64 FFT + filterbank"},
            "ms_per_step": round(both_ms, 4), "rtfx": round(audio_s / (both_ms / 1e3), 1), "steps": steps}


def greedy_decode(gm, cfg, stream, d_enc, valid_out, reps=3):
    """Batched greedy TDT decode (prediction LSTM + joint + rule, device) of the
    encoder output: 16 items x 125 frames, 0.6B decoder shape (2-layer LSTM 640,
    joint 640, 1024 tokens + blank + 5 durations); wall time per batch."""
    d = tuple(cfg.tdt_durations)
    gm.transducer_greedy(d_enc, valid_out, durations=d, stream=stream)
    t0 = time.perf_counter()
    for _ in range(reps):
        out = gm.transducer_greedy(d_enc, valid_out, durations=d, stream=stream)
    ms = (time.perf_counter() - t0) * 1e3 / reps
    toks = int(sum(len(o[0]) for o in out))
    audio_s = B * T_MEL * HOP_S
    return {"workload": "greedy TDT decode of the encoder output, batch 16 x 125 frames (random-init decoder)",
            "ms": round(ms, 3), "rtfx": round(audio_s / (ms / 1e3), 1), "tokens": toks, "reps": reps}


def streaming(stream, n_streams=256, steps=50, warmup=5):
    """Cache-aware streaming encoder (pkx_streaming_step): the streaming model's
    shape (17 blocks, d_model 512, 8 heads, ff 2048, causal, att_context [70, 1],
    q8_0 linears), n_streams streams in lockstep, steady-state windows of
    9 + 16 mel frames (160 ms of new audio, 2 encoder frames per stream and
    step).  Reports per-step latency, stream RTFx, and the step's HBM bytes
    (device weights once + per stream the f16 key/value rings and the f32 conv
    history) against 8 TB/s."""
    cfg = pm.eou_config()
    model = pm.synthesize(cfg, "q8_0", heads=False)
    gm = pkx.Model.from_tensors(model, pkx.PREC_AUTO)
    S, W = n_streams, 25
    st = pkx.Streaming(gm, n_streams=S, max_window=W, stream=stream)
    rng = np.random.default_rng(3)
    d_first = pkx.DeviceArray.from_numpy(rng.normal(0, 1, (S, cfg.n_mels, 9)).astype(np.float32), stream)
    d_win = pkx.DeviceArray.from_numpy(rng.normal(0, 1, (S, cfg.n_mels, W)).astype(np.float32), stream)
    d_out = pkx.DeviceArray((S, st.chunk_len(9), cfg.d_model), np.float32)
    st.step(d_first, d_out, stream=stream)
    for _ in range(warmup):
        st.step(d_win, d_out, stream=stream)
    stream.sync()
    e0, e1 = pkx.Event(), pkx.Event()
    e0.record(stream)
    for _ in range(steps):
        st.step(d_win, d_out, stream=stream)
    e1.record(stream)
    ms = e0.elapsed_ms(e1) / steps
    stream.sync()
    assert np.isfinite(d_out.numpy(stream)).all(), "non-finite streaming output"
    gm.set_profiling(True)
    n_prof = 5
    for _ in range(n_prof):
        st.step(d_win, d_out, stream=stream)
    prof = gm.profile()
    gm.set_profiling(False)
    D, FF, L, CL, LP, C = cfg.d_model, cfg.ff_dim, cfg.n_layers, 70, cfg.conv_kernel - 1, cfg.sub_channels
    n_w = L * (4 * D * FF + 7 * D * D) + D * C * cfg.sub_feat() + 2 * C * C
    w_bytes = n_w * 34 / 32                                   # q8_0: 32 int8 + one f16 scale per block
    # per stream and layer: f16 key + value rings read, the chunk's 2 rows written
    # back, the f32 conv history read and rewritten
    state_bytes = S * L * (2 * CL * D * 2 + 2 * 2 * D * 2 + 2 * LP * D * 4)
    total = w_bytes + state_bytes
    audio_s = S * 16 * HOP_S
    st.close()
    fams = {f: {"launches_per_step": round(n / n_prof, 1), "us_per_step": round(t / n_prof * 1e3, 1)}
            for f, (t, n) in prof.items() if n}
    return {"workload": "cache-aware streaming encoder, 17 blocks d_model 512 q8_0 (streaming model shape), "
                        "%d streams x windows of 9 + 16 mel frames (2 encoder frames per stream and step)" % S,
            "ms_per_step": round(ms, 4), "rtfx": round(audio_s / (ms / 1e3), 1),
            "hbm": {"bytes_per_step": int(total), "weights": int(w_bytes), "stream_state": int(state_bytes),
                    "achieved": round(total / (ms / 1e3) / 1e9, 1), "unit": "GB/s",
                    "frac": round(total / (ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4)},
            "kernels": fams, "steps": steps}


def cpu_model_name():
    """The host CPU's model name as lscpu prints it ("Model name", with its
    "BIOS Model name" when lscpu gives one), else /proc/cpuinfo's."""
    import subprocess
    names = []
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            key, _, val = line.partition(":")
            if key.strip() in ("Model name", "BIOS Model name") and val.strip():
                names.append("%s: %s" % (key.strip(), val.strip()))
    except (OSError, subprocess.SubprocessError):
        pass
    if names:
        return "; ".join(names)
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(model, mel, valid):
    """The oracle (C restatement of the reference encoder, OpenMP over rows and
    heads) on the benchmarked workload itself: the whole B x 1000-frame batch,
    once with every host thread this process may use and once with 8 threads
    (the reference's default, kDefaultThreads in src/ggml_graph.cpp:47)."""
    import oracle
    om = oracle.OracleModel(model)
    n_all = oracle.get_threads()
    om.encoder(mel[:1, :, :200], np.array([199]))               # warm-up (page in weights)
    runs = []
    for threads in (n_all, 8):
        oracle.set_threads(threads)
        t0 = time.perf_counter()
        om.encoder(mel, valid - 1)
        el = time.perf_counter() - t0
        audio = mel.shape[0] * mel.shape[2] * HOP_S
        runs.append({"threads": threads, "value": round(audio / el, 3), "wall_s": round(el, 2)})
    oracle.set_threads(n_all)
    return {"value": runs[0]["value"], "unit": "RTFx (audio s / wall s)", "cores": n_all, "kind": "port",
            "cpu_model": cpu_model_name(), "nproc": os.cpu_count(), "runs": runs,
            "sample": f"the benchmarked batch ({mel.shape[0]} x {mel.shape[2]} frames = "
                      f"{mel.shape[0] * mel.shape[2] * HOP_S:.0f} s of audio), same 0.6B q8_0 weights "
                      f"dequantised to f32, C restatement of the reference encoder (ggml absent); "
                      f"{runs[0]['wall_s']} s at {n_all} threads, {runs[1]['wall_s']} s at 8 threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the other workload shapes")
    ap.add_argument("--streaming-only", action="store_true",
                    help="run only the streaming-encoder workload and print its record")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this encoder build runs on one GPU; --gpus {args.gpus} is not supported "
              "(utterance-level data parallelism across GPUs is described, not built).", file=sys.stderr)
        sys.exit(2)
    if args.streaming_only:
        print(json.dumps(streaming(pkx.Stream())))
        return

    cfg = pm.Config(**CFG)
    t0 = time.perf_counter()
    model = pm.add_prediction(pm.synthesize(cfg, "q8_0", heads=True))
    gm = pkx.Model.from_tensors(model, pkx.PREC_AUTO)
    assert gm.precision == pkx.PREC_F16
    setup_s = time.perf_counter() - t0

    rng = np.random.default_rng(42)
    mel = rng.standard_normal((B, cfg.n_mels, T_MEL)).astype(np.float32)
    stream = pkx.Stream()
    d_mel = pkx.DeviceArray.from_numpy(mel, stream)
    Tp = pkx.subsampled_len(T_MEL)
    d_out = pkx.DeviceArray((B, Tp, cfg.d_model), np.float32)
    valid = np.full(B, T_MEL, dtype=np.int32)

    for _ in range(args.warmup):
        gm.encoder_forward(d_mel, valid, d_out, stream=stream)
    stream.sync()
    # Timed region.  Every 25th FFN GEMM launch carries start/stop events on its
    # own dispatch packet (no extra packets, no syncs); 25 is coprime with the
    # 96 FFN launches per step, so the sampled positions rotate through all
    # FFN1/FFN2 launches of the 24 blocks as the steps go by, and the event cost
    # (about 4 launches per step) stays off the rest.
    gm.set_profiling(["gemm_ffn"], stride=25)
    ev = [pkx.Event() for _ in range(args.steps + 1)]
    ev[0].record(stream)
    for i in range(args.steps):
        gm.encoder_forward(d_mel, valid, d_out, stream=stream)
        ev[i + 1].record(stream)
    ms_total = ev[0].elapsed_ms(ev[-1])
    stream.sync()
    ms_med, ms_p90 = step_stats(ev)
    ffn_ms, ffn_n = gm.profile()["gemm_ffn"]
    ms_step = ms_total / args.steps
    out = d_out.numpy(stream)
    assert np.isfinite(out).all(), "non-finite encoder output"

    # A plain device-to-device copy of known size: under `rocprofv3 --pmc` its
    # FETCH_SIZE / WRITE_SIZE calibrate the counters the traffic figure uses.
    calib_n = 64 << 20
    c_src, c_dst = pkx.DeviceArray((calib_n,), np.uint8), pkx.DeviceArray((calib_n,), np.uint8)
    pkx.check(pkx.lib().pkx_memcpy_d2d(c_dst.ptr, c_src.ptr, calib_n, stream.handle))
    stream.sync()
    c_src.free()
    c_dst.free()

    # Per-family breakdown: a separate pass with every launch timed the same way.
    n_prof = 3
    gm.set_profiling(True)
    for _ in range(n_prof):
        gm.encoder_forward(d_mel, valid, d_out, stream=stream)
    prof = gm.profile()
    gm.set_profiling(False)
    work = family_work(cfg, B, Tp)
    kernels = {}
    busy_ms = 0.0
    for fam, (ms, n) in prof.items():
        if n == 0:
            continue
        busy_ms += ms / n_prof
        avg_s = ms / 1e3 / n
        rec = {"launches_per_step": round(n / n_prof, 2), "avg_us": round(avg_s * 1e6, 2),
               "us_per_step": round(ms / n_prof * 1e3, 1)}
        if fam in work:
            unit, per = work[fam]
            if fam == "layernorm":
                per = layernorm_bytes(cfg, B, Tp, round(n / n_prof))
            if unit == "TFLOP/s":
                rec.update(achieved=round(per / avg_s / 1e12, 2), unit=unit,
                           frac=round(per / avg_s / 1e12 / PEAK_F16_TFLOPS, 4))
            else:
                rec.update(achieved=round(per / avg_s / 1e9, 1), unit=unit,
                           frac=round(per / avg_s / 1e9 / PEAK_HBM_GBS, 4))
        kernels[fam] = rec
    ffn_avg_s = ffn_ms / 1e3 / ffn_n
    ffn_tf = work["gemm_ffn"][1] / ffn_avg_s / 1e12
    traffic, traffic_src = None, None
    tpath = os.path.join(ROOT, "profiles", "gemm_ffn_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        traffic = tj["traffic_bytes_per_launch"]["family_avg"]
        traffic_src = ("profiles/gemm_ffn_traffic.json: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch, "
                       "scaled by a 64 MiB copy (factors %.4f / %.4f); algorithmic %d B" % (
                           tj["calibration"]["fetch_factor"], tj["calibration"]["write_factor"],
                           tj["algorithmic_bytes_per_launch"]["family_avg"]))
    roofline = {"bound": "mfma",
                "kernel": "gemm_ffn (f16 MFMA; q8_0 weights dequantised in registers: linear1 on 128x256 tiles, linear2 on 64x128 tiles in two K groups)",
                "achieved": round(ffn_tf, 2), "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ffn_tf / PEAK_F16_TFLOPS, 4), "traffic": traffic, "traffic_source": traffic_src,
                "avg_us": round(ffn_avg_s * 1e6, 2), "launches_sampled": int(ffn_n),
                "launches_in_region": 4 * cfg.n_layers * args.steps,
                "per_launch": "2*M*D*FF = %.3f GFLOP (M=B*T'=%d, D=%d, FF=%d)" % (
                    work["gemm_ffn"][1] / 1e9, B * Tp, cfg.d_model, cfg.ff_dim)}

    lnk = kernels.get("layernorm", {})
    roofline_hbm = {"bound": "hbm", "kernel": "layernorm (norm_out fused with the next block's "
                                              "norm_feed_forward1; layer 0's norm_feed_forward1)",
                    "achieved": lnk.get("achieved"), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": lnk.get("frac"), "traffic": None, "avg_us": lnk.get("avg_us"),
                    "per_launch": "f32 residual read + f16 normalised rows (+ f32 write of the last norm_out, "
                                  "per-row statistics of the others): %.1f MB average" % (
                        layernorm_bytes(cfg, B, Tp, cfg.n_layers + 1) / 1e6)}

    pcm_line = pcm_in(gm, cfg, stream, min(args.steps, 10))
    _, vo_dec = gm.encoder_forward(d_mel, valid, d_out, stream=stream)
    dec_line = greedy_decode(gm, cfg, stream, d_out, vo_dec)
    stream_line = streaming(stream)   # 256 streams

    audio_s = B * T_MEL * HOP_S
    rtfx = audio_s / (ms_step / 1e3)
    line = {
        "metric": "encoder RTFx + HBM GB/s / MFMA util, 0.6B conformer q8_0 bs16 on 1 MI355X",
        "value": round(rtfx, 1), "unit": "RTFx (audio s / wall s)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "ms_per_step_median": ms_med, "ms_per_step_p90": ms_p90,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded N(0,1) log-mel; random-init q8_0 weights)",
        "config": {"workload": "FastConformer encoder 0.6B shape: 24 blocks, d_model 1024, 8 heads x 128, "
                               "ff 4096, conv kernel 9, dw-striding x8 (256 ch); q8_0 linears; "
                               "128-mel, batch 16 x 1000 frames (10 s) -> T'=125",
                   "global_batch": B, "seq_len": T_MEL, "parallelism": "none (1 GPU)"},
        "frames_per_s": round(B * Tp / (ms_step / 1e3), 1),
        "roofline": roofline,
        "roofline_hbm": roofline_hbm,
        "kernels": kernels,
        "kernel_busy_ms_per_step": round(busy_ms, 4),
        "pcm_in": pcm_line,
        "decode": dec_line,
        "streaming": stream_line,
        "setup_s": round(setup_s, 1),
    }
    if not args.no_extra:
        # the ragged f16 batch (16 clips of 2-20 s) and the 1.1B shape at 8 x 30 s
        lens = (200 + np.floor(np.random.default_rng(7).random(16) * 1801)).astype(np.int32)
        cfg11 = pm.Config(**dict(CFG, n_layers=42))
        gm11 = pkx.Model.from_tensors(pm.synthesize(cfg11, "q8_0", heads=False), pkx.PREC_AUTO)
        line["other_configs"] = [
            other_config("0.6B f16 weights, batch 16 ragged 2-20 s (T_max %d frames)" % int(lens.max()), "f16", {},
                         lens, int(lens.max()), 10, 2, stream),
            other_config("1.1B shape q8_0 (42 blocks), batch 8 x 30 s (3000 frames -> T'=375)", "q8_0",
                         dict(n_layers=42), np.full(8, 3000, dtype=np.int32), 3000, 5, 1, stream, gm=gm11),
            # the long-sequence stress case: 300 s per item, T' = 3750 (the O(T'^2) attention)
            other_config("1.1B shape q8_0 (42 blocks), batch 8 x 300 s (30000 frames -> T'=3750)", "q8_0",
                         dict(n_layers=42), np.full(8, 30000, dtype=np.int32), 30000, 2, 1, stream, gm=gm11),
            other_config("0.6B q4_K weights, batch 16 x 10 s", "q4_k", {}, np.full(16, 1000, dtype=np.int32), 1000,
                         10, 2, stream),
            # the 110M shape in f32 (f32 MFMA 16x16x4; FFN against the f32 peak)
            other_config("110M shape f32 (17 blocks, d_model 512, 8 heads x 64, ff 2048, 80-mel), batch 1 x 10 s",
                         "f32", {}, np.full(1, 1000, dtype=np.int32), 1000, 20, 3, stream, base=CFG110),
            other_config("110M shape f32, batch 16 x 10 s", "f32", {}, np.full(16, 1000, dtype=np.int32), 1000,
                         10, 2, stream, base=CFG110),
        ]
        gm11.close()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(model, mel, valid)
    print(json.dumps(line))


if __name__ == "__main__":
    main()

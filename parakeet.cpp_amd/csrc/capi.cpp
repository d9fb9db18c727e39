// extern "C" boundary (include/pkx.h).  Every entry point catches all C++
// exceptions and reports them through a thread-local last-error string, the
// same no-throw convention as the reference C API (src/parakeet_capi.cpp:207-225).
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/pkx.h"
#include "mel.hpp"
#include "model.hpp"
#include "quantize.hpp"

struct pkx_mel {
    std::unique_ptr<pkx::MelFront> impl;
};

struct pkx_model {
    pkx_config cfg;
    int precision;
    std::unique_ptr<pkx::Model> impl;
};

struct pkx_streaming {
    pkx::Model* model;
    std::unique_ptr<pkx::StreamState> st;
};

// Fixed device scratch of pkx_tdt_joint_argmax_noalloc: one copy per GPU,
// held until the process ends.  Host code never passes the symbol's name as an
// address (it is a host-side stand-in there); joint_scratch() finds each GPU's
// copy with hipGetSymbolAddress (at model set-up, with the model's device
// current) and that address is used from then on.
static __device__ __align__(256) float scratch[PKX_JOINT_NOALLOC_MAX_FLOATS];

namespace {
thread_local std::string g_last_error;

template <typename F>
int guarded(F&& f) {
    try {
        f();
        g_last_error.clear();
        return 0;
    } catch (const std::exception& e) {
        g_last_error = e.what();
    } catch (...) {
        g_last_error = "unknown error";
    }
    pkx::tl_launch_hook = nullptr;   // a failed call may leave a profiled region open
    return 1;
}

hipStream_t st(void* s) { return (hipStream_t)s; }

constexpr int kMaxDevices = 64;

// Device address of this GPU's copy of `scratch` (below the namespace), looked
// up with hipGetSymbolAddress once per device with that device current.

float* joint_scratch() {
    static std::mutex mu;
    static float* ptr[kMaxDevices] = {};
    int dev = 0;
    PKX_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) throw std::invalid_argument("device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        PKX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        // the code objects of the kernels the entry point launches, loaded now
        // rather than at its first launch
        pkx::gemm_module_ready();
        pkx::elementwise_module_ready();
        ptr[dev] = (float*)p;
    }
    return ptr[dev];
}

void need(bool ok, const char* what) {
    if (!ok) throw std::invalid_argument(what);
}

pkx::ModelConfig to_internal(const pkx_config& c) {
    pkx::ModelConfig m;
    m.d_model = c.d_model;
    m.n_layers = c.n_layers;
    m.n_heads = c.n_heads;
    m.ff_dim = c.ff_dim;
    m.conv_kernel = c.conv_kernel;
    m.n_mels = c.n_mels;
    m.sub_channels = c.sub_channels;
    m.xscaling = c.xscaling;
    m.vocab_size = c.vocab_size;
    m.n_durations = c.n_durations;
    m.conv_ln = c.conv_ln;
    m.causal_sub = c.causal_sub;
    m.conv_causal = c.conv_causal;
    m.att_limited = c.att_limited;
    m.att_left = c.att_left;
    m.att_right = c.att_right;
    m.stream_chunk_first = c.stream_chunk_first;
    m.stream_chunk = c.stream_chunk;
    m.stream_pre_cache = c.stream_pre_cache;
    m.stream_cache_len = c.stream_cache_len;
    m.stream_valid_out_len = c.stream_valid_out_len;
    m.stream_drop_extra = c.stream_drop_extra;
    return m;
}

pkx_config to_public(const pkx::ModelConfig& m) {
    pkx_config c;
    c.d_model = m.d_model;
    c.n_layers = m.n_layers;
    c.n_heads = m.n_heads;
    c.ff_dim = m.ff_dim;
    c.conv_kernel = m.conv_kernel;
    c.n_mels = m.n_mels;
    c.sub_channels = m.sub_channels;
    c.xscaling = m.xscaling;
    c.vocab_size = m.vocab_size;
    c.n_durations = m.n_durations;
    c.conv_ln = m.conv_ln;
    c.causal_sub = m.causal_sub;
    c.conv_causal = m.conv_causal;
    c.att_limited = m.att_limited;
    c.att_left = m.att_left;
    c.att_right = m.att_right;
    c.stream_chunk_first = m.stream_chunk_first;
    c.stream_chunk = m.stream_chunk;
    c.stream_pre_cache = m.stream_pre_cache;
    c.stream_cache_len = m.stream_cache_len;
    c.stream_valid_out_len = m.stream_valid_out_len;
    c.stream_drop_extra = m.stream_drop_extra;
    return c;
}
}  // namespace

extern "C" {

int pkx_abi_version(void) { return PKX_ABI_VERSION; }
const char* pkx_last_error(void) { return g_last_error.c_str(); }

int pkx_device_count(int* n) {
    return guarded([&] { need(n, "null n"); PKX_HIP(hipGetDeviceCount(n)); });
}
int pkx_malloc(void** dev, size_t bytes) {
    return guarded([&] { need(dev, "null out"); PKX_HIP(hipMalloc(dev, bytes ? bytes : 16)); });
}
int pkx_free(void* dev) {
    return guarded([&] { if (dev) PKX_HIP(hipFree(dev)); });
}
int pkx_mem_info(size_t* free_bytes, size_t* total_bytes) {
    return guarded([&] {
        need(free_bytes && total_bytes, "null out");
        PKX_HIP(hipMemGetInfo(free_bytes, total_bytes));
    });
}
int pkx_memcpy_h2d(void* dst, const void* src, size_t bytes, void* s) {
    return guarded([&] {
        PKX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st(s)));
        PKX_HIP(hipStreamSynchronize(st(s)));
    });
}
int pkx_memcpy_d2h(void* dst, const void* src, size_t bytes, void* s) {
    return guarded([&] {
        PKX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st(s)));
        PKX_HIP(hipStreamSynchronize(st(s)));
    });
}
int pkx_memcpy_d2d(void* dst, const void* src, size_t bytes, void* s) {
    return guarded([&] { PKX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st(s))); });
}
int pkx_stream_create(void** s) {
    return guarded([&] {
        need(s, "null out");
        hipStream_t h;
        PKX_HIP(hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
        *s = h;
    });
}
int pkx_stream_destroy(void* s) {
    return guarded([&] { if (s) PKX_HIP(hipStreamDestroy(st(s))); });
}
int pkx_stream_synchronize(void* s) {
    return guarded([&] { PKX_HIP(hipStreamSynchronize(st(s))); });
}
int pkx_event_create(void** e) {
    return guarded([&] {
        need(e, "null out");
        hipEvent_t h;
        PKX_HIP(hipEventCreate(&h));
        *e = h;
    });
}
int pkx_event_destroy(void* e) {
    return guarded([&] { if (e) PKX_HIP(hipEventDestroy((hipEvent_t)e)); });
}
int pkx_event_record(void* e, void* s) {
    return guarded([&] { PKX_HIP(hipEventRecord((hipEvent_t)e, st(s))); });
}
int pkx_event_elapsed_ms(float* ms, void* a, void* b) {
    return guarded([&] {
        need(ms && a && b, "null argument");
        PKX_HIP(hipEventSynchronize((hipEvent_t)b));
        PKX_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    });
}

int pkx_model_load_gguf(const char* path, int precision, pkx_model** out) {
    return guarded([&] {
        need(path && out, "null argument");
        *out = nullptr;
        std::unique_ptr<pkx::Model> impl = pkx::load_gguf(path, precision);
        (void)joint_scratch();   // set-up: this GPU's scratch address (see pkx_model_finalize)
        pkx_model* m = new pkx_model;
        m->cfg = to_public(impl->config());
        m->precision = impl->precision();
        m->impl = std::move(impl);
        *out = m;
    });
}

int pkx_gguf_read_kv(const char* path, pkx_gguf_kv_fn fn, void* user) {
    return guarded([&] {
        need(path && fn, "null argument");
        std::vector<pkx_gguf_str> tmp;
        pkx::read_gguf_kv(path, [&](const std::string& key, int type, int et, uint64_t n, const void* raw,
                                    const std::vector<std::string>* strs) {
            if (strs) {
                tmp.resize(strs->size());
                for (size_t i = 0; i < strs->size(); ++i) tmp[i] = pkx_gguf_str{(*strs)[i].data(), (*strs)[i].size()};
                fn(user, key.c_str(), type, et, n, tmp.data());
            } else {
                fn(user, key.c_str(), type, et, n, raw);
            }
        });
    });
}

int pkx_model_create(const pkx_config* cfg, int precision, pkx_model** out) {
    return guarded([&] {
        need(cfg && out, "null argument");
        need(precision >= -1 && precision <= 1, "precision must be PKX_PREC_AUTO/F32/F16");
        *out = nullptr;
        pkx_model* m = new pkx_model;
        m->cfg = *cfg;
        m->precision = precision;
        try {
            m->impl.reset(new pkx::Model(to_internal(*cfg), precision));
        } catch (...) {
            delete m;
            throw;
        }
        *out = m;
    });
}

int pkx_model_set_tensor(pkx_model* m, const char* name, int gtype, int n_dims, const int64_t* ne,
                         const void* data, size_t nbytes) {
    return guarded([&] {
        need(m && name && ne && data, "null argument");
        m->impl->set_tensor(name, gtype, n_dims, ne, data, nbytes);
    });
}

int pkx_model_finalize(pkx_model* m) {
    return guarded([&] {
        need(m, "null model");
        m->impl->finalize();
        m->precision = m->impl->precision();
        // Set-up of pkx_tdt_joint_argmax_noalloc on this GPU: the symbol lookup
        // (the first one on a device materialises the array's storage) happens
        // here, so that entry point itself takes no device memory.
        (void)joint_scratch();
    });
}

int pkx_model_free(pkx_model* m) {
    return guarded([&] { delete m; });
}

int pkx_model_info(pkx_model* m, pkx_config* cfg, int* precision, int* has_ctc, int* has_joint) {
    return guarded([&] {
        need(m, "null model");
        if (cfg) *cfg = to_public(m->impl->config());
        if (precision) *precision = m->impl->precision();
        if (has_ctc) *has_ctc = m->impl->has_ctc() ? 1 : 0;
        if (has_joint) *has_joint = m->impl->has_joint() ? 1 : 0;
    });
}

int pkx_subsampled_len(int T) { return pkx::subsampled_len(T); }
int pkx_valid_out_len(int T, int in_valid) { return pkx::valid_out_len(T, in_valid); }

int pkx_encoder_forward(pkx_model* m, const float* mel, int B, int T_max, const int* valid_T, int mask_mode,
                        float* out, int* T_out, int* valid_out, float* capture, void* s) {
    return guarded([&] {
        need(m && mel && out, "null argument");
        need(mask_mode == PKX_MASK_BATCHED || mask_mode == PKX_MASK_SCALAR, "bad mask_mode");
        const int Tp = m->impl->encoder_forward(mel, B, T_max, valid_T, mask_mode == PKX_MASK_BATCHED, out,
                                                valid_out, capture, st(s));
        if (T_out) *T_out = Tp;
    });
}

int pkx_compact_channels_first(const float* x, int B, int T, int D, const int* valid, const int64_t* offs,
                               float* out, void* s) {
    return guarded([&] {
        need(x && valid && offs && out, "null argument");
        pkx::launch_compact_channels_first(x, B, T, D, valid, offs, out, st(s));
    });
}

int pkx_subsampling_forward(pkx_model* m, const float* mel, int B, int T_max, const int* valid_T, int mask_mode,
                            float* out, int* T_out, int* valid_out, void* s) {
    return guarded([&] {
        need(m && mel && out, "null argument");
        const int base = mask_mode & ~PKX_MASK_WHOLE_FRAMES;
        need(base == PKX_MASK_BATCHED || base == PKX_MASK_SCALAR, "bad mask_mode");
        const int Tp = m->impl->subsampling_forward(mel, B, T_max, valid_T, base == PKX_MASK_BATCHED, out,
                                                    valid_out, st(s), false,
                                                    (mask_mode & PKX_MASK_WHOLE_FRAMES) != 0);
        if (T_out) *T_out = Tp;
    });
}

int pkx_conformer_layer_forward(pkx_model* m, int layer, const float* x, int B, int T, const int* valid,
                                const float* pos_emb, float* out, float* conv_out, void* s) {
    return guarded([&] {
        need(m && x && out, "null argument");
        m->impl->conformer_layer_forward(layer, x, B, T, valid, pos_emb, out, conv_out, st(s));
    });
}

int pkx_relpos_attention_forward(pkx_model* m, int layer, const float* x, int B, int T, const int* valid,
                                 const float* pos_emb, float* out, void* s) {
    return guarded([&] {
        need(m && x && out, "null argument");
        m->impl->relpos_attention_forward(layer, x, B, T, valid, pos_emb, out, st(s));
    });
}

int pkx_conv_module_forward(pkx_model* m, int layer, const float* c, int B, int T, const int* valid,
                            float* out, void* s) {
    return guarded([&] {
        need(m && c && out, "null argument");
        m->impl->conv_module_forward(layer, c, B, T, valid, out, st(s));
    });
}

int pkx_ctc_forward(pkx_model* m, const float* enc, int64_t M, float* logprobs, int32_t* argmax, void* s) {
    return guarded([&] {
        need(m && enc && logprobs && argmax, "null argument");
        m->impl->ctc_forward(enc, M, logprobs, argmax, st(s));
    });
}

int pkx_tdt_joint_argmax(pkx_model* m, const float* enc, int64_t M, const float* g, float* logits, int32_t* tok,
                         int32_t* dur, void* s) {
    return guarded([&] {
        need(m && enc && g && logits && tok && dur, "null argument");
        m->impl->tdt_joint_argmax(enc, M, g, logits, tok, dur, st(s));
    });
}

int pkx_tdt_joint_argmax_noalloc(pkx_model* m, const float* enc, int64_t M, const float* g, float* logits,
                                 int32_t* tok, int32_t* dur, void* s) {
    return guarded([&] {
        need(m && enc && g && logits && tok && dur, "null argument");
        need(m->impl->has_joint(), "model has no TDT joint");
        const int64_t Hj = m->impl->joint_hidden();
        need(M >= 1, "joint: no frames");
        // scratch layout: pp [Hj] at 0, hid [M][Hj] from the next 256-byte boundary
        const int64_t hid_off = (Hj + 63) / 64 * 64;
        need(M <= ((int64_t)PKX_JOINT_NOALLOC_MAX_FLOATS - hid_off) / Hj,
             "pkx_tdt_joint_argmax_noalloc: M frames need more than the fixed scratch array of "
             "PKX_JOINT_NOALLOC_MAX_FLOATS floats (at most (PKX_JOINT_NOALLOC_MAX_FLOATS - joint_hidden) / "
             "joint_hidden frames); use pkx_tdt_joint_argmax");
        float* sc = joint_scratch();
        m->impl->tdt_joint_argmax_in(enc, M, g, logits, tok, dur, sc, sc + hid_off, st(s));
    });
}

int pkx_dequantize(int gtype, const void* src, float* dst, int64_t n, void* s) {
    return guarded([&] {
        need(src && dst, "null argument");
        pkx::launch_dequantize(gtype, src, dst, n, st(s));
    });
}

int pkx_linear(int precision, int gtype, int N, int K, const void* host_w, size_t nbytes, const float* bias,
               const float* x, int64_t M, float* y, void* s) {
    return guarded([&] {
        need(host_w && x && y, "null argument");
        need(precision == PKX_PREC_F32 || precision == PKX_PREC_F16, "precision must be F32 or F16");
        pkx::HostTensor t;
        t.gtype = gtype;
        t.n_dims = 2;
        t.ne[0] = K;
        t.ne[1] = N;
        t.bytes.assign((const uint8_t*)host_w, (const uint8_t*)host_w + nbytes);
        pkx::linear_raw((pkx::Precision)precision, t, N, K, bias, x, M, y, st(s));
    });
}

int pkx_linear_residual(int precision, int gtype, int N, int K, const void* host_w, size_t nbytes, const float* bias,
                        const float* x, int64_t M, float alpha, float* y, void* s) {
    return guarded([&] {
        need(host_w && x && y, "null argument");
        need(precision == PKX_PREC_F32 || precision == PKX_PREC_F16, "precision must be F32 or F16");
        pkx::HostTensor t;
        t.gtype = gtype;
        t.n_dims = 2;
        t.ne[0] = K;
        t.ne[1] = N;
        t.bytes.assign((const uint8_t*)host_w, (const uint8_t*)host_w + nbytes);
        pkx::linear_raw((pkx::Precision)precision, t, N, K, bias, x, M, y, st(s), true, alpha);
    });
}

int pkx_layernorm(const float* x, const float* g, const float* b, float* y, int64_t M, int D, float eps,
                  void* s) {
    return guarded([&] {
        need(x && g && b && y, "null argument");
        pkx::LnParams p;
        p.x = x;
        p.g = g;
        p.b = b;
        p.y = y;
        p.M = M;
        p.D = D;
        p.eps = eps;
        pkx::launch_layernorm(pkx::PREC_F32, p, st(s));
    });
}

int pkx_rel_pos_encoding(int T, int D, float* out, void* s) {
    return guarded([&] {
        need(out && T > 0 && D > 0, "bad argument");
        pkx::launch_rel_pos_encoding(pkx::PREC_F32, out, T, D, st(s));
    });
}

int pkx_model_set_profiling(pkx_model* m, unsigned family_mask, int stride) {
    return guarded([&] {
        need(m, "null model");
        m->impl->set_profiling(family_mask, stride);
    });
}

int pkx_model_profile_read(pkx_model* m, double* ms, int64_t* launches) {
    return guarded([&] {
        need(m, "null model");
        m->impl->profile_read(ms, launches);
    });
}

int pkx_transducer_greedy(pkx_model* m, const float* enc, int B, int T_max, const int* T_valid,
                          const int32_t* durations, int n_durations, int blank_id, int max_symbols, int cap,
                          int32_t* ids, int32_t* frames, float* conf, int32_t* span, int* counts, void* s) {
    return guarded([&] {
        need(m && enc, "null argument");
        m->impl->transducer_greedy(enc, B, T_max, T_valid, durations, n_durations, blank_id, max_symbols, cap, ids,
                                   frames, conf, span, counts, st(s));
    });
}
int pkx_streaming_create(pkx_model* m, int n_streams, int max_window, void* s, pkx_streaming** out) {
    return guarded([&] {
        need(m && out, "null argument");
        *out = nullptr;
        std::unique_ptr<pkx_streaming> h(new pkx_streaming);
        h->model = m->impl.get();
        h->st = h->model->stream_create(n_streams, max_window, st(s));
        *out = h.release();
    });
}
int pkx_streaming_free(pkx_streaming* h) {
    return guarded([&] { delete h; });
}
int pkx_streaming_reset(pkx_streaming* h, void* s) {
    return guarded([&] {
        need(h, "null argument");
        h->model->stream_reset(*h->st, st(s));
    });
}
int pkx_streaming_info(const pkx_streaming* h, int* chunk_first, int* chunk, int* pre_cache, int* valid_out_len,
                       int* step) {
    return guarded([&] {
        need(h, "null argument");
        const pkx::ModelConfig& c = h->model->config();
        if (chunk_first) *chunk_first = c.stream_chunk_first;
        if (chunk) *chunk = c.stream_chunk;
        if (pre_cache) *pre_cache = c.stream_pre_cache;
        if (valid_out_len) *valid_out_len = c.stream_valid_out_len;
        if (step) *step = h->st->step;
    });
}
int pkx_streaming_chunk_len(const pkx_streaming* h, int n) { return h ? h->model->stream_chunk_len(*h->st, n) : -1; }
int pkx_streaming_step(pkx_streaming* h, const float* mel, int n, int is_last, float* out, int* n_valid, void* s) {
    return guarded([&] {
        need(h && mel && out && n_valid, "null argument");
        *n_valid = h->model->stream_step(*h->st, mel, n, is_last != 0, out, st(s));
    });
}
int pkx_mel_create(const pkx_mel_config* cfg, const float* window, int window_len, const float* fb,
                   pkx_mel** out) {
    return guarded([&] {
        need(cfg && out && window && fb, "null argument");
        *out = nullptr;
        pkx::MelConfig c;
        c.n_fft = cfg->n_fft;
        c.win_length = window_len;
        c.hop = cfg->hop_length;
        c.n_mels = cfg->n_mels;
        c.per_feature = cfg->per_feature ? 1 : 0;
        c.preemph = cfg->preemph;
        c.mag_power = cfg->mag_power;
        c.log_guard = cfg->log_zero_guard;
        std::unique_ptr<pkx_mel> h(new pkx_mel);
        h->impl.reset(new pkx::MelFront(c, window, window_len, fb));
        *out = h.release();
    });
}
int pkx_mel_load_gguf(const char* path, pkx_mel** out) {
    return guarded([&] {
        need(path && out, "null argument");
        *out = nullptr;
        pkx::MelConfig c;
        std::vector<float> window, fb;
        pkx::load_mel_gguf(path, c, window, fb);
        std::unique_ptr<pkx_mel> h(new pkx_mel);
        h->impl.reset(new pkx::MelFront(c, window.data(), (int)window.size(), fb.data()));
        *out = h.release();
    });
}
int pkx_mel_free(pkx_mel* m) {
    return guarded([&] { delete m; });
}
int pkx_mel_info(const pkx_mel* m, pkx_mel_config* cfg) {
    return guarded([&] {
        need(m && cfg, "null argument");
        const pkx::MelConfig& c = m->impl->config();
        cfg->n_fft = c.n_fft;
        cfg->win_length = c.win_length;
        cfg->hop_length = c.hop;
        cfg->n_mels = c.n_mels;
        cfg->per_feature = c.per_feature;
        cfg->preemph = c.preemph;
        cfg->mag_power = c.mag_power;
        cfg->log_zero_guard = c.log_guard;
    });
}
int pkx_mel_frames(const pkx_mel* m, int n_samples) { return m ? m->impl->frames(n_samples) : -1; }
int pkx_mel_forward(pkx_mel* m, const float* pcm, int B, int64_t S_stride, const int* n_samples, float* mel,
                    int T_max, int* T_out, void* s) {
    return guarded([&] {
        need(m != nullptr, "null mel handle");
        m->impl->forward(pcm, B, S_stride, n_samples, mel, T_max, T_out, st(s));
    });
}

int pkx_quantize(int gtype, const float* src, void* dst, int64_t n_rows, int64_t n_per_row, void* s) {
    return guarded([&] {
        need(src && dst, "null buffer");
        pkx::quantize_rows(gtype, src, dst, n_rows, n_per_row, st(s));
    });
}
int pkx_quantize_gguf(const char* in_path, const char* out_path, int gtype, int* n_quantized, int* n_kept,
                      int* n_skipped) {
    return guarded([&] {
        need(in_path && out_path, "null path");
        const pkx::QuantizeCounts c = pkx::quantize_gguf(in_path, out_path, gtype);
        if (n_quantized) *n_quantized = c.quantized;
        if (n_kept) *n_kept = c.kept;
        if (n_skipped) *n_skipped = c.skipped;
    });
}

}  // extern "C"

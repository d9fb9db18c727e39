// Host classes of the encoder path (include/pk_encoder.hpp) over the pkx C ABI.
// Each call stages host vectors into grow-only device buffers owned by the
// loader, runs the device path on the loader's stream and copies the result
// back.  Plain C++17; the only device interface is pkx.h.
#include "pk_encoder.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>

namespace pk {

namespace {

void chk(int rc, const char* what) {
    if (rc != 0) throw std::runtime_error(std::string(what) + ": " + pkx_last_error());
}

void need(bool ok, const std::string& msg) {
    if (!ok) throw std::invalid_argument(msg);
}

// The caller's positional table is used as given (uploaded with the input),
// as the reference's graph takes pos_emb as a leaf (src/conformer.cpp:359-424):
// only its shape is checked, [pos_len = 2T-1][d_model].
void check_pos_emb(const std::vector<float>& pe, int T, int pos_len, int d) {
    need(T >= 1 && pos_len == 2 * T - 1, "pos_emb: pos_len must be 2T-1");
    need(pe.size() == (size_t)pos_len * d, "pos_emb: size must be pos_len * d_model");
}

// One GGUF KV value as read through pkx_gguf_read_kv.
struct Kv {
    int type = 0, elem = 0;
    std::vector<uint8_t> raw;            // packed little-endian numbers / bools
    std::vector<std::string> strs;       // strings
    uint64_t n = 0;
};

void collect_kv(void* user, const char* key, int type, int elem, uint64_t n, const void* data) {
    auto& kv = *static_cast<std::map<std::string, Kv>*>(user);
    Kv v;
    v.type = type;
    v.elem = elem;
    v.n = n;
    if (elem == 8) {   // GGUF string
        const pkx_gguf_str* s = static_cast<const pkx_gguf_str*>(data);
        for (uint64_t i = 0; i < n; ++i) v.strs.emplace_back(s[i].s, s[i].n);
    } else {
        const size_t es = elem == 0 || elem == 1 || elem == 7 ? 1 : elem == 2 || elem == 3 ? 2
                        : elem == 10 || elem == 11 || elem == 12 ? 8 : 4;
        v.raw.assign(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + n * es);
    }
    kv[key] = std::move(v);
}

int64_t kv_int_at(const Kv& v, uint64_t i) {
    const uint8_t* p = v.raw.data();
    switch (v.elem) {
    case 0: case 7: return p[i];
    case 1: return (int8_t)p[i];
    case 2: { uint16_t x; std::memcpy(&x, p + 2 * i, 2); return x; }
    case 3: { int16_t x; std::memcpy(&x, p + 2 * i, 2); return x; }
    case 4: { uint32_t x; std::memcpy(&x, p + 4 * i, 4); return x; }
    case 5: { int32_t x; std::memcpy(&x, p + 4 * i, 4); return x; }
    case 10: { uint64_t x; std::memcpy(&x, p + 8 * i, 8); return (int64_t)x; }
    case 11: { int64_t x; std::memcpy(&x, p + 8 * i, 8); return x; }
    default: return 0;
    }
}

// ParakeetConfig from the GGUF header: the keys and defaults of
// pk::ModelLoader::load (src/model_loader.cpp:99-156).
bool read_config(const std::string& path, ParakeetConfig& c) {
    std::map<std::string, Kv> kv;
    if (pkx_gguf_read_kv(path.c_str(), collect_kv, &kv) != 0) return false;
    auto find = [&](const char* k) -> const Kv* {
        auto it = kv.find(k);
        return it == kv.end() || it->second.n == 0 ? nullptr : &it->second;
    };
    auto u32 = [&](const char* k, uint32_t d = 0) -> uint32_t {
        const Kv* v = find(k);
        return v && v->elem != 8 && v->elem != 6 ? (uint32_t)kv_int_at(*v, 0) : d;
    };
    auto i32 = [&](const char* k, int32_t d = 0) -> int32_t {
        const Kv* v = find(k);
        return v && v->elem != 8 && v->elem != 6 ? (int32_t)kv_int_at(*v, 0) : d;
    };
    auto f32 = [&](const char* k, float d = 0.0f) -> float {
        const Kv* v = find(k);
        if (!v || v->elem != 6) return d;
        float x;
        std::memcpy(&x, v->raw.data(), 4);
        return x;
    };
    auto bln = [&](const char* k, bool d = false) -> bool {
        const Kv* v = find(k);
        return v && v->elem == 7 ? v->raw[0] != 0 : d;
    };
    auto str = [&](const char* k, const char* d = "") -> std::string {
        const Kv* v = find(k);
        return v && v->type == 8 ? v->strs[0] : std::string(d);
    };
    auto i32_arr = [&](const char* k) -> std::vector<int32_t> {
        std::vector<int32_t> out;
        auto it = kv.find(k);
        if (it != kv.end() && it->second.type == 9 && it->second.elem == 5)
            for (uint64_t i = 0; i < it->second.n; ++i) out.push_back((int32_t)kv_int_at(it->second, i));
        return out;
    };
    c.arch = str("parakeet.arch");
    c.feat_in = u32("parakeet.encoder.feat_in");
    c.d_model = u32("parakeet.encoder.d_model");
    c.n_layers = u32("parakeet.encoder.n_layers");
    c.n_heads = u32("parakeet.encoder.n_heads");
    c.ff_dim = u32("parakeet.encoder.ff_dim");
    c.conv_kernel = u32("parakeet.encoder.conv_kernel");
    c.conv_norm_type = str("parakeet.encoder.conv_norm_type", "batch_norm");
    c.subsampling_factor = u32("parakeet.encoder.subsampling_factor");
    c.subsampling_conv_channels = u32("parakeet.encoder.subsampling_conv_channels");
    c.xscaling = bln("parakeet.encoder.xscaling", true);
    c.pos_emb_max_len = u32("parakeet.encoder.pos_emb_max_len", 5000);
    c.att_context_left = i32("parakeet.encoder.att_context_left", -1);
    c.att_context_right = i32("parakeet.encoder.att_context_right", -1);
    c.att_context_style = str("parakeet.encoder.att_context_style", "regular");
    c.causal_downsampling = bln("parakeet.encoder.causal_downsampling", false);
    c.conv_causal = bln("parakeet.encoder.conv_causal", false);
    c.streaming = StreamingCfg();
    if (c.att_context_style != "regular") {
        StreamingCfg& s = c.streaming;
        s.chunk_size = i32_arr("parakeet.streaming.chunk_size");
        s.shift_size = i32_arr("parakeet.streaming.shift_size");
        s.pre_encode_cache_size = i32_arr("parakeet.streaming.pre_encode_cache_size");
        s.cache_drop_size = i32("parakeet.streaming.cache_drop_size", 0);
        s.last_channel_cache_size = i32("parakeet.streaming.last_channel_cache_size", 0);
        s.valid_out_len = i32("parakeet.streaming.valid_out_len", 0);
        s.drop_extra_pre_encoded = i32("parakeet.streaming.drop_extra_pre_encoded", 0);
        s.present = true;
    }
    c.sample_rate = u32("parakeet.preprocessor.sample_rate", 16000);
    c.n_mels = u32("parakeet.preprocessor.n_mels");
    c.n_fft = u32("parakeet.preprocessor.n_fft");
    c.win_length = u32("parakeet.preprocessor.win_length");
    c.hop_length = u32("parakeet.preprocessor.hop_length");
    c.preemph = f32("parakeet.preprocessor.preemph", 0.0f);
    c.mag_power = f32("parakeet.preprocessor.mag_power", 2.0f);
    c.normalize = str("parakeet.preprocessor.normalize", "per_feature");
    c.log_zero_guard = f32("parakeet.preprocessor.log_zero_guard", 0.0f);
    c.pred_hidden = u32("parakeet.decoder.pred_hidden");
    c.pred_rnn_layers = u32("parakeet.decoder.pred_rnn_layers");
    c.joint_hidden = u32("parakeet.joint.joint_hidden");
    c.joint_activation = str("parakeet.joint.activation");
    c.max_symbols = u32("parakeet.decoding.max_symbols", 10);
    c.vocab_size = u32("parakeet.vocab_size");
    c.blank_id = u32("parakeet.blank_id");
    c.tdt_durations = i32_arr("parakeet.tdt.durations");
    auto tp = kv.find("parakeet.tokenizer.pieces");
    c.tokenizer_pieces.clear();
    if (tp != kv.end() && tp->second.type == 9 && tp->second.elem == 8) c.tokenizer_pieces = tp->second.strs;
    return true;
}

}  // namespace

struct ModelLoader::Device {
    struct Buf {
        void* p = nullptr;
        size_t n = 0;
    };
    void* stream = nullptr;
    std::mutex mu;
    Buf in, out, aux, cap, meta, pos;

    void* get(Buf& b, size_t bytes) {
        if (bytes == 0) bytes = 1;
        if (b.n < bytes) {
            if (b.p) pkx_free(b.p);
            b.p = nullptr;
            b.n = 0;
            chk(pkx_malloc(&b.p, bytes), "pkx_malloc");
            b.n = bytes;
        }
        return b.p;
    }
    void h2d(void* dst, const void* src, size_t bytes) { chk(pkx_memcpy_h2d(dst, src, bytes, stream), "h2d"); }
    void d2h(void* dst, const void* src, size_t bytes) { chk(pkx_memcpy_d2h(dst, src, bytes, stream), "d2h"); }
    void sync() { chk(pkx_stream_synchronize(stream), "synchronize"); }
    ~Device() {
        for (Buf* b : {&in, &out, &aux, &cap, &meta, &pos})
            if (b->p) pkx_free(b->p);
        if (stream) pkx_stream_destroy(stream);
    }
};

// ---------------------------------------------------------------------------
// ModelLoader
// ---------------------------------------------------------------------------
ModelLoader::ModelLoader() = default;

ModelLoader::~ModelLoader() {
    dev_.reset();
    if (mel_) pkx_mel_free(mel_);
    if (model_) pkx_model_free(model_);
}

bool ModelLoader::load(const std::string& path, int precision) {
    if (model_) {
        err_ = "ModelLoader::load: already loaded";
        std::fprintf(stderr, "[pk] %s\n", err_.c_str());
        return false;
    }
    pkx_model* m = nullptr;
    if (pkx_model_load_gguf(path.c_str(), precision, &m) != 0) {
        err_ = std::string("gguf load failed: ") + path + ": " + pkx_last_error();
        std::fprintf(stderr, "[pk] %s\n", err_.c_str());
        return false;
    }
    pkx_config c{};
    int prec = 0, has_ctc = 0, has_joint = 0;
    auto dev = std::make_unique<Device>();
    if (pkx_model_info(m, &c, &prec, &has_ctc, &has_joint) != 0 || pkx_stream_create(&dev->stream) != 0) {
        err_ = std::string("device set-up failed: ") + pkx_last_error();
        std::fprintf(stderr, "[pk] %s\n", err_.c_str());
        pkx_model_free(m);
        return false;
    }
    ParakeetConfig pc;
    if (!read_config(path, pc)) {
        err_ = std::string("gguf KV read failed: ") + path + ": " + pkx_last_error();
        std::fprintf(stderr, "[pk] %s\n", err_.c_str());
        pkx_model_free(m);
        return false;
    }
    cfg_ = std::move(pc);
    precision_ = prec;
    model_ = m;
    dev_ = std::move(dev);
    err_.clear();
    // the front end is optional: encoder-only files carry no featurizer
    if (pkx_mel_load_gguf(path.c_str(), &mel_) != 0) {
        mel_ = nullptr;
        mel_err_ = pkx_last_error();
    }
    return true;
}

static ModelLoader::Device& dev_of(const ModelLoader& ml) {
    need(ml.handle() != nullptr, "model not loaded");
    return ml.device();
}

// ---------------------------------------------------------------------------
// Encoder
// ---------------------------------------------------------------------------
Encoder::Encoder(const ModelLoader& ml)
    : ml_(ml), d_model_(ml.config().d_model), n_layers_(ml.config().n_layers), xscaling_(ml.config().xscaling) {
    need(ml.handle() != nullptr, "Encoder: model not loaded");
}

void Encoder::forward(const std::vector<float>& mel, int n_mels, int T, std::vector<float>& enc_out,
                      int& d_model, int& Tout) const {
    std::vector<std::vector<float>> none;
    forward_capture(mel, n_mels, T, enc_out, d_model, Tout, {}, none);
}

void Encoder::forward_capture(const std::vector<float>& mel, int n_mels, int T, std::vector<float>& enc_out,
                              int& d_model, int& Tout, const std::vector<int>& capture_layers,
                              std::vector<std::vector<float>>& layer_outs) const {
    need(n_mels == (int)ml_.config().feat_in, "Encoder::forward: n_mels does not match the model");
    need(T >= 1 && mel.size() == (size_t)n_mels * T, "Encoder::forward: mel must be [n_mels][T]");
    for (int l : capture_layers) need(l >= 0 && l < n_layers_, "Encoder::forward_capture: layer out of range");
    ModelLoader::Device& d = dev_of(ml_);
    std::lock_guard<std::mutex> lock(d.mu);
    const int Tp = pkx_subsampled_len(T), D = d_model_;
    float* dmel = (float*)d.get(d.in, mel.size() * 4);
    float* dout = (float*)d.get(d.out, (size_t)Tp * D * 4);
    float* dcf = (float*)d.get(d.aux, (size_t)Tp * D * 4);
    float* dcap = capture_layers.empty() ? nullptr : (float*)d.get(d.cap, (size_t)n_layers_ * Tp * D * 4);
    struct { int32_t v; int32_t pad; int64_t off; } meta{0, 0, 0};
    char* dmeta = (char*)d.get(d.meta, sizeof(meta));
    d.h2d(dmel, mel.data(), mel.size() * 4);
    int tout = 0, vout = 0;
    // B=1 path: the scalar subsampling graph (src/encoder.cpp:30-95).
    chk(pkx_encoder_forward(ml_.handle(), dmel, 1, T, nullptr, PKX_MASK_SCALAR, dout, &tout, &vout, dcap, d.stream),
        "pkx_encoder_forward");
    // full-width channels-first transpose (src/encoder.cpp:84-86)
    meta.v = tout;
    d.h2d(dmeta, &meta, sizeof(meta));
    chk(pkx_compact_channels_first(dout, 1, tout, D, (const int*)dmeta, (const int64_t*)(dmeta + 8), dcf, d.stream),
        "pkx_compact_channels_first");
    enc_out.resize((size_t)D * tout);
    d.d2h(enc_out.data(), dcf, enc_out.size() * 4);
    layer_outs.assign(capture_layers.size(), {});
    for (size_t i = 0; i < capture_layers.size(); ++i) {
        layer_outs[i].resize((size_t)tout * D);
        d.d2h(layer_outs[i].data(), dcap + (size_t)capture_layers[i] * tout * D, layer_outs[i].size() * 4);
    }
    d.sync();
    d_model = D;
    Tout = tout;
}

void Encoder::forward_batch(const MelBatch& mels, std::vector<std::vector<float>>& enc_outs, int& d_model,
                            int& Tout, std::vector<int>& valid_Tout) const {
    const int B = mels.B, F = mels.n_mels, T = mels.T_max, D = d_model_;
    need(B >= 1 && T >= 1, "Encoder::forward_batch: empty batch");
    need(F == (int)ml_.config().feat_in, "Encoder::forward_batch: n_mels does not match the model");
    need(mels.data.size() == (size_t)B * F * T, "Encoder::forward_batch: data must be [B][n_mels][T_max]");
    need(mels.valid_T.size() == (size_t)B, "Encoder::forward_batch: valid_T must have B entries");
    ModelLoader::Device& d = dev_of(ml_);
    std::lock_guard<std::mutex> lock(d.mu);
    const int Tp = pkx_subsampled_len(T);
    float* dmel = (float*)d.get(d.in, mels.data.size() * 4);
    float* dout = (float*)d.get(d.out, (size_t)B * Tp * D * 4);
    float* dcf = (float*)d.get(d.aux, (size_t)B * Tp * D * 4);
    d.h2d(dmel, mels.data.data(), mels.data.size() * 4);
    int tout = 0;
    std::vector<int> vo(B);
    chk(pkx_encoder_forward(ml_.handle(), dmel, B, T, mels.valid_T.data(), PKX_MASK_BATCHED, dout, &tout,
                            vo.data(), nullptr, d.stream),
        "pkx_encoder_forward");
    // per-item compaction to [d_model][valid_Tout[b]] (src/encoder.cpp:158-166)
    std::vector<char> meta((size_t)B * 4 + 8 + (size_t)B * 8, 0);
    std::vector<int64_t> offs(B);
    int64_t total = 0;
    for (int b = 0; b < B; ++b) {
        offs[b] = total;
        total += (int64_t)vo[b] * D;
    }
    const size_t off_pos = ((size_t)B * 4 + 7) / 8 * 8;
    std::memcpy(meta.data(), vo.data(), (size_t)B * 4);
    std::memcpy(meta.data() + off_pos, offs.data(), (size_t)B * 8);
    char* dmeta = (char*)d.get(d.meta, meta.size());
    d.h2d(dmeta, meta.data(), meta.size());
    chk(pkx_compact_channels_first(dout, B, tout, D, (const int*)dmeta, (const int64_t*)(dmeta + off_pos), dcf,
                                   d.stream),
        "pkx_compact_channels_first");
    std::vector<float> flat((size_t)total);
    d.d2h(flat.data(), dcf, flat.size() * 4);
    d.sync();
    enc_outs.assign(B, {});
    for (int b = 0; b < B; ++b)
        enc_outs[b].assign(flat.begin() + offs[b], flat.begin() + offs[b] + (int64_t)vo[b] * D);
    d_model = D;
    Tout = tout;
    valid_Tout = vo;
}

// ---------------------------------------------------------------------------
// Subsampling
// ---------------------------------------------------------------------------
Subsampling::Subsampling(const ModelLoader& ml) : ml_(ml), d_model_(ml.config().d_model) {
    need(ml.handle() != nullptr, "Subsampling: model not loaded");
}

void Subsampling::forward(const std::vector<float>& mel, int n_mels, int T, std::vector<float>& out, int& Tout,
                          int& d_model) const {
    int v = 0;
    forward(mel, n_mels, T, out, Tout, d_model, v, -1);
}

void Subsampling::forward(const std::vector<float>& mel, int n_mels, int T, std::vector<float>& out, int& Tout,
                          int& d_model, int& valid_len) const {
    forward(mel, n_mels, T, out, Tout, d_model, valid_len, -1);
}

void Subsampling::forward(const std::vector<float>& mel, int n_mels, int T, std::vector<float>& out, int& Tout,
                          int& d_model, int& valid_len, int in_valid_frames) const {
    need(n_mels == (int)ml_.config().feat_in, "Subsampling::forward: n_mels does not match the model");
    need(T >= 1 && mel.size() == (size_t)n_mels * T, "Subsampling::forward: mel must be [n_mels][T]");
    need(in_valid_frames <= T, "Subsampling::forward: in_valid_frames must be at most T (the window's frames)");
    ModelLoader::Device& d = dev_of(ml_);
    std::lock_guard<std::mutex> lock(d.mu);
    const int Tp = pkx_subsampled_len(T), D = d_model_;
    float* dmel = (float*)d.get(d.in, mel.size() * 4);
    float* dout = (float*)d.get(d.out, (size_t)Tp * D * 4);
    d.h2d(dmel, mel.data(), mel.size() * 4);
    // The C ABI takes true frame counts (entry valid length one less); a whole
    // window (in_valid_frames == T, the streaming convention) goes as an entry
    // valid length of its own.
    const bool whole = in_valid_frames == T;
    const int vT = in_valid_frames < 0 ? T : whole ? T : in_valid_frames + 1;
    int tout = 0, vo = 0;
    chk(pkx_subsampling_forward(ml_.handle(), dmel, 1, T, &vT, PKX_MASK_SCALAR | (whole ? PKX_MASK_WHOLE_FRAMES : 0),
                                dout, &tout, &vo, d.stream),
        "pkx_subsampling_forward");
    out.resize((size_t)tout * D);
    d.d2h(out.data(), dout, out.size() * 4);
    d.sync();
    Tout = tout;
    d_model = D;
    valid_len = vo;
}

void Subsampling::forward_batch(const float* mel, int n_mels, int T, int B, const std::vector<int>& valid_in,
                                std::vector<float>& out, int& Tp, std::vector<int>& valid_out) const {
    need(mel != nullptr && B >= 1 && T >= 1, "Subsampling::forward_batch: empty batch");
    need(n_mels == (int)ml_.config().feat_in, "Subsampling::forward_batch: n_mels does not match the model");
    need(valid_in.size() == (size_t)B, "Subsampling::forward_batch: valid_in must have B entries");
    std::vector<int> vT(B);
    for (int b = 0; b < B; ++b) {
        need(valid_in[b] <= T - 1, "Subsampling::forward_batch: valid_in[b] must be <= T-1");
        vT[b] = valid_in[b] < 0 ? T : valid_in[b] + 1;
    }
    ModelLoader::Device& d = dev_of(ml_);
    std::lock_guard<std::mutex> lock(d.mu);
    const int tp = pkx_subsampled_len(T), D = d_model_;
    const size_t nmel = (size_t)B * n_mels * T;
    float* dmel = (float*)d.get(d.in, nmel * 4);
    float* dout = (float*)d.get(d.out, (size_t)B * tp * D * 4);
    d.h2d(dmel, mel, nmel * 4);
    int tout = 0;
    std::vector<int> vo(B);
    chk(pkx_subsampling_forward(ml_.handle(), dmel, B, T, vT.data(), PKX_MASK_BATCHED, dout, &tout, vo.data(),
                                d.stream),
        "pkx_subsampling_forward");
    out.resize((size_t)B * tout * D);
    d.d2h(out.data(), dout, out.size() * 4);
    d.sync();
    Tp = tout;
    valid_out = vo;
}

int Subsampling::valid_out_len(int T, int in_valid_frames) const { return pkx_valid_out_len(T, in_valid_frames); }

// ---------------------------------------------------------------------------
// ConformerLayer / RelPosAttention
// ---------------------------------------------------------------------------
namespace {

enum class Unit { Layer, Attention, Conv };

void run_unit(const ModelLoader& ml, Unit u, int layer, const std::vector<float>& x, int T, int B,
              const std::vector<int>& valid, std::vector<float>& out, std::vector<float>* conv_out,
              const std::vector<float>* pos_emb = nullptr) {
    const int D = ml.config().d_model;
    need(T >= 1 && B >= 1 && x.size() == (size_t)B * T * D, "input must be [B][T][d_model]");
    need(valid.size() == (size_t)B, "valid_len must have B entries");
    for (int v : valid) need(v >= 0 && v <= T, "valid_len must be in [0, T]");
    ModelLoader::Device& d = dev_of(ml);
    std::lock_guard<std::mutex> lock(d.mu);
    const size_t n = x.size();
    float* dx = (float*)d.get(d.in, n * 4);
    float* dy = (float*)d.get(d.out, n * 4);
    float* dc = conv_out ? (float*)d.get(d.aux, n * 4) : nullptr;
    float* dpe = pos_emb ? (float*)d.get(d.pos, pos_emb->size() * 4) : nullptr;
    d.h2d(dx, x.data(), n * 4);
    if (pos_emb) d.h2d(dpe, pos_emb->data(), pos_emb->size() * 4);
    switch (u) {
    case Unit::Layer:
        chk(pkx_conformer_layer_forward(ml.handle(), layer, dx, B, T, valid.data(), dpe, dy, dc, d.stream),
            "pkx_conformer_layer_forward");
        break;
    case Unit::Attention:
        chk(pkx_relpos_attention_forward(ml.handle(), layer, dx, B, T, valid.data(), dpe, dy, d.stream),
            "pkx_relpos_attention_forward");
        break;
    case Unit::Conv:
        chk(pkx_conv_module_forward(ml.handle(), layer, dx, B, T, valid.data(), dy, d.stream),
            "pkx_conv_module_forward");
        break;
    }
    out.resize(n);
    d.d2h(out.data(), dy, n * 4);
    if (conv_out) {
        conv_out->resize(n);
        d.d2h(conv_out->data(), dc, n * 4);
    }
    d.sync();
}

}  // namespace

ConformerLayer::ConformerLayer(const ModelLoader& ml, int layer_idx)
    : ml_(ml), layer_idx_(layer_idx), d_model_(ml.config().d_model) {
    need(ml.handle() != nullptr, "ConformerLayer: model not loaded");
    need(layer_idx >= 0 && layer_idx < (int)ml.config().n_layers, "ConformerLayer: layer index out of range");
}

void ConformerLayer::forward(const std::vector<float>& x, int T, const std::vector<float>& pos_emb, int pos_len,
                             int valid_len, std::vector<float>& out) const {
    check_pos_emb(pos_emb, T, pos_len, d_model_);
    run_unit(ml_, Unit::Layer, layer_idx_, x, T, 1, {valid_len}, out, nullptr, &pos_emb);
}

void ConformerLayer::forward_with_conv(const std::vector<float>& x, int T, const std::vector<float>& pos_emb,
                                       int pos_len, int valid_len, std::vector<float>& out,
                                       std::vector<float>& conv_out) const {
    check_pos_emb(pos_emb, T, pos_len, d_model_);
    run_unit(ml_, Unit::Layer, layer_idx_, x, T, 1, {valid_len}, out, &conv_out, &pos_emb);
}

void ConformerLayer::conv_module_forward(const std::vector<float>& conv_in, int T, int valid_len,
                                         std::vector<float>& out) const {
    run_unit(ml_, Unit::Conv, layer_idx_, conv_in, T, 1, {valid_len}, out, nullptr);
}

void ConformerLayer::forward_batch(const std::vector<float>& x, int T, int B, const std::vector<float>& pos_emb,
                                   int pos_len, const std::vector<int>& valid_len, std::vector<float>& out) const {
    check_pos_emb(pos_emb, T, pos_len, d_model_);
    run_unit(ml_, Unit::Layer, layer_idx_, x, T, B, valid_len, out, nullptr, &pos_emb);
}

RelPosAttention::RelPosAttention(const ModelLoader& ml, int layer_idx)
    : ml_(ml), layer_idx_(layer_idx), d_model_(ml.config().d_model) {
    need(ml.handle() != nullptr, "RelPosAttention: model not loaded");
    need(layer_idx >= 0 && layer_idx < (int)ml.config().n_layers, "RelPosAttention: layer index out of range");
}

void RelPosAttention::forward(const std::vector<float>& x, int T, const std::vector<float>& pos_emb, int pos_len,
                              int valid_len, std::vector<float>& out) const {
    check_pos_emb(pos_emb, T, pos_len, d_model_);
    run_unit(ml_, Unit::Attention, layer_idx_, x, T, 1, {valid_len}, out, nullptr, &pos_emb);
}

void RelPosAttention::forward_batch(const std::vector<float>& x, int T, int B, const std::vector<float>& pos_emb,
                                    int pos_len, const std::vector<int>& valid_len, std::vector<float>& out) const {
    check_pos_emb(pos_emb, T, pos_len, d_model_);
    run_unit(ml_, Unit::Attention, layer_idx_, x, T, B, valid_len, out, nullptr, &pos_emb);
}

// ---------------------------------------------------------------------------
void rel_pos_encoding(int T, int d_model, std::vector<float>& out) {
    need(T >= 1 && d_model >= 2 && d_model % 2 == 0, "rel_pos_encoding: T >= 1 and even d_model");
    const size_t n = (size_t)(2 * T - 1) * d_model;
    void* dp = nullptr;
    chk(pkx_malloc(&dp, n * 4), "pkx_malloc");
    int rc = pkx_rel_pos_encoding(T, d_model, (float*)dp, nullptr);
    out.resize(n);
    if (rc == 0) rc = pkx_memcpy_d2h(out.data(), dp, n * 4, nullptr);
    if (rc == 0) rc = pkx_stream_synchronize(nullptr);
    const std::string msg = rc ? pkx_last_error() : "";
    pkx_free(dp);
    if (rc) throw std::runtime_error("rel_pos_encoding: " + msg);
}

}  // namespace pk

namespace pk {

// ---------------------------------------------------------------------------
// MelFrontend / build_mel_batch
// ---------------------------------------------------------------------------
static pkx_mel* mel_of(const ModelLoader& ml) {
    need(ml.handle() != nullptr, "model not loaded");
    need(ml.mel_handle() != nullptr, "no log-mel front end in this model: " + ml.mel_error());
    return ml.mel_handle();
}

// ---------------------------------------------------------------------------
// StreamingEncoder (streaming_encoder.hpp:33-95) over pkx_streaming_*
// ---------------------------------------------------------------------------
StreamingEncoder::StreamingEncoder(const ModelLoader& ml) : ml_(ml) {
    need(ml.handle() != nullptr, "StreamingEncoder: model not loaded");
    need(ml.config().streaming.present, "StreamingEncoder requires a streaming model");
    d_model_ = ml.config().d_model;
    n_mels_ = ml.config().feat_in;
    int pc = 0, ch = 0, cf = 0, vo = 0;
    ModelLoader::Device& d = ml.device();
    std::lock_guard<std::mutex> lock(d.mu);
    // the longest window the schedule produces: pre-encode overlap + a later chunk
    max_window_ = std::max(ml.config().streaming.chunk_size[0],
                           ml.config().streaming.pre_encode_cache_size[1] + ml.config().streaming.chunk_size[1]);
    chk(pkx_streaming_create(ml.handle(), 1, max_window_, d.stream, &st_), "pkx_streaming_create");
    chk(pkx_streaming_info(st_, &cf, &ch, &pc, &vo, nullptr), "pkx_streaming_info");
    chunk_first_ = cf;
    chunk_main_ = ch;
    pre_cache_ = pc;
    valid_out_len_ = vo;
    chk(pkx_malloc(&mel_dev_, (size_t)n_mels_ * max_window_ * 4), "pkx_malloc");
    chk(pkx_malloc(&out_dev_, (size_t)pkx_streaming_chunk_len(st_, max_window_) * d_model_ * 4), "pkx_malloc");
}

StreamingEncoder::~StreamingEncoder() {
    if (st_) pkx_streaming_free(st_);
    if (mel_dev_) pkx_free(mel_dev_);
    if (out_dev_) pkx_free(out_dev_);
}

void StreamingEncoder::reset() {
    ModelLoader::Device& d = ml_.device();
    std::lock_guard<std::mutex> lock(d.mu);
    chk(pkx_streaming_reset(st_, d.stream), "pkx_streaming_reset");
    d.sync();
}

int StreamingEncoder::step_num() const {
    int s = 0;
    chk(pkx_streaming_info(st_, nullptr, nullptr, nullptr, nullptr, &s), "pkx_streaming_info");
    return s;
}

std::vector<float> StreamingEncoder::step(const std::vector<float>& mel, int n, bool is_last, int& n_valid_out) {
    need((int64_t)mel.size() == (int64_t)n_mels_ * n, "StreamingEncoder::step: mel size != n_mels * n_mel_frames");
    need(n >= 1 && n <= max_window_, "StreamingEncoder::step: window longer than the schedule's");
    ModelLoader::Device& d = ml_.device();
    std::lock_guard<std::mutex> lock(d.mu);
    d.h2d(mel_dev_, mel.data(), mel.size() * 4);
    int nv = 0;
    chk(pkx_streaming_step(st_, (const float*)mel_dev_, n, is_last ? 1 : 0, (float*)out_dev_, &nv, d.stream),
        "pkx_streaming_step");
    std::vector<float> out((size_t)nv * d_model_);
    if (nv) d.d2h(out.data(), out_dev_, out.size() * 4);
    d.sync();
    n_valid_out = nv;
    return out;
}

MelFrontend::MelFrontend(const ModelLoader& ml) : ml_(ml) { (void)mel_of(ml); }

void MelFrontend::compute(const std::vector<float>& samples, std::vector<float>& feats, int& n_mels,
                          int& T) const {
    MelBatch mb = build_mel_batch(ml_, {samples});
    n_mels = mb.n_mels;
    T = mb.valid_T[0];
    feats.assign(mb.data.begin(), mb.data.begin() + (size_t)n_mels * T);
}

MelBatch build_mel_batch(const ModelLoader& ml, const std::vector<std::vector<float>>& pcms16k) {
    pkx_mel* mel = mel_of(ml);
    pkx_mel_config mc{};
    chk(pkx_mel_info(mel, &mc), "pkx_mel_info");
    MelBatch mb;
    mb.B = (int)pcms16k.size();
    mb.n_mels = mc.n_mels;
    need(mb.B >= 1, "build_mel_batch: empty batch");
    size_t S = 1;
    std::vector<int> ns(mb.B);
    for (int b = 0; b < mb.B; ++b) {
        need(pcms16k[b].size() < (size_t)INT32_MAX, "build_mel_batch: clip too long");
        ns[b] = (int)pcms16k[b].size();
        S = std::max(S, pcms16k[b].size());
        mb.T_max = std::max(mb.T_max, pkx_mel_frames(mel, ns[b]));
    }
    mb.valid_T.assign(mb.B, 0);
    if (mb.T_max == 0) return mb;
    std::vector<float> pcm((size_t)mb.B * S, 0.0f);
    for (int b = 0; b < mb.B; ++b) std::copy(pcms16k[b].begin(), pcms16k[b].end(), pcm.begin() + (size_t)b * S);
    ModelLoader::Device& d = ml.device();
    std::lock_guard<std::mutex> lock(d.mu);
    float* dpcm = (float*)d.get(d.in, pcm.size() * 4);
    float* dout = (float*)d.get(d.out, (size_t)mb.B * mb.n_mels * mb.T_max * 4);
    d.h2d(dpcm, pcm.data(), pcm.size() * 4);
    chk(pkx_mel_forward(mel, dpcm, mb.B, (int64_t)S, ns.data(), dout, mb.T_max, mb.valid_T.data(), d.stream),
        "pkx_mel_forward");
    mb.data.resize((size_t)mb.B * mb.n_mels * mb.T_max);
    d.d2h(mb.data.data(), dout, mb.data.size() * 4);
    d.sync();
    return mb;
}

}  // namespace pk

namespace pk {

// ---------------------------------------------------------------------------
// transducer_greedy_batch
// ---------------------------------------------------------------------------
void transducer_greedy_batch(const ModelLoader& ml, const std::vector<std::vector<float>>& encs,
                             const std::vector<int>& T, int enc_hidden, const std::vector<int32_t>& durations,
                             int blank_id, int max_symbols, std::vector<std::vector<int32_t>>& ids,
                             std::vector<std::vector<TokenInfo>>* toks) {
    need(ml.handle() != nullptr, "model not loaded");
    const int N = (int)encs.size();
    need(N >= 1 && (int)T.size() == N, "transducer_greedy_batch: encs / T size mismatch");
    need(enc_hidden == (int)ml.config().d_model, "transducer_greedy_batch: enc_hidden != d_model");
    int T_max = 1;
    for (int n = 0; n < N; ++n) {
        need(T[n] >= 0 && encs[n].size() >= (size_t)T[n] * enc_hidden, "transducer_greedy_batch: enc too short");
        T_max = std::max(T_max, T[n]);
    }
    // stack to [N][T_max][enc_hidden] (rows past T[n] are never read)
    std::vector<float> stacked((size_t)N * T_max * enc_hidden, 0.0f);
    for (int n = 0; n < N; ++n)
        std::copy(encs[n].begin(), encs[n].begin() + (size_t)T[n] * enc_hidden,
                  stacked.begin() + (size_t)n * T_max * enc_hidden);
    const int cap = T_max * std::max(max_symbols, 1);
    std::vector<int32_t> id((size_t)N * cap), fr((size_t)N * cap), sp((size_t)N * cap);
    std::vector<float> cf((size_t)N * cap);
    std::vector<int> cnt(N);
    ModelLoader::Device& d = ml.device();
    std::lock_guard<std::mutex> lock(d.mu);
    float* denc = (float*)d.get(d.in, stacked.size() * 4);
    d.h2d(denc, stacked.data(), stacked.size() * 4);
    chk(pkx_transducer_greedy(ml.handle(), denc, N, T_max, T.data(), durations.data(), (int)durations.size(),
                              blank_id, max_symbols, cap, id.data(), fr.data(), cf.data(), sp.data(), cnt.data(),
                              d.stream),
        "pkx_transducer_greedy");
    ids.assign(N, {});
    if (toks) toks->assign(N, {});
    for (int n = 0; n < N; ++n) {
        ids[n].assign(id.begin() + (size_t)n * cap, id.begin() + (size_t)n * cap + cnt[n]);
        if (toks)
            for (int i = 0; i < cnt[n]; ++i) {
                const size_t j = (size_t)n * cap + i;
                (*toks)[n].push_back(TokenInfo{id[j], fr[j], cf[j], sp[j]});
            }
    }
}

PredictionNet::PredictionNet(const ModelLoader& ml) : ml_(ml) {
    need(ml.handle() != nullptr, "PredictionNet: model not loaded");
}

Joint::Joint(const ModelLoader& ml) : ml_(ml) { need(ml.handle() != nullptr, "Joint: model not loaded"); }

void transducer_greedy_batch(const PredictionNet& pred, const Joint& joint,
                             const std::vector<std::vector<float>>& encs, const std::vector<int>& T,
                             int enc_hidden, const std::vector<int32_t>& durations, int blank_id, int max_symbols,
                             std::vector<std::vector<int32_t>>& ids, std::vector<std::vector<TokenInfo>>* toks) {
    need(&pred.loader() == &joint.loader(), "transducer_greedy_batch: pred and joint of different models");
    transducer_greedy_batch(pred.loader(), encs, T, enc_hidden, durations, blank_id, max_symbols, ids, toks);
}

}  // namespace pk

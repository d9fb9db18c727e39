// GGUF v3 reader for the encoder path (pk::ModelLoader::load,
// src/model_loader.cpp:99-167): parakeet.* KV -> ModelConfig, verbatim NeMo
// tensor names -> Model::set_tensor.  Only the tensors the encoder, the CTC
// head and the TDT joint use are read; the file is streamed tensor by tensor.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "mel.hpp"
#include "model.hpp"
#include "quantize.hpp"

namespace pkx {
namespace {

enum : uint32_t {
    KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6,
    KV_BOOL = 7, KV_STR = 8, KV_ARR = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12
};

struct File {
    FILE* f = nullptr;
    explicit File(const std::string& p) : f(std::fopen(p.c_str(), "rb")) {
        require(f != nullptr, "cannot open GGUF file: " + p);
    }
    ~File() { if (f) std::fclose(f); }
    void read(void* dst, size_t n) {
        require(std::fread(dst, 1, n, f) == n, "GGUF: truncated file");
    }
    template <typename T> T get() {
        T v;
        read(&v, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        require(n < (1ull << 24), "GGUF: string too long");
        std::string s((size_t)n, '\0');
        if (n) read(&s[0], (size_t)n);
        return s;
    }
    void skip(uint64_t n) { require(std::fseek(f, (long)n, SEEK_CUR) == 0, "GGUF: seek failed"); }
    void seek(uint64_t off) { require(std::fseek(f, (long)off, SEEK_SET) == 0, "GGUF: seek failed"); }
    uint64_t tell() { return (uint64_t)std::ftell(f); }
};

struct KvVal {
    uint32_t type = 0;
    int64_t i = 0;
    double d = 0;
    std::string s;
    std::vector<int64_t> arr;
    uint32_t arr_type = 0;
};

size_t scalar_size(uint32_t t) {
    switch (t) {
    case KV_U8: case KV_I8: case KV_BOOL: return 1;
    case KV_U16: case KV_I16: return 2;
    case KV_U32: case KV_I32: case KV_F32: return 4;
    case KV_U64: case KV_I64: case KV_F64: return 8;
    default: return 0;
    }
}

int64_t read_int(File& f, uint32_t t) {
    switch (t) {
    case KV_U8: return f.get<uint8_t>();
    case KV_I8: return f.get<int8_t>();
    case KV_U16: return f.get<uint16_t>();
    case KV_I16: return f.get<int16_t>();
    case KV_U32: return f.get<uint32_t>();
    case KV_I32: return f.get<int32_t>();
    case KV_U64: return (int64_t)f.get<uint64_t>();
    case KV_I64: return f.get<int64_t>();
    case KV_BOOL: return f.get<uint8_t>() ? 1 : 0;
    default: throw std::invalid_argument("GGUF: not an integer type");
    }
}

KvVal read_val(File& f, uint32_t t) {
    KvVal v;
    v.type = t;
    if (t == KV_STR) {
        v.s = f.str();
    } else if (t == KV_F32) {
        v.d = f.get<float>();
    } else if (t == KV_F64) {
        v.d = f.get<double>();
    } else if (t == KV_ARR) {
        v.arr_type = f.get<uint32_t>();
        const uint64_t n = f.get<uint64_t>();
        if (v.arr_type == KV_STR) {
            for (uint64_t k = 0; k < n; ++k) f.skip(f.get<uint64_t>());   // e.g. tokenizer pieces
        } else if (v.arr_type == KV_F32 || v.arr_type == KV_F64) {
            f.skip(n * scalar_size(v.arr_type));
        } else {
            require(scalar_size(v.arr_type) > 0, "GGUF: bad array element type");
            v.arr.reserve((size_t)n);
            for (uint64_t k = 0; k < n; ++k) v.arr.push_back(read_int(f, v.arr_type));
        }
    } else {
        require(scalar_size(t) > 0, "GGUF: bad KV type " + std::to_string(t));
        v.i = read_int(f, t);
    }
    return v;
}

struct TensorInfo {
    std::string name;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    int gtype = 0;
    uint64_t offset = 0;
};

int64_t tensor_bytes(const TensorInfo& t) {
    int64_t blk = 1, bs = 4;
    switch (t.gtype) {
    case GT_F32: blk = 1; bs = 4; break;
    case GT_F16: blk = 1; bs = 2; break;
    case GT_Q8_0: blk = 32; bs = 34; break;
    case GT_Q4_K: blk = 256; bs = 144; break;
    default: return -1;
    }
    require(t.ne[0] % blk == 0, "GGUF: row not a multiple of the block size in " + t.name);
    return t.ne[0] / blk * bs * t.ne[1] * t.ne[2] * t.ne[3];
}

bool wanted(const std::string& n) {
    auto starts = [&](const char* p) { return n.compare(0, std::strlen(p), p) == 0; };
    return starts("encoder.") || starts("ctc_decoder.") || starts("decoder.decoder_layers.") ||
           starts("decoder.prediction.") ||
           starts("joint.enc.") || starts("joint.pred.") || starts("joint.joint_net.2.");
}

struct Header {
    std::map<std::string, KvVal> kv;
    std::vector<TensorInfo> infos;
    uint64_t data0 = 0;
    uint64_t kv_begin = 0, kv_end = 0, n_kv = 0;   // byte range of the KV section
    uint64_t align = 32;
};

Header read_header(File& f, const std::string& path) {
    require(f.get<uint32_t>() == 0x46554747u, "not a GGUF file: " + path);
    const uint32_t version = f.get<uint32_t>();
    require(version == 3 || version == 2, "unsupported GGUF version " + std::to_string(version));
    const uint64_t n_tensors = f.get<uint64_t>();
    const uint64_t n_kv = f.get<uint64_t>();
    Header h;
    h.n_kv = n_kv;
    h.kv_begin = f.tell();
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = f.str();
        const uint32_t t = f.get<uint32_t>();
        h.kv[key] = read_val(f, t);
    }
    h.kv_end = f.tell();
    h.infos.resize((size_t)n_tensors);
    for (auto& ti : h.infos) {
        ti.name = f.str();
        ti.n_dims = (int)f.get<uint32_t>();
        require(ti.n_dims >= 1 && ti.n_dims <= 4, "GGUF: bad n_dims");
        for (int d = 0; d < ti.n_dims; ++d) ti.ne[d] = (int64_t)f.get<uint64_t>();
        ti.gtype = (int)f.get<uint32_t>();
        ti.offset = f.get<uint64_t>();
    }
    uint64_t align = 32;
    if (h.kv.count("general.alignment")) align = (uint64_t)h.kv["general.alignment"].i;
    require(align > 0 && (align & (align - 1)) == 0, "GGUF: general.alignment must be a power of two");
    h.align = align;
    h.data0 = (f.tell() + align - 1) / align * align;
    return h;
}

// an f32 or f16 tensor read as f32
std::vector<float> read_f32_tensor(File& f, const Header& h, const TensorInfo& ti) {
    require(ti.gtype == GT_F32 || ti.gtype == GT_F16, "GGUF: " + ti.name + " must be f32 or f16");
    const int64_t n = ti.ne[0] * ti.ne[1] * ti.ne[2] * ti.ne[3];
    std::vector<float> out((size_t)n);
    f.seek(h.data0 + ti.offset);
    if (ti.gtype == GT_F32) {
        f.read(out.data(), sizeof(float) * (size_t)n);
    } else {
        std::vector<uint16_t> hb((size_t)n);
        f.read(hb.data(), 2 * (size_t)n);
        for (int64_t i = 0; i < n; ++i) {
            _Float16 hv;   // exact binary16 -> binary32
            std::memcpy(&hv, &hb[(size_t)i], 2);
            out[(size_t)i] = (float)hv;
        }
    }
    return out;
}

}  // namespace

// Every KV pair of the header, in file order, with its value in raw form: the
// key-value half of gguf_init_from_file that pk::ModelLoader::load reads its
// ParakeetConfig from (src/model_loader.cpp:99-156).
void read_gguf_kv(const std::string& path, const KvVisitor& visit) {
    File f(path);
    require(f.get<uint32_t>() == 0x46554747u, "not a GGUF file: " + path);
    const uint32_t version = f.get<uint32_t>();
    require(version == 3 || version == 2, "unsupported GGUF version " + std::to_string(version));
    (void)f.get<uint64_t>();   // tensor count
    const uint64_t n_kv = f.get<uint64_t>();
    std::vector<uint8_t> raw;
    std::vector<std::string> strs;
    for (uint64_t i = 0; i < n_kv; ++i) {
        const std::string key = f.str();
        const uint32_t t = f.get<uint32_t>();
        uint32_t et = t;
        uint64_t n = 1;
        if (t == KV_ARR) {
            et = f.get<uint32_t>();
            n = f.get<uint64_t>();
        }
        strs.clear();
        if (et == KV_STR) {
            require(n < (1ull << 24), "GGUF: string array too long");
            for (uint64_t k = 0; k < n; ++k) strs.push_back(f.str());
            visit(key, (int)t, (int)et, n, nullptr, &strs);
        } else {
            const size_t es = scalar_size(et);
            require(es > 0 && n < (1ull << 28), "GGUF: bad KV value type in " + key);
            raw.resize((size_t)(n * es));
            if (!raw.empty()) f.read(raw.data(), raw.size());
            visit(key, (int)t, (int)et, n, raw.data(), nullptr);
        }
    }
}

void load_mel_gguf(const std::string& path, MelConfig& c, std::vector<float>& window, std::vector<float>& fb) {
    File f(path);
    Header h = read_header(f, path);
    auto has = [&](const char* k) { return h.kv.count(k) > 0; };
    auto u = [&](const char* k, int64_t dflt) -> int64_t { return has(k) ? h.kv[k].i : dflt; };
    auto fl = [&](const char* k, double dflt) -> double { return has(k) ? h.kv[k].d : dflt; };
    // src/model_loader.cpp:133-141 keys and defaults
    require(has("parakeet.preprocessor.n_mels") && has("parakeet.preprocessor.n_fft") &&
                has("parakeet.preprocessor.win_length") && has("parakeet.preprocessor.hop_length"),
            "GGUF: missing parakeet.preprocessor.{n_mels,n_fft,win_length,hop_length}: " + path);
    c.n_mels = (int)u("parakeet.preprocessor.n_mels", 0);
    c.n_fft = (int)u("parakeet.preprocessor.n_fft", 0);
    c.win_length = (int)u("parakeet.preprocessor.win_length", 0);
    c.hop = (int)u("parakeet.preprocessor.hop_length", 0);
    c.preemph = (float)fl("parakeet.preprocessor.preemph", 0.0);
    c.mag_power = (float)fl("parakeet.preprocessor.mag_power", 2.0);
    c.log_guard = (float)fl("parakeet.preprocessor.log_zero_guard", 0.0);
    const std::string norm = has("parakeet.preprocessor.normalize") ? h.kv["parakeet.preprocessor.normalize"].s
                                                                    : std::string("per_feature");
    c.per_feature = norm == "per_feature" ? 1 : 0;
    const TensorInfo* tw = nullptr;
    const TensorInfo* tf = nullptr;
    for (const auto& ti : h.infos) {
        if (ti.name == "preprocessor.featurizer.window") tw = &ti;
        if (ti.name == "preprocessor.featurizer.fb") tf = &ti;
    }
    require(tw && tf, "GGUF: missing preprocessor.featurizer.window / .fb: " + path);
    window = read_f32_tensor(f, h, *tw);
    fb = read_f32_tensor(f, h, *tf);
    // fb: ggml ne [n_bins, n_mels, 1] (src/mel.cpp:50-61)
    require(tf->ne[0] == c.n_fft / 2 + 1 && tf->ne[1] == c.n_mels,
            "GGUF: preprocessor.featurizer.fb must be [n_mels][n_fft/2+1]");
    c.win_length = (int)window.size();
}

std::unique_ptr<Model> load_gguf(const std::string& path, int precision) {
    File f(path);
    Header h = read_header(f, path);
    std::map<std::string, KvVal>& kv = h.kv;
    const std::vector<TensorInfo>& infos = h.infos;
    const uint64_t data0 = h.data0;

    auto u = [&](const char* k, int64_t dflt) -> int64_t {
        auto it = kv.find(k);
        return it == kv.end() ? dflt : it->second.i;
    };
    auto s = [&](const char* k, const char* dflt) -> std::string {
        auto it = kv.find(k);
        return it == kv.end() ? std::string(dflt) : it->second.s;
    };
    // model_loader.cpp:103-161 keys and defaults
    ModelConfig c;
    c.d_model = (int)u("parakeet.encoder.d_model", 0);
    c.n_layers = (int)u("parakeet.encoder.n_layers", 0);
    c.n_heads = (int)u("parakeet.encoder.n_heads", 0);
    c.ff_dim = (int)u("parakeet.encoder.ff_dim", 0);
    c.conv_kernel = (int)u("parakeet.encoder.conv_kernel", 0);
    c.n_mels = (int)u("parakeet.encoder.feat_in", 0);
    c.sub_channels = (int)u("parakeet.encoder.subsampling_conv_channels", 0);
    c.xscaling = (int)u("parakeet.encoder.xscaling", 1);
    c.vocab_size = (int)u("parakeet.vocab_size", 0);
    if (kv.count("parakeet.tdt.durations")) c.n_durations = (int)kv["parakeet.tdt.durations"].arr.size();
    require(c.d_model > 0 && c.vocab_size > 0, "GGUF: missing parakeet.encoder.d_model / parakeet.vocab_size");
    const std::string cnt = s("parakeet.encoder.conv_norm_type", "batch_norm");
    require(cnt == "batch_norm" || cnt == "layer_norm", "conv_norm_type must be batch_norm or layer_norm");
    c.conv_ln = cnt == "layer_norm";
    c.causal_sub = (int)u("parakeet.encoder.causal_downsampling", 0);
    c.conv_causal = (int)u("parakeet.encoder.conv_causal", 0);
    c.att_left = (int)u("parakeet.encoder.att_context_left", -1);
    c.att_right = (int)u("parakeet.encoder.att_context_right", -1);
    const std::string style = s("parakeet.encoder.att_context_style", "regular");
    c.att_limited = style == "chunked_limited" && c.att_right >= 0;
    if (style != "regular") {
        // streaming_encoder.cpp:38-55: [0] for the first chunk, [1] after
        auto arr = [&](const char* k, int idx, int dflt) -> int {
            auto it = kv.find(k);
            return it == kv.end() || (int)it->second.arr.size() <= idx ? dflt : (int)it->second.arr[(size_t)idx];
        };
        c.stream_chunk_first = arr("parakeet.streaming.chunk_size", 0, 9);
        c.stream_chunk = arr("parakeet.streaming.chunk_size", 1, 16);
        c.stream_pre_cache = arr("parakeet.streaming.pre_encode_cache_size", 1, 9);
        c.stream_cache_len = (int)u("parakeet.streaming.last_channel_cache_size", 0);
        c.stream_valid_out_len = (int)u("parakeet.streaming.valid_out_len", 0);
        c.stream_drop_extra = (int)u("parakeet.streaming.drop_extra_pre_encoded", 0);
    }
    const int64_t sf = u("parakeet.encoder.subsampling_factor", 8);
    require(sf == 8, "only dw_striding x8 subsampling is supported");

    std::unique_ptr<Model> m(new Model(c, precision));
    std::vector<uint8_t> buf;
    for (const auto& ti : infos) {
        if (!wanted(ti.name)) continue;
        const int64_t nb = tensor_bytes(ti);
        require(nb >= 0, "GGUF: unsupported type " + std::to_string(ti.gtype) + " for tensor " + ti.name);
        buf.resize((size_t)nb);
        f.seek(data0 + ti.offset);
        f.read(buf.data(), (size_t)nb);
        m->set_tensor(ti.name, ti.gtype, ti.n_dims, ti.ne, buf.data(), (size_t)nb);
    }
    m->finalize();
    return m;
}

}  // namespace pkx

namespace pkx {

bool is_quantizable_name(const std::string& n) {
    // examples/cli/main.cpp:279-303
    if (n == "encoder.pre_encode.out.weight" || n == "joint.enc.weight" || n == "joint.pred.weight") return true;
    const std::string prefix = "encoder.layers.";
    if (n.compare(0, prefix.size(), prefix) != 0) return false;
    size_t i = prefix.size();
    const size_t start = i;
    while (i < n.size() && n[i] >= '0' && n[i] <= '9') ++i;
    if (i == start || i >= n.size() || n[i] != '.') return false;
    const std::string rest = n.substr(i + 1);
    for (const char* r : {"feed_forward1.linear1.weight", "feed_forward1.linear2.weight",
                          "feed_forward2.linear1.weight", "feed_forward2.linear2.weight",
                          "self_attn.linear_q.weight", "self_attn.linear_k.weight", "self_attn.linear_v.weight",
                          "self_attn.linear_out.weight", "self_attn.linear_pos.weight"})
        if (rest == r) return true;
    return false;
}

namespace {
struct Out {
    FILE* f = nullptr;
    std::string path;
    explicit Out(const std::string& p) : f(std::fopen(p.c_str(), "wb")), path(p) {
        require(f != nullptr, "cannot create " + p);
    }
    ~Out() { if (f) std::fclose(f); }
    void write(const void* p, size_t n) { require(std::fwrite(p, 1, n, f) == n, "write failed: " + path); }
    template <typename T> void put(T v) { write(&v, sizeof v); }
    void str(const std::string& s) { put<uint64_t>(s.size()); write(s.data(), s.size()); }
    void pad_to(uint64_t align) {
        const long pos = std::ftell(f);
        const uint64_t padn = ((uint64_t)pos + align - 1) / align * align - (uint64_t)pos;
        static const char zeros[256] = {};
        for (uint64_t k = 0; k < padn; k += 256) write(zeros, (size_t)std::min<uint64_t>(256, padn - k));
    }
};
}  // namespace

QuantizeCounts quantize_gguf(const std::string& in_path, const std::string& out_path, int gtype) {
    require(gtype == GT_Q8_0 || gtype == GT_Q4_K, "quantize: type must be q8_0 or q4_K");
    require(in_path != out_path, "quantize: output must differ from input");
    const int64_t block = gtype == GT_Q8_0 ? 32 : 256, bbytes = gtype == GT_Q8_0 ? 34 : 144;
    File f(in_path);
    Header h = read_header(f, in_path);
    struct Plan {
        TensorInfo out;
        bool quant = false;
        int64_t src_bytes = 0, dst_bytes = 0;
    };
    QuantizeCounts cnt;
    std::vector<Plan> plan(h.infos.size());
    uint64_t off = 0;
    for (size_t i = 0; i < h.infos.size(); ++i) {
        const TensorInfo& ti = h.infos[i];
        Plan& p = plan[i];
        p.out = ti;
        p.src_bytes = tensor_bytes(ti);
        require(p.src_bytes >= 0, "GGUF: unsupported type " + std::to_string(ti.gtype) + " for tensor " + ti.name);
        if (is_quantizable_name(ti.name) && ti.gtype == GT_F32) {
            const bool two_d = ti.ne[2] == 1 && ti.ne[3] == 1 && ti.ne[0] >= 32 && ti.ne[1] >= 32;
            if (two_d && ti.ne[0] % block == 0) p.quant = true;
            else if (two_d) ++cnt.skipped;
        }
        if (p.quant) {
            p.out.gtype = gtype;
            p.out.n_dims = 2;
            p.dst_bytes = ti.ne[0] / block * bbytes * ti.ne[1];
            ++cnt.quantized;
        } else {
            p.dst_bytes = p.src_bytes;
            ++cnt.kept;
        }
        p.out.offset = off;
        off = (off + (uint64_t)p.dst_bytes + h.align - 1) / h.align * h.align;
    }
    Out o(out_path);
    o.put<uint32_t>(0x46554747u);
    o.put<uint32_t>(3);
    o.put<uint64_t>(h.infos.size());
    o.put<uint64_t>(h.n_kv);
    {   // every KV pair verbatim
        std::vector<uint8_t> kvb((size_t)(h.kv_end - h.kv_begin));
        f.seek(h.kv_begin);
        if (!kvb.empty()) f.read(kvb.data(), kvb.size());
        if (!kvb.empty()) o.write(kvb.data(), kvb.size());
    }
    for (const Plan& p : plan) {
        o.str(p.out.name);
        o.put<uint32_t>((uint32_t)p.out.n_dims);
        for (int d = 0; d < p.out.n_dims; ++d) o.put<uint64_t>((uint64_t)p.out.ne[d]);
        o.put<uint32_t>((uint32_t)p.out.gtype);
        o.put<uint64_t>(p.out.offset);
    }
    o.pad_to(h.align);
    const long data_start = std::ftell(o.f);
    hipStream_t s = nullptr;
    PKX_HIP(hipStreamCreate(&s));
    void *dsrc = nullptr, *ddst = nullptr;
    size_t cap_src = 0, cap_dst = 0;
    std::vector<uint8_t> buf, qbuf;
    try {
        for (size_t i = 0; i < plan.size(); ++i) {
            const Plan& p = plan[i];
            const uint64_t pos = (uint64_t)(std::ftell(o.f) - data_start);
            require(pos <= p.out.offset, "quantize: layout error");
            static const char zeros[256] = {};
            for (uint64_t k = pos; k < p.out.offset; k += 256)
                o.write(zeros, (size_t)std::min<uint64_t>(256, p.out.offset - k));
            buf.resize((size_t)p.src_bytes);
            f.seek(h.data0 + h.infos[i].offset);
            if (!buf.empty()) f.read(buf.data(), buf.size());
            if (!p.quant) {
                if (!buf.empty()) o.write(buf.data(), buf.size());
                continue;
            }
            if ((size_t)p.src_bytes > cap_src) {
                if (dsrc) PKX_HIP(hipFree(dsrc));
                dsrc = nullptr;
                PKX_HIP(hipMalloc(&dsrc, (size_t)p.src_bytes));
                cap_src = (size_t)p.src_bytes;
            }
            if ((size_t)p.dst_bytes > cap_dst) {
                if (ddst) PKX_HIP(hipFree(ddst));
                ddst = nullptr;
                PKX_HIP(hipMalloc(&ddst, (size_t)p.dst_bytes));
                cap_dst = (size_t)p.dst_bytes;
            }
            PKX_HIP(hipMemcpyAsync(dsrc, buf.data(), (size_t)p.src_bytes, hipMemcpyHostToDevice, s));
            quantize_rows(gtype, (const float*)dsrc, ddst, h.infos[i].ne[1], h.infos[i].ne[0], s);
            qbuf.resize((size_t)p.dst_bytes);
            PKX_HIP(hipMemcpyAsync(qbuf.data(), ddst, (size_t)p.dst_bytes, hipMemcpyDeviceToHost, s));
            PKX_HIP(hipStreamSynchronize(s));
            o.write(qbuf.data(), qbuf.size());
        }
    } catch (...) {
        if (dsrc) (void)hipFree(dsrc);
        if (ddst) (void)hipFree(ddst);
        (void)hipStreamDestroy(s);
        throw;
    }
    if (dsrc) PKX_HIP(hipFree(dsrc));
    if (ddst) PKX_HIP(hipFree(ddst));
    PKX_HIP(hipStreamDestroy(s));
    return cnt;
}

}  // namespace pkx

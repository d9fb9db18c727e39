// Device model: upload + repack, workspace, and the encoder forward schedule.
#include "model.hpp"

#include <cmath>
#include <cstring>

namespace pkx {

// ---------------------------------------------------------------------------
// host binary16 helpers (IEEE 754, round to nearest even)
// ---------------------------------------------------------------------------
static float half_bits_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t bits;
    float f;
    if (ex == 0) {
        f = std::ldexp((float)man, -24);
        std::memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    std::memcpy(&f, &bits, 4);
    return f;
}

static uint16_t float_to_half_bits(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        float af;
        std::memcpy(&af, &ax, 4);
        return (uint16_t)(sign | (uint16_t)std::nearbyint(af * 16777216.0f));
    }
    const uint32_t e = (ax >> 23) - 112u, m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

static int64_t row_bytes(int gtype, int64_t K) {
    switch (gtype) {
    case GT_F32: return K * 4;
    case GT_F16: return K * 2;
    case GT_Q8_0: return K / 32 * 34;
    case GT_Q4_K: return K / 256 * 144;
    default: throw std::invalid_argument("unsupported ggml type " + std::to_string(gtype));
    }
}

int subsampled_len(int T, bool causal) {
    int t = T;
    for (int s = 0; s < 3; ++s) t = sub_stage_len(t, causal);
    return t;
}

int valid_out_len(int T, int in_valid, bool causal) {
    int v = in_valid >= 0 ? in_valid : T - 1;
    for (int s = 0; s < 3; ++s) v = sub_stage_len(v, causal);
    return v;
}

// ---------------------------------------------------------------------------
// workspace
// ---------------------------------------------------------------------------
struct Buf {
    void* p = nullptr;
    size_t cap = 0;
};

// Split-K workspace: 2^20 floats of partial tiles (256 64 x 64 tile splits)
// and 512 tile counters, zero between launches
constexpr int64_t SK_FLOATS = (int64_t)1 << 20;
constexpr int SK_TILES = 512;

struct Model::Ws {
    Buf a2, a2p, a3, flat;              // subsampling maps
    Buf h, u, qkv, g, pe, p, xin, tmp;  // layer activations
    Buf lnst;                           // row statistics for the folded LayerNorms
    Buf lnrows;                         // norm_out's per-row {mean, rstd} (not stored norm_out output)
    Buf logits, pp;                     // heads
    Buf skpart;                         // split-K partial tiles
    int* skcnt = nullptr;               // split-K tile counters (zero between launches)
    int* d_valid = nullptr;             // 4 x Bcap ints: v0, v1, v2, vout
    int* h_valid = nullptr;             // pinned staging
    int Bcap = 0;
    hipEvent_t staged = nullptr;
    ~Ws() {
        for (Buf* b : {&a2, &a2p, &a3, &flat, &h, &u, &qkv, &g, &pe, &p, &xin, &tmp, &lnst, &lnrows, &logits, &pp, &skpart})
            if (b->p) (void)hipFree(b->p);
        if (d_valid) (void)hipFree(d_valid);
        if (skcnt) (void)hipFree(skcnt);
        if (h_valid) (void)hipHostFree(h_valid);
        if (staged) (void)hipEventDestroy(staged);
    }
};

static void grow(Buf& b, size_t bytes) {
    if (bytes <= b.cap) return;
    if (b.p) PKX_HIP(hipFree(b.p));
    b.p = nullptr;
    b.cap = 0;
    PKX_HIP(hipMalloc(&b.p, bytes));
    b.cap = bytes;
}

// ---------------------------------------------------------------------------
// construction / upload
// ---------------------------------------------------------------------------
Model::Model(const ModelConfig& cfg, int precision) : cfg_(cfg), ws_(new Ws) {
    require(cfg.d_model > 0 && cfg.n_layers > 0 && cfg.n_heads > 0 && cfg.ff_dim > 0, "config: bad encoder dims");
    require(cfg.d_model % cfg.n_heads == 0, "config: d_model % n_heads != 0");
    require(cfg.conv_kernel % 2 == 1, "config: depthwise kernel must be odd");
    require(cfg.n_mels > 0 && cfg.sub_channels > 0 && cfg.sub_channels % 8 == 0,
            "config: subsampling channels must be a positive multiple of 8");
    prec_ = precision == PREC_F32 ? PREC_F32 : PREC_F16;
    if (precision < 0) prec_ = (Precision)-1;  // resolved in finalize()
}

Model::~Model() {
    auto fr = [](void* p) { if (p) (void)hipFree(p); };
    for (void* p : allocs_) fr(p);
    ws_.reset();
    if (tl_launch_hook && tl_launch_hook == (LaunchHook*)prof_hook_.get()) tl_launch_hook = nullptr;
    for (auto& e : prof_ev_) {
        (void)hipEventDestroy(e.first);
        (void)hipEventDestroy(e.second);
    }
}

void Model::set_tensor(const std::string& name, int gtype, int n_dims, const int64_t* ne,
                       const void* data, size_t nbytes) {
    require(!finalized_, "set_tensor after finalize");
    require(n_dims >= 1 && n_dims <= 4, "set_tensor: n_dims must be 1..4");
    HostTensor t;
    t.gtype = gtype;
    t.n_dims = n_dims;
    for (int i = 0; i < n_dims; ++i) t.ne[i] = ne[i];
    const int64_t rows = t.nelem() / t.ne[0];
    const int64_t want = row_bytes(gtype, t.ne[0]) * rows;
    require((int64_t)nbytes == want, "set_tensor '" + name + "': expected " + std::to_string(want) +
                                         " bytes, got " + std::to_string(nbytes));
    t.bytes.assign((const uint8_t*)data, (const uint8_t*)data + nbytes);
    host_[name] = std::move(t);
}

const HostTensor* Model::find(const std::string& n) const {
    auto it = host_.find(n);
    return it == host_.end() ? nullptr : &it->second;
}

const HostTensor& Model::need(const std::string& n) const {
    const HostTensor* t = find(n);
    require(t != nullptr, "missing tensor '" + n + "'");
    return *t;
}

void* Model::dalloc(size_t bytes) {
    void* p = nullptr;
    PKX_HIP(hipMalloc(&p, bytes ? bytes : 16));
    allocs_.push_back(p);
    return p;
}

static std::vector<float> to_f32(const HostTensor& t) {
    const int64_t n = t.nelem();
    std::vector<float> v((size_t)n);
    if (t.gtype == GT_F32) {
        std::memcpy(v.data(), t.bytes.data(), (size_t)n * 4);
    } else if (t.gtype == GT_F16) {
        const uint16_t* h = (const uint16_t*)t.bytes.data();
        for (int64_t i = 0; i < n; ++i) v[(size_t)i] = half_bits_to_float(h[i]);
    } else if (t.gtype == GT_Q8_0) {
        // ggml block_q8_0 {f16 d; i8 q[32]}: w = d * q (exact in f32)
        require(n % 32 == 0 && (int64_t)t.bytes.size() == n / 32 * 34, "q8_0 tensor size");
        for (int64_t b = 0; b < n / 32; ++b) {
            const uint8_t* blk = t.bytes.data() + b * 34;
            const float d = half_bits_to_float((uint16_t)(blk[0] | (blk[1] << 8)));
            for (int j = 0; j < 32; ++j) v[(size_t)(b * 32 + j)] = d * (float)(int8_t)blk[2 + j];
        }
    } else if (t.gtype == GT_Q4_K) {
        // ggml block_q4_K {f16 d, dmin; u8 scales[12]; u8 qs[128]}: w = d*sc*q - dmin*m
        require(n % 256 == 0 && (int64_t)t.bytes.size() == n / 256 * 144, "q4_K tensor size");
        for (int64_t b = 0; b < n / 256; ++b) {
            const uint8_t* blk = t.bytes.data() + b * 144;
            const float d = half_bits_to_float((uint16_t)(blk[0] | (blk[1] << 8)));
            const float dmin = half_bits_to_float((uint16_t)(blk[2] | (blk[3] << 8)));
            const uint8_t* sc = blk + 4;
            const uint8_t* qs = blk + 16;
            for (int j = 0; j < 8; ++j) {
                int s6, m6;
                if (j < 4) {
                    s6 = sc[j] & 63;
                    m6 = sc[j + 4] & 63;
                } else {
                    s6 = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
                    m6 = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
                }
                const float dj = d * (float)s6, mj = dmin * (float)m6;
                for (int l = 0; l < 32; ++l) {
                    const uint8_t byte = qs[32 * (j / 2) + l];
                    const int q = (j & 1) ? (byte >> 4) : (byte & 0xF);
                    v[(size_t)(b * 256 + 32 * j + l)] = dj * (float)q - mj;
                }
            }
        }
    } else {
        throw std::invalid_argument("expected an f32/f16/q8_0/q4_K tensor");
    }
    return v;
}

float* Model::upload_f32(const std::vector<float>& v) {
    float* d = (float*)dalloc(v.size() * 4);
    PKX_HIP(hipMemcpy(d, v.data(), v.size() * 4, hipMemcpyHostToDevice));
    return d;
}

float* Model::upload_f32(const HostTensor& t) { return upload_f32(to_f32(t)); }

static void* dalloc_into(std::vector<void*>& allocs, size_t bytes) {
    void* p = nullptr;
    PKX_HIP(hipMalloc(&p, bytes ? bytes : 16));
    allocs.push_back(p);
    return p;
}

DevWeight Model::make_weight(const HostTensor& t, int N, int K, bool f16_gemm) {
    return build_weight(t, N, K, f16_gemm, allocs_);
}

// Raw rows (GGUF layout) -> device layout for the GEMM family.
DevWeight build_weight(const HostTensor& t, int N, int K, bool f16_gemm, std::vector<void*>& allocs) {
    require(t.nelem() == (int64_t)N * K, "weight shape mismatch");
    auto dalloc = [&](size_t bytes) { return dalloc_into(allocs, bytes); };
    DevWeight w;
    w.N = N;
    w.K = K;
    const uint8_t* src = t.bytes.data();
    switch (t.gtype) {
    case GT_F32:
        if (f16_gemm) {
            std::vector<uint16_t> h((size_t)N * K);
            const float* f = (const float*)src;
            for (size_t i = 0; i < h.size(); ++i) h[i] = float_to_half_bits(f[i]);
            w.gtype = GT_F16;
            w.q = dalloc(h.size() * 2);
            PKX_HIP(hipMemcpy(w.q, h.data(), h.size() * 2, hipMemcpyHostToDevice));
        } else {
            w.gtype = GT_F32;
            w.q = dalloc((size_t)N * K * 4);
            PKX_HIP(hipMemcpy(w.q, src, (size_t)N * K * 4, hipMemcpyHostToDevice));
        }
        break;
    case GT_F16:
        w.gtype = GT_F16;
        w.q = dalloc((size_t)N * K * 2);
        PKX_HIP(hipMemcpy(w.q, src, (size_t)N * K * 2, hipMemcpyHostToDevice));
        break;
    case GT_Q8_0: {
        // slab-major: block b of row n lands in slab b / 2 at (slab * N + n) * 64 + 32 (b % 2)
        require(K % 64 == 0, "q8_0 weight: K must be a multiple of 64");
        const int nb = K / 32;
        std::vector<int8_t> q((size_t)N * K);
        std::vector<uint16_t> d((size_t)N * nb);
        for (int n = 0; n < N; ++n)
            for (int b = 0; b < nb; ++b) {
                const uint8_t* blk = src + ((size_t)n * nb + b) * 34;
                const size_t slab = (size_t)(b / 2) * N + n;
                d[slab * 2 + b % 2] = (uint16_t)(blk[0] | (blk[1] << 8));
                std::memcpy(&q[slab * 64 + (size_t)(b % 2) * 32], blk + 2, 32);
            }
        w.gtype = GT_Q8_0;
        w.ldn = N;
        w.q = dalloc(q.size());
        w.s = dalloc(d.size() * 2);
        PKX_HIP(hipMemcpy(w.q, q.data(), q.size(), hipMemcpyHostToDevice));
        PKX_HIP(hipMemcpy(w.s, d.data(), d.size() * 2, hipMemcpyHostToDevice));
        break;
    }
    case GT_Q4_K: {
        require(K % 256 == 0, "q4_K weight K % 256 != 0");
        const int nb = K / 256;
        std::vector<uint8_t> qs((size_t)N * K / 2);
        std::vector<float> sc((size_t)N * (K / 32) * 2);
        for (int n = 0; n < N; ++n)
            for (int b = 0; b < nb; ++b) {
                const uint8_t* blk = src + ((size_t)n * nb + b) * 144;
                const float d = half_bits_to_float((uint16_t)(blk[0] | (blk[1] << 8)));
                const float dmin = half_bits_to_float((uint16_t)(blk[2] | (blk[3] << 8)));
                const uint8_t* s6 = blk + 4;
                for (int j = 0; j < 8; ++j) {
                    int s, m;
                    if (j < 4) {
                        s = s6[j] & 63;
                        m = s6[j + 4] & 63;
                    } else {
                        s = (s6[j + 4] & 0xF) | ((s6[j - 4] >> 6) << 4);
                        m = (s6[j + 4] >> 4) | ((s6[j] >> 6) << 4);
                    }
                    // slab-major: sub-block 8b + j is half (j % 2) of slab 4b + j / 2
                    float* o = &sc[(((size_t)(4 * b + j / 2) * N + n) * 2 + (j % 2)) * 2];
                    o[0] = d * (float)s;
                    o[1] = dmin * (float)m;
                }
                // 32 nibble bytes per 64 elements: slab 4b + c holds bytes [32c, 32c + 32) of the block
                for (int c = 0; c < 4; ++c)
                    std::memcpy(&qs[((size_t)(4 * b + c) * N + n) * 32], blk + 16 + 32 * c, 32);
            }
        w.gtype = GT_Q4_K;
        w.ldn = N;
        w.q = dalloc(qs.size());
        w.s = dalloc(sc.size() * 4);
        PKX_HIP(hipMemcpy(w.q, qs.data(), qs.size(), hipMemcpyHostToDevice));
        PKX_HIP(hipMemcpy(w.s, sc.data(), sc.size() * 4, hipMemcpyHostToDevice));
        break;
    }
    default:
        throw std::invalid_argument("unsupported weight type " + std::to_string(t.gtype));
    }
    return w;
}

// Concatenate the rows of several same-typed weights (q|k|v), or interleave the
// two halves of one weight in 16-row groups (pointwise_conv1 for the GLU epilogue).
DevWeight Model::make_weight_rows(const std::vector<const HostTensor*>& parts, int K,
                                  bool f16_gemm, bool glu_interleave) {
    const int gt = parts[0]->gtype;
    const int64_t rb = row_bytes(gt, K);
    int N = 0;
    for (const HostTensor* p : parts) {
        require(p->gtype == gt, "concatenated weights must share a type");
        require(p->nelem() % K == 0, "concatenated weight K mismatch");
        N += (int)(p->nelem() / K);
    }
    HostTensor cat;
    cat.gtype = gt;
    cat.n_dims = 2;
    cat.ne[0] = K;
    cat.ne[1] = N;
    cat.bytes.resize((size_t)rb * N);
    if (glu_interleave) {
        require(parts.size() == 1 && N % 64 == 0, "GLU interleave needs one weight with 2D rows, D % 32 == 0");
        const int D = N / 2;
        for (int r = 0; r < N; ++r) {
            const int g = r / 64, i = r % 64;
            const int src = i < 32 ? 32 * g + i : D + 32 * g + (i - 32);
            std::memcpy(&cat.bytes[(size_t)r * rb], &parts[0]->bytes[(size_t)src * rb], (size_t)rb);
        }
    } else {
        size_t off = 0;
        for (const HostTensor* p : parts) {
            std::memcpy(&cat.bytes[off], p->bytes.data(), p->bytes.size());
            off += p->bytes.size();
        }
    }
    return make_weight(cat, N, K, f16_gemm);
}

// Rows [row0, row0 + nrows) of a device weight, as a weight of its own (no copy):
// row-major layouts by offset, the slab-major q8_0 layout by offset inside each
// slab block (ldn stays the allocation's row count).
DevWeight weight_rows_view(const DevWeight& w, int row0, int nrows) {
    DevWeight v = w;
    v.N = nrows;
    const int64_t r = row0, K = w.K;
    switch (w.gtype) {
    case GT_F32: v.q = (uint8_t*)w.q + r * K * 4; break;
    case GT_F16: v.q = (uint8_t*)w.q + r * K * 2; break;
    case GT_Q8_0:   // slab-major: the rows' offset inside every slab block
        v.q = (uint8_t*)w.q + r * 64;
        v.s = (uint8_t*)w.s + r * 4;
        break;
    case GT_Q4_K:   // slab-major as q8_0
        v.q = (uint8_t*)w.q + r * 32;
        v.s = (uint8_t*)w.s + r * 16;
        break;
    default: throw std::logic_error("weight view: unknown type");
    }
    return v;
}

void linear_raw(Precision prec, const HostTensor& t, int N, int K, const float* bias, const float* x,
                int64_t M, float* y, hipStream_t s, bool residual, float alpha) {
    std::vector<void*> allocs;
    try {
        const DevWeight w = build_weight(t, N, K, prec == PREC_F16, allocs);
        const void* A = x;
        if (prec == PREC_F16) {
            void* xa = dalloc_into(allocs, (size_t)M * K * 2);
            launch_cast_f32(prec, x, xa, M * K, s);
            A = xa;
        }
        GemmParams p;
        p.A = A;
        p.lda = K;
        p.Wq = w.q;
        p.Ws = w.s;
        p.ldw = w.ldn;
        p.bias = bias;
        p.Y = y;
        p.ldy = N;
        p.M = (int)M;
        p.N = N;
        p.K = K;
        p.alpha = residual ? alpha : 1.0f;
        if (residual && prec == PREC_F16) {
            // the split-K workspace the encoder's residual products use
            p.sk_part = (float*)dalloc_into(allocs, (size_t)SK_FLOATS * 4);
            p.sk_part_floats = SK_FLOATS;
            p.sk_cnt = (int*)dalloc_into(allocs, SK_TILES * sizeof(int));
            p.sk_cnt_n = SK_TILES;
            PKX_HIP(hipMemsetAsync(p.sk_cnt, 0, SK_TILES * sizeof(int), s));
        }
        launch_gemm(prec, w.gtype, residual ? EPI_RESID : EPI_STORE_F32, p, s);
        PKX_HIP(hipStreamSynchronize(s));
    } catch (...) {
        (void)hipStreamSynchronize(s);
        for (void* a : allocs) (void)hipFree(a);
        throw;
    }
    for (void* a : allocs) PKX_HIP(hipFree(a));
}

static bool quantizable_linear(const std::string& n) {
    return n.find("feed_forward") != std::string::npos || n.find("self_attn.linear_") != std::string::npos ||
           n == "encoder.pre_encode.out.weight";
}

void Model::finalize() {
    require(!finalized_, "finalize called twice");
    const ModelConfig& c = cfg_;
    const int D = c.d_model, FF = c.ff_dim, H = c.n_heads, dk = D / H, K = c.conv_kernel, C = c.sub_channels;
    require(D % 32 == 0, "d_model must be a multiple of 32");

    if ((int)prec_ < 0) {
        bool any_low = false;
        for (auto& kv : host_)
            if (quantizable_linear(kv.first) && kv.second.gtype != GT_F32) any_low = true;
        prec_ = any_low ? PREC_F16 : PREC_F32;
    }
    const bool f16g = prec_ == PREC_F16;

    auto optb = [&](const std::string& n) -> float* {
        const HostTensor* t = find(n);
        return t ? upload_f32(*t) : nullptr;
    };

    layers_.resize(c.n_layers);
    for (int i = 0; i < c.n_layers; ++i) {
        const std::string p = "encoder.layers." + std::to_string(i) + ".";
        LayerDev& L = layers_[i];
        L.ff1_ln_g = upload_f32(need(p + "norm_feed_forward1.weight"));
        L.ff1_ln_b = upload_f32(need(p + "norm_feed_forward1.bias"));
        L.att_ln_g = upload_f32(need(p + "norm_self_att.weight"));
        L.att_ln_b = upload_f32(need(p + "norm_self_att.bias"));
        L.conv_ln_g = upload_f32(need(p + "norm_conv.weight"));
        L.conv_ln_b = upload_f32(need(p + "norm_conv.bias"));
        L.ff2_ln_g = upload_f32(need(p + "norm_feed_forward2.weight"));
        L.ff2_ln_b = upload_f32(need(p + "norm_feed_forward2.bias"));
        L.out_ln_g = upload_f32(need(p + "norm_out.weight"));
        L.out_ln_b = upload_f32(need(p + "norm_out.bias"));
        L.ff1_w1 = make_weight(need(p + "feed_forward1.linear1.weight"), FF, D, f16g);
        L.ff1_w2 = make_weight(need(p + "feed_forward1.linear2.weight"), D, FF, f16g);
        L.ff2_w1 = make_weight(need(p + "feed_forward2.linear1.weight"), FF, D, f16g);
        L.ff2_w2 = make_weight(need(p + "feed_forward2.linear2.weight"), D, FF, f16g);
        L.ff1_b1 = optb(p + "feed_forward1.linear1.bias");
        L.ff1_b2 = optb(p + "feed_forward1.linear2.bias");
        L.ff2_b1 = optb(p + "feed_forward2.linear1.bias");
        L.ff2_b2 = optb(p + "feed_forward2.linear2.bias");
        const std::string a = p + "self_attn.";
        L.wqkv = make_weight_rows({&need(a + "linear_q.weight"), &need(a + "linear_k.weight"),
                                   &need(a + "linear_v.weight")}, D, f16g, false);
        {
            const HostTensor *bq = find(a + "linear_q.bias"), *bk = find(a + "linear_k.bias"),
                             *bv = find(a + "linear_v.bias");
            if (bq || bk || bv) {
                std::vector<float> cat((size_t)3 * D, 0.0f);
                const HostTensor* bb[3] = {bq, bk, bv};
                for (int j = 0; j < 3; ++j)
                    if (bb[j]) {
                        std::vector<float> v = to_f32(*bb[j]);
                        std::memcpy(&cat[(size_t)j * D], v.data(), (size_t)D * 4);
                    }
                L.bqkv = upload_f32(cat);
            }
        }
        L.wo = make_weight(need(a + "linear_out.weight"), D, D, f16g);
        L.bo = optb(a + "linear_out.bias");
        // linear_pos: a row view into the all-layer concatenation built below
        require(need(a + "linear_pos.weight").nelem() == (int64_t)D * D, "linear_pos shape");
        L.pos_u = upload_f32(need(a + "pos_bias_u"));
        L.pos_v = upload_f32(need(a + "pos_bias_v"));
        require(need(a + "pos_bias_u").nelem() == (int64_t)H * dk, "pos_bias_u shape");

        const std::string cv = p + "conv.";
        L.pw1 = make_weight_rows({&need(cv + "pointwise_conv1.weight")}, D, f16g, true);
        if (const HostTensor* b1 = find(cv + "pointwise_conv1.bias")) {
            std::vector<float> v = to_f32(*b1), il(v.size());
            for (int r = 0; r < 2 * D; ++r) {
                const int g = r / 64, j = r % 64;
                il[(size_t)r] = v[(size_t)(j < 32 ? 32 * g + j : D + 32 * g + (j - 32))];
            }
            L.pw1_b = upload_f32(il);
        }
        L.pw2 = make_weight(need(cv + "pointwise_conv2.weight"), D, D, f16g);
        L.pw2_b = optb(cv + "pointwise_conv2.bias");
        {
            const HostTensor& dw = need(cv + "depthwise_conv.weight");
            require(dw.nelem() == (int64_t)D * K, "depthwise_conv.weight shape");
            L.dw_w = upload_f32(dw);
        }
        L.dw_b = optb(cv + "depthwise_conv.bias");
        if (c.conv_ln) {
            // conv_norm_type "layer_norm": LayerNorm over channels with the
            // batch_norm.weight / .bias tensors as gamma / beta (conformer.cpp:128-133)
            L.cn_g = upload_f32(need(cv + "batch_norm.weight"));
            L.cn_b = upload_f32(need(cv + "batch_norm.bias"));
        } else {
            // BatchNorm fold, exactly conformer.cpp:144-147 (f32).
            std::vector<float> g = to_f32(need(cv + "batch_norm.weight")),
                               bb = to_f32(need(cv + "batch_norm.bias")),
                               m = to_f32(need(cv + "batch_norm.running_mean")),
                               var = to_f32(need(cv + "batch_norm.running_var"));
            std::vector<float> sc((size_t)D), sh((size_t)D);
            for (int ch = 0; ch < D; ++ch) {
                sc[(size_t)ch] = g[(size_t)ch] / std::sqrt(var[(size_t)ch] + 1e-5f);
                sh[(size_t)ch] = bb[(size_t)ch] - m[(size_t)ch] * sc[(size_t)ch];
            }
            L.bn_scale = upload_f32(sc);
            L.bn_shift = upload_f32(sh);
        }
    }

    // linear_pos of every layer as one [L*D][D] weight: the positional table is
    // the same for all layers, so a forward projects it once for all of them
    // (one GEMM of N = L*D instead of L GEMMs over 2T'-1 rows).
    {
        std::vector<const HostTensor*> parts;
        bool same = true;
        for (int i = 0; i < c.n_layers; ++i) {
            parts.push_back(&need("encoder.layers." + std::to_string(i) + ".self_attn.linear_pos.weight"));
            same = same && parts.back()->gtype == parts[0]->gtype;
        }
        if (same) {
            wpos_all_ = make_weight_rows(parts, D, f16g, false);
            for (int i = 0; i < c.n_layers; ++i) layers_[i].wpos = weight_rows_view(wpos_all_, i * D, D);
        } else {
            for (int i = 0; i < c.n_layers; ++i) layers_[i].wpos = make_weight(*parts[i], D, D, f16g);
        }
    }

    // subsampling
    {
        const std::string p = "encoder.pre_encode.";
        int F = c.n_mels;
        for (int s = 0; s < 3; ++s) F = sub_stage_len(F, c.causal_sub != 0);
        sub_.w0 = upload_f32(need(p + "conv.0.weight"));
        sub_.b0 = upload_f32(need(p + "conv.0.bias"));
        sub_.w2 = upload_f32(need(p + "conv.2.weight"));
        sub_.b2 = upload_f32(need(p + "conv.2.bias"));
        sub_.w5 = upload_f32(need(p + "conv.5.weight"));
        sub_.b5 = upload_f32(need(p + "conv.5.bias"));
        require(need(p + "conv.0.weight").nelem() == (int64_t)C * 9, "conv.0.weight shape");
        sub_.w3 = make_weight(need(p + "conv.3.weight"), C, C, f16g);
        sub_.b3 = upload_f32(need(p + "conv.3.bias"));
        sub_.w6 = make_weight(need(p + "conv.6.weight"), C, C, f16g);
        sub_.b6 = upload_f32(need(p + "conv.6.bias"));
        sub_.out = make_weight(need(p + "out.weight"), D, C * F, f16g);
        sub_.bout = upload_f32(need(p + "out.bias"));
        if (sub_tail_fused()) {
            sub_.tail_w = dalloc(sub_tail_frag_bytes());
            sub_tail_prepare(sub_.w3.q, sub_.w6.q, sub_.tail_w, nullptr);
            PKX_HIP(hipDeviceSynchronize());
        }
    }

    // optional heads (always on the f32 GEMM path: argmax outputs)
    {
        const HostTensor* cw = find("ctc_decoder.decoder_layers.0.weight");
        std::string cb = "ctc_decoder.decoder_layers.0.bias";
        if (!cw) {
            cw = find("decoder.decoder_layers.0.weight");
            cb = "decoder.decoder_layers.0.bias";
        }
        if (cw) {
            const int V = (int)(cw->nelem() / D);
            heads_.ctc = make_weight(*cw, V, D, false);
            heads_.ctc_b = upload_f32(need(cb));
        }
        const HostTensor* je = find("joint.enc.weight");
        const HostTensor* jp = find("joint.pred.weight");
        const HostTensor* jo = find("joint.joint_net.2.weight");
        if (je && jp && jo) {
            const int Hj = (int)(je->nelem() / D);
            const int P = (int)(jp->nelem() / Hj);
            const int V = (int)(jo->nelem() / Hj);
            heads_.jenc = make_weight(*je, Hj, D, false);
            heads_.jpred = make_weight(*jp, Hj, P, false);
            heads_.jout = make_weight(*jo, V, Hj, false);
            heads_.jenc_b = upload_f32(need("joint.enc.bias"));
            heads_.jpred_b = upload_f32(need("joint.pred.bias"));
            heads_.jout_b = upload_f32(need("joint.joint_net.2.bias"));
            heads_.n_dur = c.n_durations;
            heads_.n_tok = V - c.n_durations;
            require(heads_.n_tok > 0, "joint: vocab/durations mismatch");
            // prediction network (prediction.cpp): layers counted from the tensors
            const HostTensor* emb = find("decoder.prediction.embed.weight");
            if (emb) {
                const std::string pre = "decoder.prediction.dec_rnn.lstm.";
                int L = 0;
                while (L < 4 && find(pre + "weight_ih_l" + std::to_string(L))) ++L;
                require(L >= 1, "prediction net: no LSTM layers");
                require(!find(pre + "weight_ih_l4"), "prediction net: at most 4 LSTM layers");
                pred_.H = P;
                pred_.V1 = (int)(emb->nelem() / P);
                require(pred_.V1 * (int64_t)P == emb->nelem(), "prediction net: embedding width != pred_hidden");
                pred_.embed = upload_f32(*emb);
                for (int l = 0; l < L; ++l) {
                    const std::string s = std::to_string(l);
                    const std::vector<float> wih = to_f32(need(pre + "weight_ih_l" + s));
                    const std::vector<float> whh = to_f32(need(pre + "weight_hh_l" + s));
                    const std::vector<float> bih = to_f32(need(pre + "bias_ih_l" + s));
                    const std::vector<float> bhh = to_f32(need(pre + "bias_hh_l" + s));
                    require(wih.size() == (size_t)4 * P * P && whh.size() == wih.size() && bih.size() == (size_t)4 * P &&
                                bhh.size() == bih.size(),
                            "prediction net: layer " + s + " must be [4H][H] with [4H] biases");
                    std::vector<float> cat((size_t)4 * P * 2 * P);
                    for (int r = 0; r < 4 * P; ++r) {
                        std::memcpy(cat.data() + (size_t)r * 2 * P, wih.data() + (size_t)r * P, sizeof(float) * P);
                        std::memcpy(cat.data() + (size_t)r * 2 * P + P, whh.data() + (size_t)r * P,
                                    sizeof(float) * P);
                    }
                    pred_.wcat[l] = upload_f32(cat);
                    std::vector<float> bs((size_t)4 * P);
                    for (size_t i = 0; i < bs.size(); ++i) bs[i] = bih[i] + bhh[i];
                    pred_.bsum[l] = upload_f32(bs);
                }
                pred_.L = L;
                pred_.jpred = upload_f32(*jp);   // f32 copies (dequantised) for the decode matvecs
                pred_.jout = upload_f32(*jo);
            }
        }
    }
    // LayerNorm folding (f16 path): every product involved must take the LDS-DMA
    // kernel, i.e. f16 / q8_0 / q4_K weights with K % 64 == 0
    {
        auto dma = [](const DevWeight& w) {
            return (w.gtype == GT_F16 || w.gtype == GT_Q8_0 || w.gtype == GT_Q4_K) && w.K % 64 == 0;
        };
        const int G = D / 32;   // row-statistics groups: a power of two up to 32
        bool ok = f16g && D % 64 == 0 && FF % 8 == 0 && G <= 32 && (G & (G - 1)) == 0;
        for (const LayerDev& L : layers_)
            ok = ok && dma(L.ff1_w2) && dma(L.wo) && dma(L.pw2) && dma(L.wqkv) && dma(L.pw1) && dma(L.ff2_w1);
        ln_fold_ = ok;
        if (ok) {
            for (LayerDev& L : layers_) {
                auto consts = [&](const DevWeight& w, const float* g, const float* b, const float* bias, float*& c1,
                                  float*& c2) {
                    c1 = (float*)dalloc((size_t)w.N * 4);
                    c2 = (float*)dalloc((size_t)w.N * 4);
                    launch_ln_fold_consts(w.gtype, w.q, w.s, w.N, w.K, g, b, bias, c1, c2, nullptr);
                };
                consts(L.wqkv, L.att_ln_g, L.att_ln_b, L.bqkv, L.qkv_c1, L.qkv_c2);
                consts(L.pw1, L.conv_ln_g, L.conv_ln_b, L.pw1_b, L.pw1_c1, L.pw1_c2);
                consts(L.ff2_w1, L.ff2_ln_g, L.ff2_ln_b, L.ff2_b1, L.ff2_c1, L.ff2_c2);
            }
            PKX_HIP(hipDeviceSynchronize());
        }
    }
    // f16 pointwise_conv1 weights in the conv-module kernel's fragment order:
    // items of T <= 128 frames run one tile per item, reading this copy
    if (f16g && cfg_.conv_kernel == GLU_DW_K && !cfg_.conv_ln && !cfg_.conv_causal) {
        for (LayerDev& L : layers_)
            if (glu_frag_supported(L.pw1.gtype, L.pw1.N, L.pw1.K)) {
                L.pw1_frag = dalloc(glu_frag_bytes(L.pw1.N, L.pw1.K));
                glu_frag_prepare(L.pw1.q, L.pw1.N, L.pw1.K, L.pw1_frag, nullptr);
            }
        PKX_HIP(hipDeviceSynchronize());
    }
    host_.clear();
    // split-K workspace (residual products of few rows): created here, once, so
    // that no forward or streaming step allocates or synchronises for it
    grow(ws_->skpart, (size_t)SK_FLOATS * 4);
    PKX_HIP(hipMalloc(&ws_->skcnt, SK_TILES * sizeof(int)));
    PKX_HIP(hipMemset(ws_->skcnt, 0, SK_TILES * sizeof(int)));
    PKX_HIP(hipDeviceSynchronize());
    finalized_ = true;
}

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------
thread_local LaunchHook* tl_launch_hook = nullptr;

// Hands an event pair to every launch made inside a profiled family region.
struct Model::ProfHook final : LaunchHook {
    Model* m = nullptr;
    bool take(hipEvent_t* a, hipEvent_t* b) override {
        if (m->cur_fam_ < 0) return false;
        if (m->prof_seen_++ % m->prof_stride_ != 0) return false;
        if (m->prof_pending_.size() == m->prof_ev_.size()) {
            hipEvent_t e0 = nullptr, e1 = nullptr;
            // timing-only events: no system-scope fence (no cache writeback at the
            // kernel's end that would lengthen what is being measured)
            if (hipEventCreateWithFlags(&e0, hipEventDisableSystemFence) != hipSuccess) return false;
            if (hipEventCreateWithFlags(&e1, hipEventDisableSystemFence) != hipSuccess) {
                (void)hipEventDestroy(e0);
                return false;
            }
            m->prof_ev_.push_back({e0, e1});
        }
        const size_t i = m->prof_pending_.size();
        m->prof_pending_.push_back(m->cur_fam_);
        *a = m->prof_ev_[i].first;
        *b = m->prof_ev_[i].second;
        return true;
    }
};

void Model::set_profiling(unsigned mask, int stride) {
    require(stride >= 1, "profiling: stride must be >= 1");
    prof_mask_ = mask & ((1u << KF_COUNT) - 1);
    prof_stride_ = stride;
    prof_seen_ = 0;
    if (!prof_hook_) {
        prof_hook_ = std::make_unique<ProfHook>();
        prof_hook_->m = this;
    }
    prof_pending_.clear();
    cur_fam_ = -1;
    for (int i = 0; i < KF_COUNT; ++i) {
        prof_ms_[i] = 0;
        prof_n_[i] = 0;
    }
}

void Model::profile_read(double* ms, int64_t* n) {
    if (!prof_pending_.empty()) {
        PKX_HIP(hipEventSynchronize(prof_ev_[prof_pending_.size() - 1].second));
        for (size_t i = 0; i < prof_pending_.size(); ++i) {
            float t = 0.f;
            PKX_HIP(hipEventElapsedTime(&t, prof_ev_[i].first, prof_ev_[i].second));
            prof_ms_[prof_pending_[i]] += t;
            prof_n_[prof_pending_[i]] += 1;
        }
        prof_pending_.clear();
    }
    for (int i = 0; i < KF_COUNT; ++i) {
        if (ms) ms[i] = prof_ms_[i];
        if (n) n[i] = prof_n_[i];
    }
}

// Opens (begin) or closes a family region: while open, every kernel launched
// on this thread is timed into that family.  Regions do not nest; fam < 0 is
// a no-op so helpers called inside another family's region stay in it.
void Model::mark(int fam, bool begin) {
    if (fam < 0 || !(prof_mask_ >> fam & 1u)) return;
    if (begin) {
        cur_fam_ = fam;
        tl_launch_hook = prof_hook_.get();
    } else {
        cur_fam_ = -1;
        tl_launch_hook = nullptr;
    }
}

void Model::gemm(const DevWeight& w, int epi, const void* A, int64_t lda, int64_t M,
                 const float* bias, void* Y, int64_t ldy, float alpha, const int* valid, int T,
                 hipStream_t s, Precision prec, int fam, const float* bias2, int trF) {
    GemmParams p;
    p.A = A;
    p.lda = lda;
    p.Wq = w.q;
    p.Ws = w.s;
    p.ldw = w.ldn;
    p.bias = bias;
    p.bias2 = bias2;
    p.Y = Y;
    p.ldy = ldy;
    p.alpha = alpha;
    p.valid = valid;
    p.T = T;
    p.trF = trF;
    p.M = (int)M;
    p.N = w.N;
    p.K = w.K;
    if (epi == EPI_RESID) splitk_ws(p, s);
    mark(fam, true);
    launch_gemm(prec, w.gtype, epi, p, s);
    mark(fam, false);
}

void Model::splitk_ws(GemmParams& p, hipStream_t) {
    if (p.M > 512 || !ws_->skcnt) return;
    p.sk_part = (float*)ws_->skpart.p;
    p.sk_part_floats = SK_FLOATS;
    p.sk_cnt = ws_->skcnt;
    p.sk_cnt_n = SK_TILES;
}

void Model::gemm_resid_ln(const DevWeight& w, const void* A, int64_t M, const float* bias, float* x, float alpha,
                          const float* g, void* h, hipStream_t s, int fam, const float* res_rows,
                          const float* res_g, const float* res_b) {
    grow(ws_->lnst, (size_t)M * (w.N / 32) * 8);
    GemmParams p;
    p.res_rows = res_rows;
    p.res_g = res_g;
    p.res_b = res_b;
    p.A = A;
    p.lda = w.K;
    p.Wq = w.q;
    p.Ws = w.s;
    p.ldw = w.ldn;
    p.bias = bias;
    p.Y = x;
    p.ldy = w.N;
    p.alpha = alpha;
    p.M = (int)M;
    p.N = w.N;
    p.K = w.K;
    p.ln_g = g;
    p.ln_h = h;
    p.ln_stats = (float*)ws_->lnst.p;
    splitk_ws(p, s);
    mark(fam, true);
    launch_gemm(prec_, w.gtype, EPI_RESID_LN, p, s);
    mark(fam, false);
}

GemmParams Model::fold_params(const DevWeight& w, const void* A, int64_t M, const float* c1, const float* c2,
                              void* Y, int64_t ldy) {
    GemmParams p;
    p.A = A;
    p.lda = w.K;
    p.Wq = w.q;
    p.Ws = w.s;
    p.ldw = w.ldn;
    p.bias = c2;
    p.Y = Y;
    p.ldy = ldy;
    p.M = (int)M;
    p.N = w.N;
    p.K = w.K;
    p.fold_stats = (const float*)ws_->lnst.p;
    p.fold_c1 = c1;
    p.fold_groups = w.K / 32;
    return p;
}

void Model::conv_front(const LayerDev& L, const void* A, int64_t M, const int* valid, int B, int T, void* Y,
                       hipStream_t s, bool fold) {
    const ModelConfig& c = cfg_;
    const int D = c.d_model;
    // the one-pass epilogue is the symmetric-padding, BatchNorm conv module
    if (c.conv_kernel == GLU_DW_K && !c.conv_ln && !c.conv_causal &&
        gemm_glu_dw_supported(prec_, L.pw1.gtype, L.pw1.N, L.pw1.K)) {
        // one pass: the GEMM epilogue stages GLU rows in LDS and runs the
        // depthwise conv over time on them (conformer.cpp:48-157)
        GemmParams p;
        if (fold) p = fold_params(L.pw1, A, M, L.pw1_c1, L.pw1_c2, Y, D);
        p.A = A;
        p.lda = D;
        p.Wq = L.pw1.q;
        p.Ws = L.pw1.s;
        p.ldw = L.pw1.ldn;
        p.bias = fold ? L.pw1_c2 : L.pw1_b;
        p.Y = Y;
        p.ldy = D;
        p.valid = valid;
        p.T = T;
        p.M = (int)M;
        p.N = L.pw1.N;
        p.K = L.pw1.K;
        p.dw_w = L.dw_w;
        p.dw_b = L.dw_b;
        p.dw_scale = L.bn_scale;
        p.dw_shift = L.bn_shift;
        p.wfrag = L.pw1_frag;
        mark(KF_GEMM_PW1_GLU, true);
        launch_gemm(prec_, L.pw1.gtype, EPI_GLU_DW, p, s);
        mark(KF_GEMM_PW1_GLU, false);
        return;
    }
    // GLU output in the FFN hidden buffer (neither A nor Y in either caller)
    Ws& w = *ws_;
    Buf& glu = w.u;
    grow(glu, (size_t)M * D * (prec_ == PREC_F16 ? 2 : 4));
    require(glu.p != A && glu.p != Y, "conv module: input or output aliases the GLU scratch");
    if (fold) {
        GemmParams p = fold_params(L.pw1, A, M, L.pw1_c1, L.pw1_c2, glu.p, D);
        p.valid = valid;
        p.T = T;
        mark(KF_GEMM_PW1_GLU, true);
        launch_gemm(prec_, L.pw1.gtype, EPI_GLU, p, s);
        mark(KF_GEMM_PW1_GLU, false);
    } else {
        gemm(L.pw1, EPI_GLU, A, D, M, L.pw1_b, glu.p, D, 1.f, valid, T, s, prec_, KF_GEMM_PW1_GLU);
    }
    mark(KF_DWCONV, true);
    if (c.conv_ln) {
        // conv_norm_type "layer_norm": depthwise conv + bias in f32, then the
        // LayerNorm over channels + SiLU (conformer.cpp:126-133, :157)
        grow(w.tmp, (size_t)M * D * 4);
        launch_dwconv(prec_, glu.p, w.tmp.p, L.dw_w, L.dw_b, nullptr, nullptr, B, T, D, c.conv_kernel,
                      c.conv_causal != 0, s);
        LnParams lp;
        lp.x = (const float*)w.tmp.p;
        lp.g = L.cn_g;
        lp.b = L.cn_b;
        lp.y = Y;
        lp.M = M;
        lp.D = D;
        lp.silu = true;
        launch_layernorm(prec_, lp, s);
    } else {
        launch_dwconv(prec_, glu.p, Y, L.dw_w, L.dw_b, L.bn_scale, L.bn_shift, B, T, D, c.conv_kernel,
                      c.conv_causal != 0, s);
    }
    mark(KF_DWCONV, false);
}

void Model::ensure_ws(int B, int T_max) {
    const ModelConfig& c = cfg_;
    const size_t as = prec_ == PREC_F16 ? 2 : 4;
    const bool cz = c.causal_sub != 0;
    const int T1 = sub_stage_len(T_max, cz), T2 = sub_stage_len(T1, cz), T3 = sub_stage_len(T2, cz);
    const int F1 = sub_stage_len(c.n_mels, cz), F2 = sub_stage_len(F1, cz), F3 = sub_stage_len(F2, cz);
    const size_t C = c.sub_channels, D = c.d_model, M = (size_t)B * T3, P = 2 * (size_t)T3 - 1;
    Ws& w = *ws_;
    // (the conv0 map, B x T1 x F1 x C, is never materialised: see launch_sub_stage1)
    grow(w.a2, (size_t)B * T2 * F2 * C * as);
    if (!sub_tail_fused()) {   // the fused tail keeps both maps on chip
        grow(w.a2p, (size_t)B * T2 * F2 * C * as);
        grow(w.a3, (size_t)B * T3 * F3 * C * as);
    }
    grow(w.flat, (size_t)B * T3 * F3 * C * as);
    grow(w.h, M * D * as);
    grow(w.u, M * c.ff_dim * as);
    grow(w.qkv, M * 3 * D * as);
    grow(w.g, M * D * as);
    grow(w.pe, P * D * as);
    grow(w.p, P * D * c.n_layers * as);   // all layers' positional projections
    grow(w.tmp, M * D * 4);
    if (B > w.Bcap) {
            if (w.d_valid) PKX_HIP(hipFree(w.d_valid));
        if (w.h_valid) PKX_HIP(hipHostFree(w.h_valid));
        w.d_valid = nullptr;
        w.h_valid = nullptr;
        PKX_HIP(hipMalloc(&w.d_valid, sizeof(int) * 4 * (size_t)B));
        PKX_HIP(hipHostMalloc(&w.h_valid, sizeof(int) * 4 * (size_t)B, hipHostMallocDefault));
        w.Bcap = B;
    }
    if (!w.staged) PKX_HIP(hipEventCreateWithFlags(&w.staged, hipEventDisableTiming));
}

// Stage per-item lengths (slots v0, v1, v2, vout) through pinned memory in one copy.
void Model::stage_valid(const std::vector<int>* v[4], hipStream_t s) {
    Ws& w = *ws_;
    PKX_HIP(hipEventSynchronize(w.staged));   // the previous copy out of the staging buffer is done
    for (int k = 0; k < 4; ++k)
        std::memcpy(w.h_valid + (size_t)k * w.Bcap, v[k]->data(), v[k]->size() * sizeof(int));
    PKX_HIP(hipMemcpyAsync(w.d_valid, w.h_valid, sizeof(int) * 4 * (size_t)w.Bcap, hipMemcpyHostToDevice, s));
    PKX_HIP(hipEventRecord(w.staged, s));
}

// The chunked-limited window of a streaming model (relpos_attention.cpp:252-275):
// chunks of att_right + 1 frames, a query sees its own chunk and
// att_left / chunk_size chunks before it.
void Model::att_window(AttnParams& a) const {
    if (!cfg_.att_limited) return;
    a.chunk = cfg_.att_right + 1;
    a.left_chunks = cfg_.att_left / a.chunk;
}

void Model::ensure_pe(int T, hipStream_t s, const float* given) {
    mark(KF_POS_ENC, true);
    if (given) launch_cast_f32(prec_, given, ws_->pe.p, (int64_t)(2 * T - 1) * cfg_.d_model, s);
    else launch_rel_pos_encoding(prec_, ws_->pe.p, T, cfg_.d_model, s);
    mark(KF_POS_ENC, false);
}

void* Model::cast_to_act(const float* x, int64_t n, hipStream_t s) {
    grow(ws_->xin, (size_t)n * (prec_ == PREC_F16 ? 2 : 4));
    launch_cast_f32(prec_, x, ws_->xin.p, n, s);
    return ws_->xin.p;
}

// ---------------------------------------------------------------------------
// subsampling (subsampling.cpp:48-240 batched / :242-386 scalar masking)
// ---------------------------------------------------------------------------
int Model::subsampling_forward(const float* mel, int B, int T_max, const int* valid_T,
                               bool stage_masks, float* out, int* valid_out, hipStream_t s,
                               bool apply_xscaling, bool whole_frames) {
    const int T3 = stage_lengths(B, T_max, valid_T, valid_out, s, whole_frames);
    subsampling_kernels(mel, B, T_max, stage_masks, out, s, apply_xscaling);
    return T3;
}

// Per-item valid lengths of every subsampling stage (host arithmetic,
// subsampling.cpp:25-46) staged to the device; returns T'.
int Model::stage_lengths(int B, int T_max, const int* valid_T, int* valid_out, hipStream_t s, bool whole_frames) {
    require(finalized_, "model not finalized");
    require(B > 0 && T_max > 0, "subsampling: empty batch");
    ensure_ws(B, T_max);
    const bool cz = cfg_.causal_sub != 0;
    const int T1 = sub_stage_len(T_max, cz), T2 = sub_stage_len(T1, cz), T3 = sub_stage_len(T2, cz);
    std::vector<int> v0(B), v1(B), v2(B), vo(B);
    for (int b = 0; b < B; ++b) {
        const int vt = valid_T ? valid_T[b] : T_max;
        require(vt >= 1 && vt <= T_max, "valid_T out of range");
        // offline T-1 entry convention; a streaming window is audio to its last frame
        v0[b] = whole_frames ? vt : vt - 1;
        v1[b] = sub_stage_len(v0[b], cz);
        v2[b] = sub_stage_len(v1[b], cz);
        const int vv = valid_out_len(T_max, v0[b], cz);
        vo[b] = vv > T3 ? T3 : vv;
        if (valid_out) valid_out[b] = vo[b];
    }
    const std::vector<int>* slots[4] = {&v0, &v1, &v2, &vo};
    stage_valid(slots, s);
    return T3;
}

// The subsampling kernels on lengths staged by stage_lengths.
bool Model::sub_tail_fused() const {
    const ModelConfig& c = cfg_;
    const bool cz = c.causal_sub != 0;
    const int F2 = sub_stage_len(sub_stage_len(c.n_mels, cz), cz);
    return prec_ == PREC_F16 && sub_tail_supported(c.sub_channels, F2, cz) && sub_.w3.gtype == GT_F16 &&
           sub_.w6.gtype == GT_F16 && sub_.w3.N == c.sub_channels && sub_.w3.K == c.sub_channels &&
           sub_.w6.N == c.sub_channels && sub_.w6.K == c.sub_channels;
}

void Model::subsampling_kernels(const float* mel, int B, int T_max, bool stage_masks, float* out, hipStream_t s,
                                bool apply_xscaling) {
    const ModelConfig& c = cfg_;
    const int C = c.sub_channels, F = c.n_mels;
    // causal (CausalConv2D): pad 2 before / 1 after, and the per-stage input
    // masks on every path (subsampling.cpp:100-147, :283-300)
    const bool cz = c.causal_sub != 0;
    if (cz) stage_masks = true;
    const int T1 = sub_stage_len(T_max, cz), T2 = sub_stage_len(T1, cz), T3 = sub_stage_len(T2, cz);
    const int F1 = sub_stage_len(F, cz), F2 = sub_stage_len(F1, cz), F3 = sub_stage_len(F2, cz);
    (void)T1;
    (void)F1;
    Ws& w = *ws_;
    const int* dv = w.d_valid;
    const int Bc = w.Bcap;
    mark(KF_SUBSAMPLING, true);
    if (prec_ == PREC_F16 && sub_stage1_mfma_supported(C, F, cz))
        launch_sub_stage1_mfma(mel, stage_masks ? dv : nullptr, stage_masks ? dv + Bc : nullptr, sub_.w0, sub_.b0,
                               sub_.w2, sub_.b2, w.a2.p, B, T_max, s);
    else
        launch_sub_stage1(prec_, mel, stage_masks ? dv : nullptr, stage_masks ? dv + Bc : nullptr, sub_.w0, sub_.b0,
                          sub_.w2, sub_.b2, w.a2.p, B, F, T_max, C, s, cz);
    if (sub_tail_fused()) {
        launch_sub_tail(w.a2.p, sub_.tail_w, sub_.b3, sub_.w5, sub_.b5, sub_.b6, stage_masks ? dv + 2 * Bc : nullptr,
                        dv + 3 * Bc, w.flat.p, B, T2, T3, s);
    } else {
        gemm(sub_.w3, EPI_RELU, w.a2.p, C, (int64_t)B * T2 * F2, sub_.b3, w.a2p.p, C, 1.f, nullptr, 1, s, prec_,
             -1);
        launch_sub_dwconv(prec_, w.a2p.p, stage_masks ? dv + 2 * Bc : nullptr, sub_.w5, sub_.b5, w.a3.p, B, T2, F2,
                          C, s, cz);
        gemm(sub_.w6, EPI_RELU_TR, w.a3.p, C, (int64_t)B * T3 * F3, sub_.b6, w.flat.p, 0, 1.f, dv + 3 * Bc, T3, s,
             prec_, -1, nullptr, F3);
    }
    const float xs = (apply_xscaling && c.xscaling) ? std::sqrt((float)c.d_model) : 1.0f;  // encoder.cpp:122-124
    gemm(sub_.out, EPI_STORE_F32, w.flat.p, (int64_t)C * F3, (int64_t)B * T3, sub_.bout, out, c.d_model, xs,
         nullptr, 1, s, prec_, -1);
    mark(KF_SUBSAMPLING, false);
}

// ---------------------------------------------------------------------------
// one conformer layer (conformer.cpp:285-353) on the f32 residual stream x
// ---------------------------------------------------------------------------
void Model::layer_body(int l, float* x, int B, int T, const int* d_valid, bool first_ln_done,
                       bool fuse_next_ln, bool pos_all, hipStream_t s) {
    const ModelConfig& c = cfg_;
    const LayerDev& L = layers_[l];
    const int D = c.d_model, H = c.n_heads, dk = D / H;
    const int64_t M = (int64_t)B * T;
    Ws& w = *ws_;
    auto ln = [&](const float* g, const float* b) {
        LnParams p;
        p.x = x;
        p.g = g;
        p.b = b;
        p.y = w.h.p;
        p.M = M;
        p.D = D;
        mark(KF_LAYERNORM, true);
        launch_layernorm(prec_, p, s);
        mark(KF_LAYERNORM, false);
    };
    // With ln_fold_, norm_self_att, norm_conv and norm_feed_forward2 are folded:
    // the residual product before each leaves x * gamma (f16) and the row
    // statistics, and the product after it applies the normalisation in its
    // epilogue.  Buffers: h and g alternate as LayerNorm / attention / conv
    // outputs so that no product writes what it reads.
    const bool fold = ln_fold_ && !conv_capture_;
    // x may hold the previous block's stream before its norm_out (whose
    // per-row statistics are staged): FFN1 linear2 then adds to norm_out(x)
    const bool out_ln_in = first_ln_done && out_ln_pending_;
    out_ln_pending_ = false;
    // Stage A: x += 0.5 * FFN1(LN(x))
    if (!first_ln_done) ln(L.ff1_ln_g, L.ff1_ln_b);
    gemm(L.ff1_w1, EPI_SILU, w.h.p, D, M, L.ff1_b1, w.u.p, c.ff_dim, 1.f, nullptr, 1, s, prec_, KF_GEMM_FFN);
    if (fold) {
        const LayerDev* P = out_ln_in ? &layers_[l - 1] : nullptr;
        gemm_resid_ln(L.ff1_w2, w.u.p, M, L.ff1_b2, x, 0.5f, L.att_ln_g, w.h.p, s, KF_GEMM_FFN,
                      P ? (const float*)ws_->lnrows.p : nullptr, P ? P->out_ln_g : nullptr,
                      P ? P->out_ln_b : nullptr);
    } else {
        require(!out_ln_in, "norm_out left pending for a block that does not take it");
        gemm(L.ff1_w2, EPI_RESID, w.u.p, c.ff_dim, M, L.ff1_b2, x, D, 0.5f, nullptr, 1, s, prec_, KF_GEMM_FFN);
        ln(L.att_ln_g, L.att_ln_b);
    }
    // Stage B: x += MHSA(LN(x))
    if (fold) {
        const GemmParams p = fold_params(L.wqkv, w.h.p, M, L.qkv_c1, L.qkv_c2, w.qkv.p, 3 * D);
        mark(KF_GEMM_QKV, true);
        launch_gemm(prec_, L.wqkv.gtype, EPI_STORE, p, s);
        mark(KF_GEMM_QKV, false);
    } else {
        gemm(L.wqkv, EPI_STORE, w.h.p, D, M, L.bqkv, w.qkv.p, 3 * D, 1.f, nullptr, 1, s, prec_, KF_GEMM_QKV);
    }
    const size_t as = prec_ == PREC_F16 ? 2 : 4;
    const int ldp = pos_all ? c.n_layers * D : D;
    const void* pl = pos_all ? (const void*)((const uint8_t*)w.p.p + (size_t)l * D * as) : w.p.p;
    if (!pos_all)
        gemm(L.wpos, EPI_STORE, w.pe.p, D, 2 * (int64_t)T - 1, nullptr, w.p.p, D, 1.f, nullptr, 1, s, prec_,
             KF_GEMM_POS);
    {
        AttnParams a;
        a.q = w.qkv.p;
        a.k = (const uint8_t*)w.qkv.p + (size_t)D * as;
        a.v = (const uint8_t*)w.qkv.p + (size_t)2 * D * as;
        a.ldq = a.ldk = a.ldv = 3 * D;
        a.p = pl;
        a.ldp = ldp;
        a.bias_u = L.pos_u;
        a.bias_v = L.pos_v;
        a.valid = d_valid;
        a.out = w.h.p;
        a.ldo = D;
        a.B = B;
        a.T = T;
        a.H = H;
        a.dk = dk;
        a.scale = 1.0f / std::sqrt((float)dk);
        att_window(a);
        mark(KF_ATTENTION, true);
        launch_relpos_attention(prec_, a, s);
        mark(KF_ATTENTION, false);
    }
    // Stage C: x += conv(LN(x))
    if (fold) {
        gemm_resid_ln(L.wo, w.h.p, M, L.bo, x, 1.f, L.conv_ln_g, w.g.p, s, KF_GEMM_OUT);
        conv_front(L, w.g.p, M, d_valid, B, T, w.h.p, s, true);
        gemm_resid_ln(L.pw2, w.h.p, M, L.pw2_b, x, 1.f, L.ff2_ln_g, w.g.p, s, KF_GEMM_PW2);
    } else {
        gemm(L.wo, EPI_RESID, w.h.p, D, M, L.bo, x, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_OUT);
        ln(L.conv_ln_g, L.conv_ln_b);
        conv_front(L, w.h.p, M, d_valid, B, T, w.g.p, s);
        if (conv_capture_) {
            gemm(L.pw2, EPI_STORE_F32, w.g.p, D, M, L.pw2_b, conv_capture_, D, 1.f, nullptr, 1, s, prec_,
                 KF_GEMM_PW2);
            launch_add_f32(x, conv_capture_, M * D, s);
        } else {
            gemm(L.pw2, EPI_RESID, w.g.p, D, M, L.pw2_b, x, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_PW2);
        }
        ln(L.ff2_ln_g, L.ff2_ln_b);
    }
    // Stage D: x += 0.5 * FFN2(LN(x)); x = LN_out(x) [fused with next layer's LN_ff1]
    if (fold) {
        const GemmParams p = fold_params(L.ff2_w1, w.g.p, M, L.ff2_c1, L.ff2_c2, w.u.p, c.ff_dim);
        mark(KF_GEMM_FFN, true);
        launch_gemm(prec_, L.ff2_w1.gtype, EPI_SILU, p, s);
        mark(KF_GEMM_FFN, false);
    } else {
        gemm(L.ff2_w1, EPI_SILU, w.h.p, D, M, L.ff2_b1, w.u.p, c.ff_dim, 1.f, nullptr, 1, s, prec_, KF_GEMM_FFN);
    }
    gemm(L.ff2_w2, EPI_RESID, w.u.p, c.ff_dim, M, L.ff2_b2, x, D, 0.5f, nullptr, 1, s, prec_, KF_GEMM_FFN);
    {
        LnParams p;
        p.x = x;
        p.g = L.out_ln_g;
        p.b = L.out_ln_b;
        p.y_f32 = x;
        if (fuse_next_ln) {
            p.g2 = layers_[l + 1].ff1_ln_g;
            p.b2 = layers_[l + 1].ff1_ln_b;
            p.y = w.h.p;
            if (fold) {
                // x keeps the stream before norm_out: the next block's FFN1
                // linear2 (a residual + statistics product) applies norm_out
                // from its per-row statistics as it adds, so the f32 stream is
                // not written twice
                grow(ws_->lnrows, (size_t)M * 8);
                p.y_f32 = nullptr;
                p.rows = (float*)ws_->lnrows.p;
                out_ln_pending_ = true;
            }
        }
        p.M = M;
        p.D = D;
        mark(KF_LAYERNORM, true);
        launch_layernorm(prec_, p, s);
        mark(KF_LAYERNORM, false);
    }
}

// ---------------------------------------------------------------------------
// encoder (encoder.cpp:97-167)
// ---------------------------------------------------------------------------
int Model::encoder_forward(const float* mel, int B, int T_max, const int* valid_T, bool stage_masks,
                           float* out, int* valid_out, float* capture, hipStream_t s) {
    const int T3 = stage_lengths(B, T_max, valid_T, valid_out, s, false);
    encoder_kernels(mel, B, T_max, T3, stage_masks, out, capture, s);
    return T3;
}

// subsampling -> xscaling -> positional table -> blocks, on lengths staged by
// stage_lengths (encoder.cpp:97-167)
void Model::encoder_kernels(const float* mel, int B, int T_max, int T3, bool stage_masks, float* out,
                            float* capture, hipStream_t s) {
    subsampling_kernels(mel, B, T_max, stage_masks, out, s, true);
    const int* dvalid = ws_->d_valid + 3 * ws_->Bcap;
    ensure_pe(T3, s);
    const int L = cfg_.n_layers;
    const size_t MD = (size_t)B * T3 * cfg_.d_model;
    const bool pos_all = wpos_all_.ok();
    if (pos_all)
        gemm(wpos_all_, EPI_STORE, ws_->pe.p, cfg_.d_model, 2 * (int64_t)T3 - 1, nullptr, ws_->p.p,
             (int64_t)L * cfg_.d_model, 1.f, nullptr, 1, s, prec_, KF_GEMM_POS);
    out_ln_pending_ = false;
    for (int l = 0; l < L; ++l) {
        layer_body(l, out, B, T3, dvalid, l > 0, l + 1 < L, pos_all, s);
        if (capture && out_ln_pending_) {
            // the block's output is norm_out of what x holds
            LnParams p;
            p.x = out;
            p.g = layers_[l].out_ln_g;
            p.b = layers_[l].out_ln_b;
            p.y_f32 = capture + (size_t)l * MD;
            p.M = (int64_t)B * T3;
            p.D = cfg_.d_model;
            launch_layernorm(prec_, p, s);
        } else if (capture) {
            PKX_HIP(hipMemcpyAsync(capture + (size_t)l * MD, out, MD * 4, hipMemcpyDeviceToDevice, s));
        }
    }
}

void Model::conformer_layer_forward(int layer, const float* x, int B, int T, const int* valid, const float* pos,
                                    float* out, float* conv_out, hipStream_t s) {
    require(finalized_, "model not finalized");
    require(layer >= 0 && layer < cfg_.n_layers, "layer index out of range");
    const int T_mel = 8 * T;  // any T_max whose subsampled length is >= T sizes the workspace
    ensure_ws(B, T_mel);
    std::vector<int> v(B);
    for (int b = 0; b < B; ++b) {
        v[b] = valid ? valid[b] : T;
        require(v[b] >= 1 && v[b] <= T, "valid out of range");
    }
    {
        const std::vector<int>* slots[4] = {&v, &v, &v, &v};
        stage_valid(slots, s);
    }
    ensure_pe(T, s, pos);
    const size_t MD = (size_t)B * T * cfg_.d_model;
    if (out != x) PKX_HIP(hipMemcpyAsync(out, x, MD * 4, hipMemcpyDeviceToDevice, s));
    conv_capture_ = conv_out;
    out_ln_pending_ = false;
    try {
        layer_body(layer, out, B, T, ws_->d_valid + 3 * ws_->Bcap, false, false, false, s);
    } catch (...) {
        conv_capture_ = nullptr;
        throw;
    }
    conv_capture_ = nullptr;
}

void Model::relpos_attention_forward(int layer, const float* x, int B, int T, const int* valid, const float* pos,
                                     float* out, hipStream_t s) {
    require(finalized_, "model not finalized");
    require(layer >= 0 && layer < cfg_.n_layers, "layer index out of range");
    ensure_ws(B, 8 * T);
    std::vector<int> v(B);
    for (int b = 0; b < B; ++b) {
        v[b] = valid ? valid[b] : T;
        require(v[b] >= 1 && v[b] <= T, "valid out of range");
    }
    {
        const std::vector<int>* slots[4] = {&v, &v, &v, &v};
        stage_valid(slots, s);
    }
    ensure_pe(T, s, pos);
    const ModelConfig& c = cfg_;
    const LayerDev& L = layers_[layer];
    const int D = c.d_model, H = c.n_heads, dk = D / H;
    const int64_t M = (int64_t)B * T;
    Ws& w = *ws_;
    void* xa = cast_to_act(x, M * D, s);
    gemm(L.wqkv, EPI_STORE, xa, D, M, L.bqkv, w.qkv.p, 3 * D, 1.f, nullptr, 1, s, prec_, KF_GEMM_QKV);
    gemm(L.wpos, EPI_STORE, w.pe.p, D, 2 * (int64_t)T - 1, nullptr, w.p.p, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_POS);
    const size_t as = prec_ == PREC_F16 ? 2 : 4;
    AttnParams a;
    a.q = w.qkv.p;
    a.k = (const uint8_t*)w.qkv.p + (size_t)D * as;
    a.v = (const uint8_t*)w.qkv.p + (size_t)2 * D * as;
    a.ldq = a.ldk = a.ldv = 3 * D;
    a.p = w.p.p;
    a.ldp = D;
    a.bias_u = L.pos_u;
    a.bias_v = L.pos_v;
    a.valid = w.d_valid + 3 * w.Bcap;
    a.out = w.h.p;
    a.ldo = D;
    a.B = B;
    a.T = T;
    a.H = H;
    a.dk = dk;
    a.scale = 1.0f / std::sqrt((float)dk);
    att_window(a);
    launch_relpos_attention(prec_, a, s);
    gemm(L.wo, EPI_STORE_F32, w.h.p, D, M, L.bo, out, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_OUT);
}

void Model::conv_module_forward(int layer, const float* cin, int B, int T, const int* valid, float* out,
                                hipStream_t s) {
    require(finalized_, "model not finalized");
    require(layer >= 0 && layer < cfg_.n_layers, "layer index out of range");
    ensure_ws(B, 8 * T);
    std::vector<int> v(B);
    for (int b = 0; b < B; ++b) {
        v[b] = valid ? valid[b] : T;
        require(v[b] >= 1 && v[b] <= T, "valid out of range");
    }
    {
        const std::vector<int>* slots[4] = {&v, &v, &v, &v};
        stage_valid(slots, s);
    }
    const ModelConfig& c = cfg_;
    const LayerDev& L = layers_[layer];
    const int D = c.d_model;
    const int64_t M = (int64_t)B * T;
    Ws& w = *ws_;
    void* xa = cast_to_act(cin, M * D, s);
    conv_front(L, xa, M, w.d_valid + 3 * w.Bcap, B, T, w.h.p, s);
    gemm(L.pw2, EPI_STORE_F32, w.h.p, D, M, L.pw2_b, out, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_PW2);
}

// ---------------------------------------------------------------------------
// heads
// ---------------------------------------------------------------------------
void Model::ctc_forward(const float* enc, int64_t M, float* logprobs, int32_t* argmax, hipStream_t s) {
    require(finalized_ && heads_.ctc.ok(), "model has no CTC head");
    gemm(heads_.ctc, EPI_STORE_F32, enc, cfg_.d_model, M, heads_.ctc_b, logprobs, heads_.ctc.N, 1.f, nullptr, 1,
         s, PREC_F32, -1);
    launch_log_softmax_argmax(logprobs, logprobs, argmax, M, heads_.ctc.N, s);
}

void Model::tdt_joint_argmax(const float* enc, int64_t M, const float* g, float* logits, int32_t* tok,
                             int32_t* dur, hipStream_t s) {
    require(finalized_ && heads_.jout.ok(), "model has no TDT joint");
    const int Hj = heads_.jenc.N;
    Ws& w = *ws_;
    grow(w.pp, (size_t)Hj * 4);
    grow(w.logits, (size_t)M * Hj * 4);
    tdt_joint_argmax_in(enc, M, g, logits, tok, dur, (float*)w.pp.p, (float*)w.logits.p, s);
}

void Model::tdt_joint_argmax_in(const float* enc, int64_t M, const float* g, float* logits, int32_t* tok,
                                int32_t* dur, float* pp, float* hid, hipStream_t s) {
    require(finalized_ && heads_.jout.ok(), "model has no TDT joint");
    require(M >= 1, "joint: no frames");
    const int Hj = heads_.jenc.N;
    // every element of pp and hid read below is written first by these products
    gemm(heads_.jpred, EPI_STORE_F32, g, heads_.jpred.K, 1, heads_.jpred_b, pp, Hj, 1.f, nullptr, 1, s, PREC_F32,
         -1);
    gemm(heads_.jenc, EPI_RELU2_F32, enc, cfg_.d_model, M, heads_.jenc_b, hid, Hj, 1.f, nullptr, 1, s, PREC_F32, -1,
         pp);
    gemm(heads_.jout, EPI_STORE_F32, hid, Hj, M, heads_.jout_b, logits, heads_.jout.N, 1.f, nullptr, 1, s, PREC_F32,
         -1);
    launch_split_argmax(logits, M, heads_.n_tok, heads_.n_dur, tok, dur, s);
}

}  // namespace pkx

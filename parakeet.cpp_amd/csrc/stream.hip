// Cache-aware streaming encoder (StreamingEncoder, streaming_encoder.cpp) for
// a group of streams advanced in lockstep.  One step runs the causal
// subsampling of every stream's mel window, drops the pre-encode overlap,
// then for each conformer layer the products of the offline path (M = B x Tc
// rows) around two step kernels:
//   * stream_attn_kernel: relative-position attention of the chunk's Tc
//     queries over [cache ; chunk] keys with the streaming mask (empty cache
//     slots, chunked-limited window; streaming_encoder.cpp:146-245), then the
//     chunk's keys and values enter the per-layer ring;
//   * stream_conv_kernel: causal depthwise conv over [GLU history ; chunk]
//     + bias, LayerNorm (or folded BatchNorm) over channels, SiLU
//     (streaming_encoder.cpp:268-326), then the history advances.
#include <cmath>
#include <cstring>

#include "model.hpp"

namespace pkx {

namespace {

struct StreamAttnParams {
    const void* qkv;       // [M][3D] act: q | k | v (biases applied), row b*Tc + i
    float* kc;             // [B][CL][D] this layer's key ring
    float* vc;             // [B][CL][D] value ring
    const float* ppos;     // [np][D] positional projections, row r <-> distance CL + tc_max - 1 - r
    const float* bias_u;   // [D]
    const float* bias_v;   // [D]
    void* out;             // [M][D] act
    int Tc, CL, head, clc, chunk, left_chunks, tc_max, D, dk;
    float scale;
};

// One workgroup per (stream, head), 256 threads.  LDS: the chunk's q + u,
// q + v, k, v rows (f32, [Tc][dk] each) and the score block [Tc][CL + Tc].
template <typename T>
__global__ __launch_bounds__(256) void stream_attn_kernel(StreamAttnParams p) {
    extern __shared__ float sm[];
    const int b = blockIdx.x, h = blockIdx.y, dk = p.dk, D = p.D, Tc = p.Tc, CL = p.CL;
    const int Tk = CL + Tc;
    float* qu = sm;
    float* qv = qu + Tc * dk;
    float* kn = qv + Tc * dk;
    float* vn = kn + Tc * dk;
    float* sc = vn + Tc * dk;                    // [Tc][Tk]
    const T* qkv = (const T*)p.qkv;
    for (int e = threadIdx.x; e < Tc * dk; e += blockDim.x) {
        const int i = e / dk, c = e % dk;
        const T* row = qkv + (int64_t)(b * Tc + i) * 3 * D + h * dk + c;
        const float q = (float)row[0];
        qu[e] = q + p.bias_u[h * dk + c];
        qv[e] = q + p.bias_v[h * dk + c];
        kn[e] = (float)row[D];
        vn[e] = (float)row[2 * D];
    }
    __syncthreads();
    const float* kring = p.kc + (int64_t)b * CL * D + h * dk;
    const float* vring = p.vc + (int64_t)b * CL * D + h * dk;
    const int empty = CL - p.clc;
    const int rmax = CL + p.tc_max - 1;          // ppos row of distance 0 is rmax
    for (int e = threadIdx.x; e < Tc * Tk; e += blockDim.x) {
        const int i = e / Tk, kj = e % Tk;
        const int diff = (CL + i) / p.chunk - kj / p.chunk;
        float s = -INFINITY;
        if (kj >= empty && diff >= 0 && diff <= p.left_chunks) {
            const float* kr = kj < CL ? kring + (int64_t)((p.head + kj) % CL) * D : kn + (kj - CL) * dk;
            const float* pr = p.ppos + (int64_t)(rmax - (CL + i - kj)) * D + h * dk;
            const float* a = qu + i * dk;
            const float* c2 = qv + i * dk;
            float ac = 0.f, bd = 0.f;
            for (int c = 0; c < dk; ++c) {
                ac += a[c] * kr[c];
                bd += c2[c] * pr[c];
            }
            s = (ac + bd) * p.scale;
        }
        sc[e] = s;
    }
    __syncthreads();
    // softmax per query row, one wave per row
    const int wid = threadIdx.x / 64, lane = threadIdx.x % 64;
    for (int i = wid; i < Tc; i += blockDim.x / 64) {
        float* r = sc + i * Tk;
        float mx = -INFINITY;
        for (int j = lane; j < Tk; j += 64) mx = fmaxf(mx, r[j]);
        mx = wave_max(mx);
        float den = 0.f;
        for (int j = lane; j < Tk; j += 64) {
            const float ev = r[j] == -INFINITY ? 0.f : __expf(r[j] - mx);
            r[j] = ev;
            den += ev;
        }
        den = wave_sum(den);
        const float inv = 1.0f / den;
        for (int j = lane; j < Tk; j += 64) r[j] *= inv;
    }
    __syncthreads();
    T* out = (T*)p.out;
    for (int e = threadIdx.x; e < Tc * dk; e += blockDim.x) {
        const int i = e / dk, c = e % dk;
        const float* r = sc + i * Tk;
        float acc = 0.f;
        for (int kj = 0; kj < CL; ++kj) {
            const float pj = r[kj];
            if (pj != 0.f) acc += pj * vring[(int64_t)((p.head + kj) % CL) * D + c];
        }
        for (int q = 0; q < Tc; ++q) acc += r[CL + q] * vn[q * dk + c];
        out[(int64_t)(b * Tc + i) * D + h * dk + c] = to_act<T>(acc);
    }
    __syncthreads();
    // the chunk's frames take the ring slots of the oldest ones: logical
    // order [cache[Tc:] ; chunk] with the ring start moved by Tc (host side)
    float* kw = p.kc + (int64_t)b * CL * D + h * dk;
    float* vw = p.vc + (int64_t)b * CL * D + h * dk;
    for (int e = threadIdx.x; e < Tc * dk; e += blockDim.x) {
        const int q = e / dk, c = e % dk;
        const int64_t slot = (int64_t)((p.head + q) % CL) * D + c;
        kw[slot] = kn[e];
        vw[slot] = vn[e];
    }
}

struct StreamConvParams {
    const void* glu;       // [M][D] act, row b*Tc + t
    float* cc;             // [B][LP][D] this layer's GLU history, oldest first
    const float* w;        // [D][K]
    const float* dw_b;     // [D] or null
    const float* g;        // LayerNorm gamma (ln) or BatchNorm scale
    const float* beta;     // LayerNorm beta (ln) or BatchNorm shift
    void* out;             // [M][D] act
    int Tc, D, K, ln;
};

constexpr int SC_FRAMES = 16;   // conv outputs staged in LDS per pass

// One workgroup per stream, 256 threads; a thread owns channels c = tid + 256 k
// for the depthwise conv and the history update, a wave owns frames for the
// channel normalisation.
template <typename T>
__global__ __launch_bounds__(256) void stream_conv_kernel(StreamConvParams p) {
    extern __shared__ float dwo[];               // [SC_FRAMES][D]
    const int b = blockIdx.x, D = p.D, K = p.K, LP = K - 1, Tc = p.Tc;
    const T* glu = (const T*)p.glu + (int64_t)b * Tc * D;
    float* hist = p.cc + (int64_t)b * LP * D;
    T* out = (T*)p.out + (int64_t)b * Tc * D;
    const int wid = threadIdx.x / 64, lane = threadIdx.x % 64, nw = blockDim.x / 64;
    for (int f0 = 0; f0 < Tc; f0 += SC_FRAMES) {
        const int nf = Tc - f0 < SC_FRAMES ? Tc - f0 : SC_FRAMES;
        for (int c = threadIdx.x; c < D; c += blockDim.x) {
            const float* wk = p.w + (int64_t)c * K;
            const float bias = p.dw_b ? p.dw_b[c] : 0.f;
            for (int t = 0; t < nf; ++t) {
                float acc = 0.f;
                for (int k = 0; k < K; ++k) {
                    const int u = f0 + t + k;    // index into [history (LP) ; chunk (Tc)]
                    const float v = u < LP ? hist[(int64_t)u * D + c] : (float)glu[(int64_t)(u - LP) * D + c];
                    acc += wk[k] * v;
                }
                dwo[t * D + c] = acc + bias;
            }
        }
        __syncthreads();
        for (int t = wid; t < nf; t += nw) {
            const float* r = dwo + t * D;
            T* o = out + (int64_t)(f0 + t) * D;
            if (p.ln) {
                float s = 0.f;
                for (int c = lane; c < D; c += 64) s += r[c];
                const float mean = wave_sum(s) / D;
                float s2 = 0.f;
                for (int c = lane; c < D; c += 64) {
                    const float d = r[c] - mean;
                    s2 += d * d;
                }
                const float rstd = 1.0f / sqrtf(wave_sum(s2) / D + 1e-5f);
                for (int c = lane; c < D; c += 64) {
                    float y = (r[c] - mean) * rstd;
                    y = y * p.g[c] + p.beta[c];
                    o[c] = to_act<T>(y / (1.0f + __expf(-y)));
                }
            } else {
                for (int c = lane; c < D; c += 64) {
                    const float y = r[c] * p.g[c] + p.beta[c];
                    o[c] = to_act<T>(y / (1.0f + __expf(-y)));
                }
            }
        }
        __syncthreads();
    }
    // history <- the last LP entries of [history ; chunk]; entry j reads entry
    // j + Tc, which a later iteration of the same thread overwrites
    for (int c = threadIdx.x; c < D; c += blockDim.x)
        for (int j = 0; j < LP; ++j) {
            const int u = j + Tc;
            const float v = u < LP ? hist[(int64_t)u * D + c] : (float)glu[(int64_t)(u - LP) * D + c];
            hist[(int64_t)j * D + c] = v;
        }
}

}  // namespace

StreamState::~StreamState() {
    for (void* q : allocs) hipFree(q);
}

std::unique_ptr<StreamState> Model::stream_create(int n_streams, int max_window, hipStream_t s) {
    require(finalized_, "model not finalized");
    const ModelConfig& c = cfg_;
    require(c.att_limited && c.conv_causal && c.causal_sub && c.stream_cache_len > 0,
            "streaming encoder: the model has no cache-aware streaming configuration");
    require(n_streams >= 1 && max_window >= 1, "streaming encoder: n_streams and max_window must be positive");
    require(c.conv_kernel >= 2, "streaming encoder: conv kernel must have at least 2 taps");
    const int D = c.d_model, dk = D / c.n_heads;
    require(dk <= 256 && D % 8 == 0 && D <= 2048, "streaming encoder: d_model above 2048 or head width above 256");
    // LDS beyond the default 64 KiB: attention up to (4 dk + CL + 32) x 32
    // floats, conv SC_FRAMES x D floats (both checked per launch)
    for (const void* fn : {(const void*)stream_attn_kernel<f16>, (const void*)stream_attn_kernel<float>,
                           (const void*)stream_conv_kernel<f16>, (const void*)stream_conv_kernel<float>})
        PKX_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    std::unique_ptr<StreamState> st(new StreamState());
    st->B = n_streams;
    st->max_window = max_window;
    st->tsub_max = subsampled_len(max_window, true);
    st->tc_max = st->tsub_max;
    st->CL = c.stream_cache_len;
    st->LP = c.conv_kernel - 1;
    require(st->tc_max <= st->CL, "streaming encoder: a window yields more frames than the attention cache holds");
    require(st->tc_max <= 32, "streaming encoder: at most 32 encoder frames per chunk (max_window <= 255)");
    st->np = st->CL + 2 * st->tc_max - 1;
    const size_t as = prec_ == PREC_F16 ? 2 : 4, L = (size_t)c.n_layers, B = (size_t)n_streams;
    const size_t M = B * (size_t)st->tc_max;
    auto al = [&](size_t bytes) {
        void* q = nullptr;
        PKX_HIP(hipMalloc(&q, bytes));
        st->allocs.push_back(q);
        return q;
    };
    st->kc = (float*)al(L * B * st->CL * D * 4);
    st->vc = (float*)al(L * B * st->CL * D * 4);
    st->cc = (float*)al(L * B * st->LP * D * 4);
    st->ppos = (float*)al(L * st->np * D * 4);
    st->sub = (float*)al(B * st->tsub_max * D * 4);
    st->x = (float*)al(M * D * 4);
    st->h = al(M * D * as);
    st->u = al(M * c.ff_dim * as);
    st->qkv = al(M * 3 * D * as);
    st->g = al(M * D * as);
    // linear_pos of the positional rows the chunks use (pos_enc(cache_len)
    // spans 2 (Tc + CL) - 1 positions; a query-key pair reads the row of its
    // distance, streaming_encoder.cpp:374-381 with the rel_shift of :180-190)
    const int Pn = st->CL + st->tc_max;
    void* pe = al((size_t)(2 * Pn - 1) * D * as);
    launch_rel_pos_encoding(prec_, pe, Pn, D, s);
    for (int l = 0; l < c.n_layers; ++l)
        gemm(layers_[(size_t)l].wpos, EPI_STORE_F32, pe, D, st->np, nullptr, st->ppos + (size_t)l * st->np * D, D,
             1.f, nullptr, 1, s, prec_, KF_GEMM_POS);
    stream_reset(*st, s);
    PKX_HIP(hipStreamSynchronize(s));
    return st;
}

void Model::stream_reset(StreamState& st, hipStream_t s) {
    const ModelConfig& c = cfg_;
    const size_t L = (size_t)c.n_layers, B = (size_t)st.B, D = (size_t)c.d_model;
    PKX_HIP(hipMemsetAsync(st.kc, 0, L * B * st.CL * D * 4, s));
    PKX_HIP(hipMemsetAsync(st.vc, 0, L * B * st.CL * D * 4, s));
    PKX_HIP(hipMemsetAsync(st.cc, 0, L * B * st.LP * D * 4, s));
    st.step = 0;
    st.clc = 0;
    st.head = 0;
}

int Model::stream_chunk_len(const StreamState& st, int n) const {
    const int drop = st.step != 0 ? cfg_.stream_drop_extra : 0;   // streaming_encoder.cpp:350-366
    const int tc = subsampled_len(n, true) - drop;
    return tc < 0 ? 0 : tc;
}

int Model::stream_step(StreamState& st, const float* mel, int n, bool is_last, float* out, hipStream_t s) {
    const ModelConfig& c = cfg_;
    require(n >= 1 && n <= st.max_window, "streaming encoder: window length outside [1, max_window]");
    const int Tc = stream_chunk_len(st, n);
    if (Tc == 0) {                                   // streaming_encoder.cpp:367-371
        st.step += 1;
        return 0;
    }
    const int D = c.d_model, H = c.n_heads, dk = D / H, B = st.B;
    const int drop = st.step != 0 ? c.stream_drop_extra : 0;
    const int64_t M = (int64_t)B * Tc;
    // 1. causal subsampling of every window (all frames audio), xscaling, drop
    std::vector<int> vn((size_t)B, n);
    const int Tsub = subsampling_forward(mel, B, n, vn.data(), true, st.sub, nullptr, s, true, true);
    PKX_HIP(hipMemcpy2DAsync(st.x, (size_t)Tc * D * 4, st.sub + (size_t)drop * D, (size_t)Tsub * D * 4,
                             (size_t)Tc * D * 4, (size_t)B, hipMemcpyDeviceToDevice, s));
    auto ln = [&](const float* g, const float* b, void* y, float* y32) {
        LnParams p;
        p.x = st.x;
        p.g = g;
        p.b = b;
        p.y = y;
        p.y_f32 = y32;
        p.M = M;
        p.D = D;
        mark(KF_LAYERNORM, true);
        launch_layernorm(prec_, p, s);
        mark(KF_LAYERNORM, false);
    };
    const size_t LB = (size_t)B;
    for (int l = 0; l < c.n_layers; ++l) {
        const LayerDev& L = layers_[(size_t)l];
        // A: x += 0.5 FFN1(LN(x))
        ln(L.ff1_ln_g, L.ff1_ln_b, st.h, nullptr);
        gemm(L.ff1_w1, EPI_SILU, st.h, D, M, L.ff1_b1, st.u, c.ff_dim, 1.f, nullptr, 1, s, prec_, KF_GEMM_FFN);
        gemm(L.ff1_w2, EPI_RESID, st.u, c.ff_dim, M, L.ff1_b2, st.x, D, 0.5f, nullptr, 1, s, prec_, KF_GEMM_FFN);
        // B: x += MHSA(LN(x)) over [cache ; chunk]
        ln(L.att_ln_g, L.att_ln_b, st.h, nullptr);
        gemm(L.wqkv, EPI_STORE, st.h, D, M, L.bqkv, st.qkv, 3 * D, 1.f, nullptr, 1, s, prec_, KF_GEMM_QKV);
        {
            StreamAttnParams a;
            a.qkv = st.qkv;
            a.kc = st.kc + (size_t)l * LB * st.CL * D;
            a.vc = st.vc + (size_t)l * LB * st.CL * D;
            a.ppos = st.ppos + (size_t)l * st.np * D;
            a.bias_u = L.pos_u;
            a.bias_v = L.pos_v;
            a.out = st.g;
            a.Tc = Tc;
            a.CL = st.CL;
            a.head = st.head;
            a.clc = st.clc;
            a.chunk = c.att_right + 1;
            a.left_chunks = c.att_left / a.chunk;
            a.tc_max = st.tc_max;
            a.D = D;
            a.dk = dk;
            a.scale = 1.0f / std::sqrt((float)dk);
            const uint32_t shm = (uint32_t)(4 * Tc * dk + Tc * (st.CL + Tc)) * 4u;
            require(shm <= 160u * 1024u, "streaming encoder: attention cache too long for LDS");
            mark(KF_ATTENTION, true);
            if (prec_ == PREC_F16)
                launch(stream_attn_kernel<f16>, dim3(B, H), dim3(256), shm, s, a);
            else
                launch(stream_attn_kernel<float>, dim3(B, H), dim3(256), shm, s, a);
            PKX_LAUNCH_CHECK();
            mark(KF_ATTENTION, false);
        }
        gemm(L.wo, EPI_RESID, st.g, D, M, L.bo, st.x, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_OUT);
        // C: x += conv(LN(x)) with the causal depthwise conv over [history ; chunk]
        ln(L.conv_ln_g, L.conv_ln_b, st.h, nullptr);
        gemm(L.pw1, EPI_GLU, st.h, D, M, L.pw1_b, st.g, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_PW1_GLU);
        {
            StreamConvParams q;
            q.glu = st.g;
            q.cc = st.cc + (size_t)l * LB * st.LP * D;
            q.w = L.dw_w;
            q.dw_b = L.dw_b;
            q.ln = c.conv_ln;
            q.g = c.conv_ln ? L.cn_g : L.bn_scale;
            q.beta = c.conv_ln ? L.cn_b : L.bn_shift;
            q.out = st.h;
            q.Tc = Tc;
            q.D = D;
            q.K = c.conv_kernel;
            const uint32_t shm = (uint32_t)(SC_FRAMES * D) * 4u;
            mark(KF_DWCONV, true);
            if (prec_ == PREC_F16)
                launch(stream_conv_kernel<f16>, dim3(B), dim3(256), shm, s, q);
            else
                launch(stream_conv_kernel<float>, dim3(B), dim3(256), shm, s, q);
            PKX_LAUNCH_CHECK();
            mark(KF_DWCONV, false);
        }
        gemm(L.pw2, EPI_RESID, st.h, D, M, L.pw2_b, st.x, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_PW2);
        // D: x += 0.5 FFN2(LN(x)); x = norm_out(x)
        ln(L.ff2_ln_g, L.ff2_ln_b, st.h, nullptr);
        gemm(L.ff2_w1, EPI_SILU, st.h, D, M, L.ff2_b1, st.u, c.ff_dim, 1.f, nullptr, 1, s, prec_, KF_GEMM_FFN);
        gemm(L.ff2_w2, EPI_RESID, st.u, c.ff_dim, M, L.ff2_b2, st.x, D, 0.5f, nullptr, 1, s, prec_, KF_GEMM_FFN);
        ln(L.out_ln_g, L.out_ln_b, nullptr, st.x);
    }
    PKX_HIP(hipMemcpyAsync(out, st.x, (size_t)M * D * 4, hipMemcpyDeviceToDevice, s));
    st.clc = st.clc + Tc < st.CL ? st.clc + Tc : st.CL;   // streaming_encoder.cpp:447-448
    st.head = (st.head + Tc) % st.CL;
    st.step += 1;
    return is_last ? Tc : (c.stream_valid_out_len < Tc ? c.stream_valid_out_len : Tc);
}

}  // namespace pkx

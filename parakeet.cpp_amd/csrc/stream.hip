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
    void* kc;              // [B][CL][D] act: this layer's key ring
    void* vc;              // [B][CL][D] act: value ring
    const void* ppos;      // [np][D] act: positional projections, row r <-> distance CL + tc_max - 1 - r
    const float* bias_u;   // [D]
    const float* bias_v;   // [D]
    void* out;             // [M][D] act
    int Tc, CL, head, clc, chunk, left_chunks, tc_max, D, dk;
    float scale;
};

// LDS bytes of one stream_attn_kernel workgroup: the values of the Tk = CL + Tc
// frames in the activation type, rows padded by 16 bytes (16-byte aligned rows
// whose starts step through the bank quads); q + u and q + v [Tc][dk] and the
// scores [Tc][Tk] (rounded up to 16 bytes) in f32.
inline int stream_attn_lds_bytes(int Tc, int CL, int dk, int as) {
    const int Tk = CL + Tc;
    // + the P.V partials: 256 threads x 16 bytes of f32 (4 or 8 floats)
    return Tk * (dk + 16 / as) * as + (2 * Tc * dk + (Tc * Tk + 3) / 4 * 4) * 4 + 256 * (16 / as) * 4;
}

// One workgroup per (stream, head), 256 threads.  The values are staged in LDS
// with coalesced 16-byte loads (ring rows in logical order, then the chunk's
// own); a thread owns a (query, key) score and reads that key's row and its
// positional row straight from memory (each one contiguous 16-byte vectors,
// issued together), a wave a softmax row, and a thread 16 bytes of one
// query's output channels.  Keeping only the values in LDS lets the whole
// grid of a step (streams x heads) be resident at once.
// DK > 0: the head width at compile time (dot products fully unrolled); DK = 0
// reads it from p.dk.
template <typename T, int DK>
__global__ __launch_bounds__(256) void stream_attn_kernel(StreamAttnParams p) {
    extern __shared__ float sm[];
    constexpr int VE = 16 / sizeof(T);           // elements per 16-byte vector
    const int b = blockIdx.x, h = blockIdx.y, dk = DK > 0 ? DK : p.dk, D = p.D, Tc = p.Tc, CL = p.CL;
    const int Tk = CL + Tc, ld = dk + VE;
    float* qu = sm;                              // [Tc][dk]
    float* qv = qu + Tc * dk;                    // [Tc][dk]
    float* sc = qv + Tc * dk;                    // [Tc][Tk]
    T* vs = (T*)(sc + (Tc * Tk + 3) / 4 * 4);    // [Tk][ld]
    const T* qkv = (const T*)p.qkv;
    T* kring = (T*)p.kc + (int64_t)b * CL * D + h * dk;
    T* vring = (T*)p.vc + (int64_t)b * CL * D + h * dk;
    // key row kj of [ring in logical order ; chunk]
    auto key_row = [&](int kj) -> const T* {
        return kj < CL ? kring + (int64_t)((p.head + kj) % CL) * D
                       : qkv + (int64_t)(b * Tc + kj - CL) * 3 * D + D + h * dk;
    };
    // 16-byte loads (dk % 8 == 0, D % 8 == 0), several in flight per thread
    const int vpr = dk / VE;
#pragma unroll 4
    for (int e = threadIdx.x; e < Tk * vpr; e += blockDim.x) {
        const int r = e / vpr, c0 = (e % vpr) * VE;
        const T* sv = r < CL ? vring + (int64_t)((p.head + r) % CL) * D + c0
                             : qkv + (int64_t)(b * Tc + r - CL) * 3 * D + 2 * D + h * dk + c0;
        *(int4v*)(vs + r * ld + c0) = *(const int4v*)sv;
    }
    for (int e = threadIdx.x; e < Tc * dk; e += blockDim.x) {
        const int i = e / dk, c = e % dk;
        const float q = (float)qkv[(int64_t)(b * Tc + i) * 3 * D + h * dk + c];
        qu[e] = q + p.bias_u[h * dk + c];
        qv[e] = q + p.bias_v[h * dk + c];
    }
    __syncthreads();
    // positional row of distance CL + Tc - 1 - j is ppos row tc_max - Tc + j
    const T* pband = (const T*)p.ppos + (int64_t)(p.tc_max - Tc) * D + h * dk;
    const int empty = CL - p.clc;
    for (int e = threadIdx.x; e < Tc * Tk; e += blockDim.x) {
        const int i = e / Tk, kj = e % Tk;
        const int diff = (CL + i) / p.chunk - kj / p.chunk;
        float s = -INFINITY;
        if (kj >= empty && diff >= 0 && diff <= p.left_chunks) {
            // rel_shift of the [Tc][2 Tk - 1] block: column Tc - 1 - i + kj
            const T* kr = key_row(kj);
            const T* pr = pband + (int64_t)(Tc - 1 - i + kj) * D;
            const float* a = qu + i * dk;
            const float* a2 = qv + i * dk;
            float ac = 0.f, bd = 0.f;
#pragma unroll 8
            for (int c = 0; c < dk; c += VE) {
                const int4v kk = *(const int4v*)(kr + c), pk = *(const int4v*)(pr + c);
                const T* kx = (const T*)&kk;
                const T* px = (const T*)&pk;
#pragma unroll
                for (int e4 = 0; e4 < VE; e4 += 4) {
                    const float4v av = *(const float4v*)(a + c + e4), bv = *(const float4v*)(a2 + c + e4);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        ac += av[q] * (float)kx[e4 + q];
                        bd += bv[q] * (float)px[e4 + q];
                    }
                }
            }
            s = (ac + bd) * p.scale;
        }
        sc[e] = s;
    }
    __syncthreads();
    // softmax per query row, one wave per row (the query's own frame is
    // always visible, so no row is empty)
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
    // P.V: the Tc x vpr output vectors, each over KS key slices (all threads
    // busy when Tc * vpr is small); the slices' partials are summed in slice
    // order through LDS
    const int nvo = Tc * vpr, KS = nvo >= (int)blockDim.x ? 1 : (int)blockDim.x / nvo;
    float* red = (float*)(vs + Tk * ld);         // [KS][nvo][VE] f32, after the values
    for (int e = threadIdx.x; e < nvo * KS; e += blockDim.x) {
        const int o = e % nvo, ks = e / nvo;
        const int i = o / vpr, c0 = (o % vpr) * VE;
        const float* r = sc + i * Tk;
        float acc[VE];
#pragma unroll
        for (int q = 0; q < VE; ++q) acc[q] = 0.f;
        const int k0 = ks * Tk / KS, k1 = (ks + 1) * Tk / KS;
#pragma unroll 2
        for (int kj = k0; kj < k1; ++kj) {
            const float w = r[kj];
            const int4v vv = *(const int4v*)(vs + kj * ld + c0);
            const T* vx = (const T*)&vv;
#pragma unroll
            for (int q = 0; q < VE; ++q) acc[q] += w * (float)vx[q];
        }
        if (KS == 1) {
            T ov[VE];
#pragma unroll
            for (int q = 0; q < VE; ++q) ov[q] = to_act<T>(acc[q]);
            *(int4v*)(out + (int64_t)(b * Tc + i) * D + h * dk + c0) = *(const int4v*)ov;
        } else {
#pragma unroll
            for (int q = 0; q < VE; q += 4)
                *(float4v*)(red + ((int64_t)ks * nvo + o) * VE + q) =
                    (float4v){acc[q], acc[q + 1], acc[q + 2], acc[q + 3]};
        }
    }
    if (KS > 1) {
        __syncthreads();
        for (int o = threadIdx.x; o < nvo; o += blockDim.x) {
            const int i = o / vpr, c0 = (o % vpr) * VE;
            float acc[VE];
#pragma unroll
            for (int q = 0; q < VE; ++q) acc[q] = red[(int64_t)o * VE + q];
            for (int ks = 1; ks < KS; ++ks) {
#pragma unroll
                for (int q = 0; q < VE; q += 4) {
                    const float4v v = *(const float4v*)(red + ((int64_t)ks * nvo + o) * VE + q);
                    acc[q] += v[0], acc[q + 1] += v[1], acc[q + 2] += v[2], acc[q + 3] += v[3];
                }
            }
            T ov[VE];
#pragma unroll
            for (int q = 0; q < VE; ++q) ov[q] = to_act<T>(acc[q]);
            *(int4v*)(out + (int64_t)(b * Tc + i) * D + h * dk + c0) = *(const int4v*)ov;
        }
    }
    // the chunk's frames take the ring slots of the oldest ones (every ring
    // read of this workgroup is done: the key reads fed the scores before the
    // barriers above, the value reads went through LDS): logical order
    // [cache[Tc:] ; chunk] with the ring start moved by Tc on the host
    for (int e = threadIdx.x; e < Tc * vpr; e += blockDim.x) {
        const int q = e / vpr, c0 = (e % vpr) * VE;
        const int64_t slot = (int64_t)((p.head + q) % CL) * D + c0;
        *(int4v*)(kring + slot) = *(const int4v*)(key_row(CL + q) + c0);
        *(int4v*)(vring + slot) = *(const int4v*)(vs + (CL + q) * ld + c0);
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

// The common shape (K taps known at compile time, Tc <= TCM): every global
// load of a channel (taps, history, chunk) is issued before any arithmetic,
// the history update is written from registers.
template <typename T, int K, int TCM>
__global__ __launch_bounds__(512) void stream_conv_kernel_k(StreamConvParams p) {
    extern __shared__ float dwo[];               // [TCM][D]
    constexpr int LP = K - 1;
    const int b = blockIdx.x, D = p.D, Tc = p.Tc;
    const T* glu = (const T*)p.glu + (int64_t)b * Tc * D;
    float* hist = p.cc + (int64_t)b * LP * D;
    T* out = (T*)p.out + (int64_t)b * Tc * D;
    for (int c = threadIdx.x; c < D; c += blockDim.x) {
        float wk[K], seq[LP + TCM];
#pragma unroll
        for (int k = 0; k < K; ++k) wk[k] = p.w[(int64_t)c * K + k];
#pragma unroll
        for (int u = 0; u < LP; ++u) seq[u] = hist[(int64_t)u * D + c];
#pragma unroll
        for (int t = 0; t < TCM; ++t) seq[LP + t] = t < Tc ? (float)glu[(int64_t)t * D + c] : 0.f;
        const float bias = p.dw_b ? p.dw_b[c] : 0.f;
#pragma unroll
        for (int t = 0; t < TCM; ++t) {
            if (t < Tc) {
                float acc = 0.f;
#pragma unroll
                for (int k = 0; k < K; ++k) acc += wk[k] * seq[t + k];
                dwo[t * D + c] = acc + bias;
            }
        }
        // history <- the last LP entries of [history ; chunk]
#pragma unroll
        for (int j = 0; j < LP; ++j) {
#pragma unroll
            for (int t = 0; t <= TCM; ++t)
                if (t == Tc) hist[(int64_t)j * D + c] = seq[j + t];
        }
    }
    __syncthreads();
    const int wid = threadIdx.x / 64, lane = threadIdx.x % 64, nw = blockDim.x / 64;
    for (int t = wid; t < Tc; t += nw) {
        const float* r = dwo + t * D;
        T* o = out + (int64_t)t * D;
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
}

constexpr int SC_TCM = 8;   // chunk frames of the compile-time conv path

}  // namespace

StreamState::~StreamState() {
    for (void* q : allocs) (void)hipFree(q);
}

std::unique_ptr<StreamState> Model::stream_create(int n_streams, int max_window, hipStream_t s) {
    require(finalized_, "model not finalized");
    const ModelConfig& c = cfg_;
    require(c.att_limited && c.conv_causal && c.causal_sub && c.stream_cache_len > 0,
            "streaming encoder: the model has no cache-aware streaming configuration");
    require(n_streams >= 1 && max_window >= 1, "streaming encoder: n_streams and max_window must be positive");
    require(c.conv_kernel >= 2, "streaming encoder: conv kernel must have at least 2 taps");
    const int D = c.d_model, dk = D / c.n_heads;
    require(dk <= 256 && dk % 8 == 0 && D % 8 == 0 && D <= 2048,
            "streaming encoder: d_model above 2048, or head width above 256 or not a multiple of 8");
    // LDS beyond the default 64 KiB (attention: stream_attn_lds_bytes, conv:
    // SC_FRAMES x D floats)
    for (const void* fn : {(const void*)stream_attn_kernel<f16, 0>, (const void*)stream_attn_kernel<float, 0>,
                           (const void*)stream_attn_kernel<f16, 64>, (const void*)stream_attn_kernel<float, 64>,
                           (const void*)stream_attn_kernel<f16, 128>, (const void*)stream_attn_kernel<float, 128>,
                           (const void*)stream_conv_kernel<f16>, (const void*)stream_conv_kernel<float>,
                           (const void*)stream_conv_kernel_k<f16, 9, SC_TCM>,
                           (const void*)stream_conv_kernel_k<float, 9, SC_TCM>})
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
    require(stream_attn_lds_bytes(st->tc_max, st->CL, dk, prec_ == PREC_F16 ? 2 : 4) <= 160 * 1024,
            "streaming encoder: attention cache x head width too large for one workgroup's LDS");
    st->np = st->CL + 2 * st->tc_max - 1;
    const size_t as = prec_ == PREC_F16 ? 2 : 4, L = (size_t)c.n_layers, B = (size_t)n_streams;
    const size_t M = B * (size_t)st->tc_max;
    auto al = [&](size_t bytes) {
        void* q = nullptr;
        PKX_HIP(hipMalloc(&q, bytes));
        st->allocs.push_back(q);
        return q;
    };
    st->kc = al(L * B * st->CL * D * as);
    st->vc = al(L * B * st->CL * D * as);
    st->cc = (float*)al(L * B * st->LP * D * 4);
    st->ppos = al(L * st->np * D * as);
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
        gemm(layers_[(size_t)l].wpos, EPI_STORE, pe, D, st->np, nullptr, (uint8_t*)st->ppos + (size_t)l * st->np * D * as, D,
             1.f, nullptr, 1, s, prec_, KF_GEMM_POS);
    stream_reset(*st, s);
    PKX_HIP(hipStreamSynchronize(s));
    return st;
}

void Model::stream_reset(StreamState& st, hipStream_t s) {
    const ModelConfig& c = cfg_;
    const size_t L = (size_t)c.n_layers, B = (size_t)st.B, D = (size_t)c.d_model;
    const size_t as = prec_ == PREC_F16 ? 2 : 4;
    PKX_HIP(hipMemsetAsync(st.kc, 0, L * B * st.CL * D * as, s));
    PKX_HIP(hipMemsetAsync(st.vc, 0, L * B * st.CL * D * as, s));
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
    auto ln = [&](const float* g, const float* b, void* y, float* y32, const float* g2 = nullptr,
                  const float* b2 = nullptr) {
        LnParams p;
        p.x = st.x;
        p.g = g;
        p.b = b;
        p.y = y;
        p.y_f32 = y32;
        p.g2 = g2;
        p.b2 = b2;
        p.M = M;
        p.D = D;
        mark(KF_LAYERNORM, true);
        launch_layernorm(prec_, p, s);
        mark(KF_LAYERNORM, false);
    };
    const size_t LB = (size_t)B, as = prec_ == PREC_F16 ? 2 : 4;
    // f16 path: norm_self_att, norm_conv and norm_feed_forward2 folded into the
    // products after them, as in the offline forward (the residual product
    // before each leaves x * gamma and the row statistics); norm_out fused with
    // the next layer's norm_feed_forward1.
    const bool fold = ln_fold_;
    ln(layers_[0].ff1_ln_g, layers_[0].ff1_ln_b, st.h, nullptr);
    for (int l = 0; l < c.n_layers; ++l) {
        const LayerDev& L = layers_[(size_t)l];
        // A: x += 0.5 FFN1(LN(x))   (h holds LN_ff1(x))
        gemm(L.ff1_w1, EPI_SILU, st.h, D, M, L.ff1_b1, st.u, c.ff_dim, 1.f, nullptr, 1, s, prec_, KF_GEMM_FFN);
        // B: x += MHSA(LN(x)) over [cache ; chunk]
        if (fold) {
            gemm_resid_ln(L.ff1_w2, st.u, M, L.ff1_b2, st.x, 0.5f, L.att_ln_g, st.h, s, KF_GEMM_FFN);
            const GemmParams p = fold_params(L.wqkv, st.h, M, L.qkv_c1, L.qkv_c2, st.qkv, 3 * D);
            mark(KF_GEMM_QKV, true);
            launch_gemm(prec_, L.wqkv.gtype, EPI_STORE, p, s);
            mark(KF_GEMM_QKV, false);
        } else {
            gemm(L.ff1_w2, EPI_RESID, st.u, c.ff_dim, M, L.ff1_b2, st.x, D, 0.5f, nullptr, 1, s, prec_,
                 KF_GEMM_FFN);
            ln(L.att_ln_g, L.att_ln_b, st.h, nullptr);
            gemm(L.wqkv, EPI_STORE, st.h, D, M, L.bqkv, st.qkv, 3 * D, 1.f, nullptr, 1, s, prec_, KF_GEMM_QKV);
        }
        {
            StreamAttnParams a;
            a.qkv = st.qkv;
            a.kc = (uint8_t*)st.kc + (size_t)l * LB * st.CL * D * as;
            a.vc = (uint8_t*)st.vc + (size_t)l * LB * st.CL * D * as;
            a.ppos = (const uint8_t*)st.ppos + (size_t)l * st.np * D * as;
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
            const uint32_t shm = (uint32_t)stream_attn_lds_bytes(Tc, st.CL, dk, (int)as);
            mark(KF_ATTENTION, true);
            const dim3 grid(B, H);
            if (prec_ == PREC_F16) {
                if (dk == 64) launch(stream_attn_kernel<f16, 64>, grid, dim3(256), shm, s, a);
                else if (dk == 128) launch(stream_attn_kernel<f16, 128>, grid, dim3(256), shm, s, a);
                else launch(stream_attn_kernel<f16, 0>, grid, dim3(256), shm, s, a);
            } else {
                if (dk == 64) launch(stream_attn_kernel<float, 64>, grid, dim3(256), shm, s, a);
                else if (dk == 128) launch(stream_attn_kernel<float, 128>, grid, dim3(256), shm, s, a);
                else launch(stream_attn_kernel<float, 0>, grid, dim3(256), shm, s, a);
            }
            PKX_LAUNCH_CHECK();
            mark(KF_ATTENTION, false);
        }
        // C: x += conv(LN(x)) with the causal depthwise conv over [history ; chunk]
        if (fold) {
            gemm_resid_ln(L.wo, st.g, M, L.bo, st.x, 1.f, L.conv_ln_g, st.h, s, KF_GEMM_OUT);
            GemmParams p = fold_params(L.pw1, st.h, M, L.pw1_c1, L.pw1_c2, st.g, D);
            mark(KF_GEMM_PW1_GLU, true);
            launch_gemm(prec_, L.pw1.gtype, EPI_GLU, p, s);
            mark(KF_GEMM_PW1_GLU, false);
        } else {
            gemm(L.wo, EPI_RESID, st.g, D, M, L.bo, st.x, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_OUT);
            ln(L.conv_ln_g, L.conv_ln_b, st.h, nullptr);
            gemm(L.pw1, EPI_GLU, st.h, D, M, L.pw1_b, st.g, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_PW1_GLU);
        }
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
            if (c.conv_kernel == 9 && Tc <= SC_TCM) {
                // one stream per workgroup, one channel per thread up to 512
                // (every load of a channel in flight at once, 8 waves per CU)
                const uint32_t shk = (uint32_t)(SC_TCM * D) * 4u;
                if (prec_ == PREC_F16)
                    launch(stream_conv_kernel_k<f16, 9, SC_TCM>, dim3(B), dim3(512), shk, s, q);
                else
                    launch(stream_conv_kernel_k<float, 9, SC_TCM>, dim3(B), dim3(512), shk, s, q);
            } else if (prec_ == PREC_F16) {
                launch(stream_conv_kernel<f16>, dim3(B), dim3(256), shm, s, q);
            } else {
                launch(stream_conv_kernel<float>, dim3(B), dim3(256), shm, s, q);
            }
            PKX_LAUNCH_CHECK();
            mark(KF_DWCONV, false);
        }
        // D: x += 0.5 FFN2(LN(x)); x = norm_out(x) (+ the next layer's LN_ff1 into h)
        if (fold) {
            gemm_resid_ln(L.pw2, st.h, M, L.pw2_b, st.x, 1.f, L.ff2_ln_g, st.g, s, KF_GEMM_PW2);
            const GemmParams p = fold_params(L.ff2_w1, st.g, M, L.ff2_c1, L.ff2_c2, st.u, c.ff_dim);
            mark(KF_GEMM_FFN, true);
            launch_gemm(prec_, L.ff2_w1.gtype, EPI_SILU, p, s);
            mark(KF_GEMM_FFN, false);
        } else {
            gemm(L.pw2, EPI_RESID, st.h, D, M, L.pw2_b, st.x, D, 1.f, nullptr, 1, s, prec_, KF_GEMM_PW2);
            ln(L.ff2_ln_g, L.ff2_ln_b, st.h, nullptr);
            gemm(L.ff2_w1, EPI_SILU, st.h, D, M, L.ff2_b1, st.u, c.ff_dim, 1.f, nullptr, 1, s, prec_, KF_GEMM_FFN);
        }
        gemm(L.ff2_w2, EPI_RESID, st.u, c.ff_dim, M, L.ff2_b2, st.x, D, 0.5f, nullptr, 1, s, prec_, KF_GEMM_FFN);
        if (l + 1 < c.n_layers)
            ln(L.out_ln_g, L.out_ln_b, st.h, st.x, layers_[(size_t)l + 1].ff1_ln_g, layers_[(size_t)l + 1].ff1_ln_b);
        else
            ln(L.out_ln_g, L.out_ln_b, nullptr, st.x);
    }
    PKX_HIP(hipMemcpyAsync(out, st.x, (size_t)M * D * 4, hipMemcpyDeviceToDevice, s));
    st.clc = st.clc + Tc < st.CL ? st.clc + Tc : st.CL;   // streaming_encoder.cpp:447-448
    st.head = (st.head + Tc) % st.CL;
    st.step += 1;
    return is_last ? Tc : (c.stream_valid_out_len < Tc ? c.stream_valid_out_len : Tc);
}

}  // namespace pkx

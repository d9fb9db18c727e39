// MFMA GEMM family for gfx950 (see gemm.hpp for the reference ops it replaces).
//
// Block = 256 threads = 4 waves in a 2x2 grid; each wave owns TM x TN 16x16
// MFMA subtiles, so the block tile is (32*TM) x (32*TN).  The K loop is
// software pipelined: the next K slab is fetched from HBM into registers
// (and dequantised there) while MFMAs consume the current slab from LDS;
// one barrier per slab with double-buffered LDS.  Block ids are remapped so
// each XCD owns a contiguous run of output tiles (consecutive tiles share a
// weight column-block, so its dequantised slabs are served from that XCD's L2).
#include "gemm.hpp"

namespace pkx {

// ---------------------------------------------------------------------------
// XCD-aware tile order: hardware dispatches block b to XCD b % 8.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int xcd_tile(int bid, int total) {
    const int per = total / 8, rem = total % 8;
    const int x = bid % 8, loc = bid / 8;
    return x * per + (x < rem ? x : rem) + loc;
}

// ---------------------------------------------------------------------------
// Epilogue for one accumulator element (everything except GLU).
// ---------------------------------------------------------------------------
template <int EPI, typename ActT>
__device__ __forceinline__ void epi_one(const GemmParams& p, int m, int n, float acc) {
    float v = acc + (p.bias ? p.bias[n] : 0.0f);
    if constexpr (EPI == EPI_STORE) {
        ((ActT*)p.Y)[(int64_t)m * p.ldy + n] = to_act<ActT>(v * p.alpha);
    } else if constexpr (EPI == EPI_STORE_F32) {
        ((float*)p.Y)[(int64_t)m * p.ldy + n] = v * p.alpha;
    } else if constexpr (EPI == EPI_SILU) {
        ((ActT*)p.Y)[(int64_t)m * p.ldy + n] = to_act<ActT>(silu_dev(v));
    } else if constexpr (EPI == EPI_RESID) {
        float* r = (float*)p.Y + (int64_t)m * p.ldy + n;
        *r = *r + v * p.alpha;
    } else if constexpr (EPI == EPI_RELU) {
        ((ActT*)p.Y)[(int64_t)m * p.ldy + n] = to_act<ActT>(v > 0.f ? v : 0.f);
    } else if constexpr (EPI == EPI_RELU_TR) {
        // rows are pixels (b, t, f), f fastest; store [b][t][c][f] (channel-major flatten)
        const int F = p.trF;
        const int bt = m / F, f = m - bt * F;
        const int t = bt % p.T, b = bt / p.T;
        float o = v > 0.f ? v : 0.f;
        if (p.valid && t >= p.valid[b]) o = 0.f;
        ((ActT*)p.Y)[((int64_t)bt * p.N + n) * F + f] = to_act<ActT>(o);
    } else if constexpr (EPI == EPI_RELU2_F32) {
        float o = v + (p.bias2 ? p.bias2[n] : 0.0f);
        ((float*)p.Y)[(int64_t)m * p.ldy + n] = o > 0.f ? o : 0.f;
    }
}

template <int EPI, typename ActT, int TM, int TN>
__device__ __forceinline__ void epilogue(const GemmParams& p, float4v (&acc)[TM][TN], int mw,
                                         int nw, int lane) {
    const int lr = 4 * (lane >> 4), lc = lane & 15;
    if constexpr (EPI == EPI_GLU) {
        // Weight rows were interleaved in 16-row groups (a0..15, b0..15, a16..31, ...),
        // so subtile 2jj holds GLU inputs a and subtile 2jj+1 the matching gates b.
        const int half_n = p.N / 2;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int jj = 0; jj < TN / 2; ++jj)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = mw + 16 * i + lr + r;
                    const int na = nw + 32 * jj + lc;
                    const int og = nw / 2 + 16 * jj + lc;
                    if (m < p.M && og < half_n) {
                        const float a = acc[i][2 * jj][r] + (p.bias ? p.bias[na] : 0.f);
                        const float g = acc[i][2 * jj + 1][r] + (p.bias ? p.bias[na + 16] : 0.f);
                        float o = a * sigmoid_dev(g);
                        if (p.valid) {
                            const int b = m / p.T, t = m - b * p.T;
                            if (t >= p.valid[b]) o = 0.f;
                        }
                        ((ActT*)p.Y)[(int64_t)m * p.ldy + og] = to_act<ActT>(o);
                    }
                }
    } else {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = mw + 16 * i + lr + r;
                    const int n = nw + 16 * j + lc;
                    if (m < p.M && n < p.N) epi_one<EPI, ActT>(p, m, n, acc[i][j][r]);
                }
    }
}

// ===========================================================================
// f16 path: A f16, weights -> f16, v_mfma_f32_16x16x32_f16, BK = 64
// ===========================================================================
constexpr int BK16 = 64;
constexpr int LDK16 = BK16 + 8;  // +16 B row pad: 8 consecutive rows cover all banks

template <int BM> struct ALoad16 {
    static constexpr int NC = (BM * 8 + 255) / 256;  // 16-byte chunks per thread
    half8v r[NC];
    __device__ void load(const GemmParams& p, int m0, int k0, int tid) {
        const f16* A = (const f16*)p.A;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 3, col = (c & 7) * 8;
            const int m = m0 + row, k = k0 + col;
            half8v v = {};
            if (c < BM * 8 && m < p.M && k < p.K) v = *(const half8v*)(A + (int64_t)m * p.lda + k);
            r[i] = v;
        }
    }
    __device__ void store(f16* As, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c < BM * 8) *(half8v*)(As + (c >> 3) * LDK16 + (c & 7) * 8) = r[i];
        }
    }
};

template <int WT, int BN> struct BLoad16;

template <int BN> struct BLoad16<GT_F16, BN> {
    static constexpr int NC = (BN * 8 + 255) / 256;
    half8v r[NC];
    __device__ void load(const GemmParams& p, int n0, int k0, int tid) {
        const f16* W = (const f16*)p.Wq;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 3, col = (c & 7) * 8;
            const int n = n0 + row, k = k0 + col;
            half8v v = {};
            if (c < BN * 8 && n < p.N && k < p.K) v = *(const half8v*)(W + (int64_t)n * p.K + k);
            r[i] = v;
        }
    }
    __device__ void store(f16* Bs, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c < BN * 8) *(half8v*)(Bs + (c >> 3) * LDK16 + (c & 7) * 8) = r[i];
        }
    }
};

// q8_0 device layout: int8 q[N][K] and f16 d[N][K/32]; w = d*q.
template <int BN> struct BLoad16<GT_Q8_0, BN> {
    static constexpr int NC = (BN * 4 + 255) / 256;
    int4v q[NC];
    f16 d[NC];
    __device__ void load(const GemmParams& p, int n0, int k0, int tid) {
        const int8_t* W = (const int8_t*)p.Wq;
        const f16* S = (const f16*)p.Ws;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 2, col = (c & 3) * 16;
            const int n = n0 + row, k = k0 + col;
            int4v v = {};
            f16 s = (f16)0.f;
            if (c < BN * 4 && n < p.N && k < p.K) {
                v = *(const int4v*)(W + (int64_t)n * p.K + k);
                s = S[(int64_t)n * (p.K / 32) + k / 32];
            }
            q[i] = v;
            d[i] = s;
        }
    }
    __device__ void store(f16* Bs, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c >= BN * 4) continue;
            f16* dst = Bs + (c >> 2) * LDK16 + (c & 3) * 16;
            half8v lo, hi;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                lo[b] = (f16)(float)(int8_t)(q[i][b >> 2] >> ((b & 3) * 8)) * d[i];
                hi[b] = (f16)(float)(int8_t)(q[i][2 + (b >> 2)] >> ((b & 3) * 8)) * d[i];
            }
            *(half8v*)dst = lo;
            *(half8v*)(dst + 8) = hi;
        }
    }
};

// q4_K device layout: nibbles u8 qs[N][K/2] in ggml order (per 64 elements, byte l
// holds element l in the low and element 32+l in the high nibble) and float2
// {d*sc, dmin*m}[N][K/32]; w = s.x*q - s.y.
template <int BN> struct BLoad16<GT_Q4_K, BN> {
    static constexpr int NC = (BN * 2 + 255) / 256;
    int4v q[NC];
    float2v s0[NC], s1[NC];
    __device__ void load(const GemmParams& p, int n0, int k0, int tid) {
        const uint8_t* W = (const uint8_t*)p.Wq;
        const float2v* S = (const float2v*)p.Ws;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 1, h = c & 1;
            const int n = n0 + row;
            int4v v = {};
            float2v a = {0.f, 0.f}, b = {0.f, 0.f};
            if (c < BN * 2 && n < p.N && k0 < p.K) {
                v = *(const int4v*)(W + (int64_t)n * (p.K / 2) + k0 / 2 + 16 * h);
                a = S[(int64_t)n * (p.K / 32) + k0 / 32];
                b = S[(int64_t)n * (p.K / 32) + k0 / 32 + 1];
            }
            q[i] = v;
            s0[i] = a;
            s1[i] = b;
        }
    }
    __device__ void store(f16* Bs, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c >= BN * 2) continue;
            const int h = c & 1;
            f16* dst = Bs + (c >> 1) * LDK16 + 16 * h;
            half8v l0, l1, h0, h1;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const uint32_t w0 = (uint32_t)q[i][b >> 2] >> ((b & 3) * 8);
                const uint32_t w1 = (uint32_t)q[i][2 + (b >> 2)] >> ((b & 3) * 8);
                l0[b] = (f16)(s0[i].x * (float)(w0 & 0xF) - s0[i].y);
                l1[b] = (f16)(s0[i].x * (float)(w1 & 0xF) - s0[i].y);
                h0[b] = (f16)(s1[i].x * (float)((w0 >> 4) & 0xF) - s1[i].y);
                h1[b] = (f16)(s1[i].x * (float)((w1 >> 4) & 0xF) - s1[i].y);
            }
            *(half8v*)dst = l0;
            *(half8v*)(dst + 8) = l1;
            *(half8v*)(dst + 32) = h0;
            *(half8v*)(dst + 40) = h1;
        }
    }
};

template <int TM, int TN, int WT, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_f16_kernel(GemmParams p) {
    constexpr int BM = 32 * TM, BN = 32 * TN;
    __shared__ __attribute__((aligned(16))) f16 As[2][BM * LDK16];
    __shared__ __attribute__((aligned(16))) f16 Bs[2][BN * LDK16];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int nbm = cdiv_dev(p.M, BM), nbn = cdiv_dev(p.N, BN);
    const int tile = xcd_tile(blockIdx.x, nbm * nbn);
    const int bm = tile % nbm, bn = tile / nbm;
    const int m0 = bm * BM, n0 = bn * BN;

    float4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = (float4v){0.f, 0.f, 0.f, 0.f};

    ALoad16<BM> al;
    BLoad16<WT, BN> bl;
    const int nk = cdiv_dev(p.K, BK16);
    al.load(p, m0, 0, tid);
    bl.load(p, n0, 0, tid);
    al.store(As[0], tid);
    bl.store(Bs[0], tid);
    __syncthreads();

    const int arow = wm * TM * 16 + (lane & 15), brow = wn * TN * 16 + (lane & 15);
    const int kq = (lane >> 4) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
            al.load(p, m0, (kt + 1) * BK16, tid);
            bl.load(p, n0, (kt + 1) * BK16, tid);
        }
        const f16* as = As[cur];
        const f16* bs = Bs[cur];
#pragma unroll
        for (int ks = 0; ks < BK16; ks += 32) {
            half8v af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = *(const half8v*)(as + (arow + 16 * i) * LDK16 + ks + kq);
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = *(const half8v*)(bs + (brow + 16 * j) * LDK16 + ks + kq);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) {
            al.store(As[cur ^ 1], tid);
            bl.store(Bs[cur ^ 1], tid);
        }
        __syncthreads();
    }
    epilogue<EPI, f16, TM, TN>(p, acc, m0 + wm * TM * 16, n0 + wn * TN * 16, lane);
}

// ===========================================================================
// f32 path: A f32, weights -> f32, v_mfma_f32_16x16x4_f32, BK = 32
// ===========================================================================
constexpr int BK32 = 32;
constexpr int LDK32 = BK32 + 4;

template <int BM> struct ALoad32 {
    static constexpr int NC = (BM * 8 + 255) / 256;  // 4-float chunks
    float4v r[NC];
    __device__ void load(const GemmParams& p, int m0, int k0, int tid) {
        const float* A = (const float*)p.A;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 3, col = (c & 7) * 4;
            const int m = m0 + row, k = k0 + col;
            float4v v = {0.f, 0.f, 0.f, 0.f};
            if (c < BM * 8 && m < p.M && k < p.K) v = *(const float4v*)(A + (int64_t)m * p.lda + k);
            r[i] = v;
        }
    }
    __device__ void store(float* As, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c < BM * 8) *(float4v*)(As + (c >> 3) * LDK32 + (c & 7) * 4) = r[i];
        }
    }
};

template <int WT, int BN> struct BLoad32;

template <int BN> struct BLoad32<GT_F32, BN> {
    static constexpr int NC = (BN * 8 + 255) / 256;
    float4v r[NC];
    __device__ void load(const GemmParams& p, int n0, int k0, int tid) {
        const float* W = (const float*)p.Wq;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 3, col = (c & 7) * 4;
            const int n = n0 + row, k = k0 + col;
            float4v v = {0.f, 0.f, 0.f, 0.f};
            if (c < BN * 8 && n < p.N && k < p.K) v = *(const float4v*)(W + (int64_t)n * p.K + k);
            r[i] = v;
        }
    }
    __device__ void store(float* Bs, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c < BN * 8) *(float4v*)(Bs + (c >> 3) * LDK32 + (c & 7) * 4) = r[i];
        }
    }
};

template <int BN> struct BLoad32<GT_F16, BN> {
    static constexpr int NC = (BN * 4 + 255) / 256;  // 8-half chunks
    half8v r[NC];
    __device__ void load(const GemmParams& p, int n0, int k0, int tid) {
        const f16* W = (const f16*)p.Wq;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 2, col = (c & 3) * 8;
            const int n = n0 + row, k = k0 + col;
            half8v v = {};
            if (c < BN * 4 && n < p.N && k < p.K) v = *(const half8v*)(W + (int64_t)n * p.K + k);
            r[i] = v;
        }
    }
    __device__ void store(float* Bs, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c >= BN * 4) continue;
            float* dst = Bs + (c >> 2) * LDK32 + (c & 3) * 8;
            float4v a, b;
#pragma unroll
            for (int e = 0; e < 4; ++e) { a[e] = (float)r[i][e]; b[e] = (float)r[i][4 + e]; }
            *(float4v*)dst = a;
            *(float4v*)(dst + 4) = b;
        }
    }
};

template <int BN> struct BLoad32<GT_Q8_0, BN> {
    static constexpr int NC = (BN * 2 + 255) / 256;  // one 32-block per row per slab: 2 x 16 B
    int4v q[NC];
    float d[NC];
    __device__ void load(const GemmParams& p, int n0, int k0, int tid) {
        const int8_t* W = (const int8_t*)p.Wq;
        const f16* S = (const f16*)p.Ws;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 1, h = c & 1;
            const int n = n0 + row;
            int4v v = {};
            float s = 0.f;
            if (c < BN * 2 && n < p.N && k0 < p.K) {
                v = *(const int4v*)(W + (int64_t)n * p.K + k0 + 16 * h);
                s = (float)S[(int64_t)n * (p.K / 32) + k0 / 32];
            }
            q[i] = v;
            d[i] = s;
        }
    }
    __device__ void store(float* Bs, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c >= BN * 2) continue;
            float* dst = Bs + (c >> 1) * LDK32 + 16 * (c & 1);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                float4v o;
#pragma unroll
                for (int b = 0; b < 4; ++b) o[b] = (float)(int8_t)(q[i][w] >> (8 * b)) * d[i];
                *(float4v*)(dst + 4 * w) = o;
            }
        }
    }
};

template <int BN> struct BLoad32<GT_Q4_K, BN> {
    static constexpr int NC = (BN * 2 + 255) / 256;
    int4v q[NC];
    float2v s[NC];
    int shift;
    __device__ void load(const GemmParams& p, int n0, int k0, int tid) {
        const uint8_t* W = (const uint8_t*)p.Wq;
        const float2v* S = (const float2v*)p.Ws;
        // 32-element sub-block k0: low nibbles of bytes [k0/2, +32) if k0 % 64 == 0,
        // else high nibbles of bytes [(k0-32)/2, +32).
        const int hi = (k0 & 32) ? 1 : 0;
        shift = hi * 4;
        const int byte0 = (k0 - 32 * hi) / 2;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 1, h = c & 1;
            const int n = n0 + row;
            int4v v = {};
            float2v sc = {0.f, 0.f};
            if (c < BN * 2 && n < p.N && k0 < p.K) {
                v = *(const int4v*)(W + (int64_t)n * (p.K / 2) + byte0 + 16 * h);
                sc = S[(int64_t)n * (p.K / 32) + k0 / 32];
            }
            q[i] = v;
            s[i] = sc;
        }
    }
    __device__ void store(float* Bs, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c >= BN * 2) continue;
            float* dst = Bs + (c >> 1) * LDK32 + 16 * (c & 1);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                float4v o;
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    o[b] = s[i].x * (float)(((uint32_t)q[i][w] >> (8 * b + shift)) & 0xF) - s[i].y;
                *(float4v*)(dst + 4 * w) = o;
            }
        }
    }
};

template <int TM, int TN, int WT, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(GemmParams p) {
    constexpr int BM = 32 * TM, BN = 32 * TN;
    __shared__ __attribute__((aligned(16))) float As[2][BM * LDK32];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN * LDK32];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int nbm = cdiv_dev(p.M, BM), nbn = cdiv_dev(p.N, BN);
    const int tile = xcd_tile(blockIdx.x, nbm * nbn);
    const int bm = tile % nbm, bn = tile / nbm;
    const int m0 = bm * BM, n0 = bn * BN;

    float4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = (float4v){0.f, 0.f, 0.f, 0.f};

    ALoad32<BM> al;
    BLoad32<WT, BN> bl;
    const int nk = cdiv_dev(p.K, BK32);
    al.load(p, m0, 0, tid);
    bl.load(p, n0, 0, tid);
    al.store(As[0], tid);
    bl.store(Bs[0], tid);
    __syncthreads();

    // Lane l covers k = 4*(l/16) .. +3 of each 16-wide K chunk (same permutation
    // for A and B, so the contraction is unchanged).
    const int arow = wm * TM * 16 + (lane & 15), brow = wn * TN * 16 + (lane & 15);
    const int kq = (lane >> 4) * 4;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
            al.load(p, m0, (kt + 1) * BK32, tid);
            bl.load(p, n0, (kt + 1) * BK32, tid);
        }
        const float* as = As[cur];
        const float* bs = Bs[cur];
#pragma unroll
        for (int ks = 0; ks < BK32; ks += 16) {
            float4v af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = *(const float4v*)(as + (arow + 16 * i) * LDK32 + ks + kq);
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = *(const float4v*)(bs + (brow + 16 * j) * LDK32 + ks + kq);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][e], bf[j][e], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) {
            al.store(As[cur ^ 1], tid);
            bl.store(Bs[cur ^ 1], tid);
        }
        __syncthreads();
    }
    epilogue<EPI, float, TM, TN>(p, acc, m0 + wm * TM * 16, n0 + wn * TN * 16, lane);
}

// ===========================================================================
// Dispatch
// ===========================================================================
template <int TM, int TN, int WT, int EPI>
static void run_f16(const GemmParams& p, hipStream_t s) {
    const int tiles = cdiv(p.M, 32 * TM) * cdiv(p.N, 32 * TN);
    hipLaunchKernelGGL((gemm_f16_kernel<TM, TN, WT, EPI>), dim3(tiles), dim3(256), 0, s, p);
    PKX_LAUNCH_CHECK();
}
template <int TM, int TN, int WT, int EPI>
static void run_f32(const GemmParams& p, hipStream_t s) {
    const int tiles = cdiv(p.M, 32 * TM) * cdiv(p.N, 32 * TN);
    hipLaunchKernelGGL((gemm_f32_kernel<TM, TN, WT, EPI>), dim3(tiles), dim3(256), 0, s, p);
    PKX_LAUNCH_CHECK();
}

#define PKX_EPI_SWITCH(RUN, TM, TN, WT)                                         \
    switch (epi) {                                                              \
    case EPI_STORE: RUN<TM, TN, WT, EPI_STORE>(p, s); break;                    \
    case EPI_STORE_F32: RUN<TM, TN, WT, EPI_STORE_F32>(p, s); break;            \
    case EPI_SILU: RUN<TM, TN, WT, EPI_SILU>(p, s); break;                      \
    case EPI_RESID: RUN<TM, TN, WT, EPI_RESID>(p, s); break;                    \
    case EPI_GLU: RUN<TM, TN, WT, EPI_GLU>(p, s); break;                        \
    case EPI_RELU: RUN<TM, TN, WT, EPI_RELU>(p, s); break;                      \
    case EPI_RELU_TR: RUN<TM, TN, WT, EPI_RELU_TR>(p, s); break;                \
    case EPI_RELU2_F32: RUN<TM, TN, WT, EPI_RELU2_F32>(p, s); break;            \
    default: throw std::invalid_argument("gemm: bad epilogue");                 \
    }

template <int TM, int TN, int WT>
static void f16_epi(int epi, const GemmParams& p, hipStream_t s) { PKX_EPI_SWITCH(run_f16, TM, TN, WT) }
template <int TM, int TN, int WT>
static void f32_epi(int epi, const GemmParams& p, hipStream_t s) { PKX_EPI_SWITCH(run_f32, TM, TN, WT) }

void launch_gemm(Precision prec, int wtype, int epi, const GemmParams& p, hipStream_t s) {
    require(p.M > 0 && p.N > 0 && p.K > 0, "gemm: empty shape");
    require(p.K % 8 == 0, "gemm: K must be a multiple of 8");
    require(p.lda >= p.K && p.lda % 8 == 0, "gemm: lda must be >= K and a multiple of 8 (16-byte rows)");
    if (wtype == GT_Q8_0) require(p.K % 32 == 0, "gemm: q8_0 needs K % 32 == 0");
    if (wtype == GT_Q4_K) require(p.K % 256 == 0, "gemm: q4_K needs K % 256 == 0");
    if (epi == EPI_GLU) require(p.N % 32 == 0, "gemm: GLU needs N % 32 == 0");
    // Tile choice: 128x128 when that already gives >= 256 tiles, else 64x128.
    const bool big = (int64_t)cdiv(p.M, 128) * cdiv(p.N, 128) >= 256;
    if (prec == PREC_F16) {
        switch (wtype) {
        case GT_F16: big ? f16_epi<4, 4, GT_F16>(epi, p, s) : f16_epi<2, 4, GT_F16>(epi, p, s); break;
        case GT_Q8_0: big ? f16_epi<4, 4, GT_Q8_0>(epi, p, s) : f16_epi<2, 4, GT_Q8_0>(epi, p, s); break;
        case GT_Q4_K: big ? f16_epi<4, 4, GT_Q4_K>(epi, p, s) : f16_epi<2, 4, GT_Q4_K>(epi, p, s); break;
        default: throw std::invalid_argument("gemm(f16): weight type must be f16/q8_0/q4_K");
        }
    } else {
        switch (wtype) {
        case GT_F32: f32_epi<2, 4, GT_F32>(epi, p, s); break;
        case GT_F16: f32_epi<2, 4, GT_F16>(epi, p, s); break;
        case GT_Q8_0: f32_epi<2, 4, GT_Q8_0>(epi, p, s); break;
        case GT_Q4_K: f32_epi<2, 4, GT_Q4_K>(epi, p, s); break;
        default: throw std::invalid_argument("gemm(f32): unknown weight type");
        }
    }
}

// ===========================================================================
// Bit-exact dequantisation of raw ggml blocks (for the weight-format checks)
// ===========================================================================
__global__ void dequant_q8_0_kernel(const uint8_t* src, float* dst, int64_t nblk) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // one element
    if (i >= nblk * 32) return;
    const uint8_t* b = src + (i / 32) * 34;
    const f16 d = __builtin_bit_cast(f16, (uint16_t)(b[0] | (b[1] << 8)));
    dst[i] = (float)(int8_t)b[2 + (i % 32)] * (float)d;
}

__global__ void dequant_q4_k_kernel(const uint8_t* src, float* dst, int64_t nblk) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk * 256) return;
    const uint8_t* b = src + (i / 256) * 144;
    const int e = (int)(i % 256), chunk = e / 64, within = e % 64, j = 2 * chunk + (within >= 32);
    const float d = (float)__builtin_bit_cast(f16, (uint16_t)(b[0] | (b[1] << 8)));
    const float dmin = (float)__builtin_bit_cast(f16, (uint16_t)(b[2] | (b[3] << 8)));
    const uint8_t* sc = b + 4;
    int s, m;
    if (j < 4) {
        s = sc[j] & 63;
        m = sc[j + 4] & 63;
    } else {
        s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
        m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
    const uint8_t byte = b[16 + 32 * chunk + (within & 31)];
    const int qv = within < 32 ? (byte & 0xF) : (byte >> 4);
    const float d1 = d * (float)s, m1 = dmin * (float)m;
    dst[i] = __fsub_rn(__fmul_rn(d1, (float)qv), m1);
}

__global__ void dequant_f16_kernel(const f16* src, float* dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = (float)src[i];
}

void launch_dequantize(int wtype, const void* src, float* dst, int64_t n, hipStream_t s) {
    const int bs = 256;
    if (wtype == GT_Q8_0) {
        require(n % 32 == 0, "dequantize: q8_0 needs n % 32 == 0");
        hipLaunchKernelGGL(dequant_q8_0_kernel, dim3(cdiv(n, bs)), dim3(bs), 0, s, (const uint8_t*)src, dst, n / 32);
    } else if (wtype == GT_Q4_K) {
        require(n % 256 == 0, "dequantize: q4_K needs n % 256 == 0");
        hipLaunchKernelGGL(dequant_q4_k_kernel, dim3(cdiv(n, bs)), dim3(bs), 0, s, (const uint8_t*)src, dst, n / 256);
    } else if (wtype == GT_F16) {
        hipLaunchKernelGGL(dequant_f16_kernel, dim3(cdiv(n, bs)), dim3(bs), 0, s, (const f16*)src, dst, n);
    } else {
        throw std::invalid_argument("dequantize: unsupported type");
    }
    PKX_LAUNCH_CHECK();
}

}  // namespace pkx

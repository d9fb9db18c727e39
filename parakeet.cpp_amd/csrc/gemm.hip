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


// Rows of each 64-wide K slab block of a slab-major (q8_0 / q4_K) weight (views
// into a larger allocation keep the allocation's row count).
__device__ __forceinline__ int slab_rows(const GemmParams& p) { return p.ldw > 0 ? p.ldw : p.N; }

// The arguments every GEMM prologue reads, pulled into SGPRs in one batch of
// scalar loads at kernel entry.  Left to itself the compiler loads the
// pointers the prologue uses later (residual stream, bias) only after the
// first batch has returned: a second serialized argument fetch of ~1k cycles
// before the first DMA is issued.
__device__ __forceinline__ void prefetch_gemm_args(const GemmParams& p) {
    asm volatile("" ::"s"(p.M), "s"(p.N), "s"(p.K), "s"(p.xcd_gm), "s"(p.ldw), "s"(p.A), "s"(p.lda), "s"(p.Wq),
                 "s"(p.Ws), "s"(p.Y), "s"(p.ldy), "s"(p.bias));
}

// Wave index as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_id_uniform() { return __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6); }

// 2-D XCD blocking: the nbm x nbn tile grid is cut into gm row bands x gn
// column bands (gm * gn = 8), one rectangle per XCD, so an XCD's L2 sees only
// its band of A rows and its band of weight columns (gn*|A| + gm*|W| bytes
// over the chip instead of 8*|A| or 8*|W|).  xcd_tile gives each XCD a
// contiguous range of positions; positions enumerate the rectangles in order,
// each rectangle M-fastest, so the map is a bijection for any grid size.
// gm and gn are powers of two, so the band edges i * nbm / gm are shifts; the
// one division left is the split of k inside its rectangle.  (With a division
// for every band edge this ran ~3k cycles at the start of every launch, all
// of it before the first load: 32-bit division by a runtime value is a
// ~40-instruction scalar / vector round trip on this hardware.)
__device__ __forceinline__ void xcd_rect(int k, int nbm, int nbn, int gm, int& bm, int& bn) {
    const int lgm = __builtin_ctz(gm), lgn = 3 - lgm;
    for (int i = 0; i < gm; ++i) {
        const int r0 = (i * nbm) >> lgm, r1 = ((i + 1) * nbm) >> lgm;
        for (int j = 0; j < (1 << lgn); ++j) {
            const int c0 = (j * nbn) >> lgn, c1 = ((j + 1) * nbn) >> lgn;
            const int h = r1 - r0, sz = h * (c1 - c0);
            if (k < sz) {   // sz > 0, so h > 0
                const int q = (int)((unsigned)k / (unsigned)h);
                bm = r0 + (k - q * h);
                bn = c0 + q;
                return;
            }
            k -= sz;
        }
    }
    bm = bn = 0;   // unreachable: the rectangles cover the grid
}
__device__ __forceinline__ void xcd_tile_2d(int bid, int nbm, int nbn, int gm, int& bm, int& bn) {
    xcd_rect(xcd_tile(bid, nbm * nbn), nbm, nbn, gm, bm, bn);
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
        // pointwise_conv1 rows are interleaved in 32-row groups (a0..31, b0..31, ...):
        // in each 64-column group, subtiles 0-1 hold GLU inputs a, subtiles 2-3 the gates b.
        static_assert(TN % 4 == 0, "GLU needs 64-column wave tiles");
        const int half_n = p.N / 2;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int jj = 0; jj < TN / 4; ++jj)
#pragma unroll
                for (int jh = 0; jh < 2; ++jh)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int ja = 4 * jj + jh;
                        const int m = mw + 16 * i + lr + r;
                        const int na = nw + 16 * ja + lc;
                        const int og = nw / 2 + 32 * jj + 16 * jh + lc;
                        if (m < p.M && og < half_n) {
                            const float a = acc[i][ja][r] + (p.bias ? p.bias[na] : 0.f);
                            const float g = acc[i][ja + 2][r] + (p.bias ? p.bias[na + 32] : 0.f);
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
//
// All global reads are raw buffer loads: rows past M / N and columns past K
// (offsets pushed beyond the buffer's num_records) return zero in hardware, so
// the loop has no branches.  Raw loads stay in registers two K slabs ahead of
// the MFMAs; they are dequantised only when written to LDS.
// ===========================================================================
constexpr int BK16 = 64;
constexpr int LDK16 = BK16 + 8;   // +16 B row pad: 8 consecutive rows cover all banks
__device__ __forceinline__ int4v bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}

template <int BM> struct ALoad16 {
    static constexpr int NC = (BM * 8 + 255) / 256;  // 16-byte chunks per thread
    int4v r[NC];
    __device__ void load(__amdgpu_buffer_rsrc_t rs, const GemmParams& p, int m0, int k0, int tid) {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int m = m0 + (c >> 3), k = k0 + (c & 7) * 8;
            const uint32_t off = (k < p.K && m < p.M) ? (uint32_t)(((int64_t)m * p.lda + k) * 2) : OOB;
            r[i] = bload16(rs, off);
        }
    }
    __device__ void store(f16* As, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c < BM * 8) *(int4v*)(As + (c >> 3) * LDK16 + (c & 7) * 8) = r[i];
        }
    }
};

template <int WT, int BN> struct BLoad16;

template <int BN> struct BLoad16<GT_F16, BN> {
    static constexpr int NC = (BN * 8 + 255) / 256;
    int4v r[NC];
    __device__ void load(__amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t, const GemmParams& p, int n0,
                         int k0, int tid) {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int n = n0 + (c >> 3), k = k0 + (c & 7) * 8;
            const uint32_t off = (k < p.K && n < p.N) ? (uint32_t)(((int64_t)n * p.K + k) * 2) : OOB;
            r[i] = bload16(rq, off);
        }
    }
    __device__ void store(f16* Bs, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c < BN * 8) *(int4v*)(Bs + (c >> 3) * LDK16 + (c & 7) * 8) = r[i];
        }
    }
};

// Exact int8 -> f16 for 4 packed bytes: byte b (two's complement) becomes the
// f16 with bit pattern 0x6400 | (b ^ 0x80) = 1024 + (b + 128); subtracting
// 1152 leaves b exactly.  Then one correctly rounded f16 multiply by d.
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, half2v d2, half2v& lo, half2v& hi) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x07010700u) ;  // [0x64,b1,0x64,b0]
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x07030702u);   // [0x64,b3,0x64,b2]
    const half2v bias = {(f16)1152.0f, (f16)1152.0f};
    lo = (__builtin_bit_cast(half2v, a) - bias) * d2;
    hi = (__builtin_bit_cast(half2v, b) - bias) * d2;
}

// Four 4-bit weights (nibble `hi` of each byte of w) to f16, w = s*q - m with
// nm2 = -m: the nibble is placed in an f16 mantissa so that the half reads
// 1024 + q (low nibble, exponent byte 0x64) or 64 + q (high nibble in mantissa
// bits 4..7, exponent byte 0x54); subtracting 1024 or 64 is exact, then one
// rounding in the fma.
__device__ __forceinline__ void nib4_to_f16(uint32_t w, int hi, half2v s2, half2v nm2, half2v& lo, half2v& up) {
    const uint32_t e = hi ? 0x54545454u : 0x64646464u;
    const uint32_t mask = hi ? 0xFFF0FFF0u : 0xFF0FFF0Fu;
    const f16 off = hi ? (f16)64.0f : (f16)1024.0f;
    const half2v off2 = {off, off};
    const uint32_t a = __builtin_amdgcn_perm(e, w, 0x07010700u) & mask;  // bytes 0, 1
    const uint32_t b = __builtin_amdgcn_perm(e, w, 0x07030702u) & mask;  // bytes 2, 3
    lo = (__builtin_bit_cast(half2v, a) - off2) * s2 + nm2;
    up = (__builtin_bit_cast(half2v, b) - off2) * s2 + nm2;
}

// q8_0 device layout (slab-major): int8 q[K/64][ldw][64] and f16 d[K/64][ldw][2]; w = d*q.
template <int BN> struct BLoad16<GT_Q8_0, BN> {
    static constexpr int NC = (BN * 4 + 255) / 256;
    int4v q[NC];
    uint32_t d[NC];
    __device__ void load(__amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rs, const GemmParams& p, int n0,
                         int k0, int tid) {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int n = n0 + (c >> 2), k = k0 + (c & 3) * 16;
            const bool in = k < p.K && n < p.N;
            const int L = slab_rows(p);   // slab-major: (slab, row) blocks of 64 bytes / 2 scales
            q[i] = bload16(rq, in ? (uint32_t)(((int64_t)(k / 64) * L + n) * 64 + (k & 63)) : OOB);
            d[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(
                rs, (int)(in ? (uint32_t)((((int64_t)(k / 64) * L + n) * 2 + ((k & 63) >> 5)) * 2) : OOB), 0, 0);
        }
    }
    __device__ void store(f16* Bs, int tid) const {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            if (c >= BN * 4) continue;
            f16* dst = Bs + (c >> 2) * LDK16 + (c & 3) * 16;
            const f16 dh = __builtin_bit_cast(f16, (uint16_t)d[i]);
            const half2v d2 = {dh, dh};
            half2v h[8];
#pragma unroll
            for (int w = 0; w < 4; ++w) i8x4_to_f16((uint32_t)q[i][w], d2, h[2 * w], h[2 * w + 1]);
            int4v lo, hi;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                lo[w] = __builtin_bit_cast(int, h[w]);
                hi[w] = __builtin_bit_cast(int, h[4 + w]);
            }
            *(int4v*)dst = lo;
            *(int4v*)(dst + 8) = hi;
        }
    }
};

// q4_K device layout (slab-major): nibbles u8 qs[K/64][ldw][32] in ggml order
// (per 64 elements, byte l holds element l in the low and element 32+l in the
// high nibble) and float2 {d*sc, dmin*m}[K/64][ldw][2]; w = s.x*q - s.y.
template <int BN> struct BLoad16<GT_Q4_K, BN> {
    static constexpr int NC = (BN * 2 + 255) / 256;
    int4v q[NC];
    float4v s[NC];   // {sc0, min0, sc1, min1}
    __device__ void load(__amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rs, const GemmParams& p, int n0,
                         int k0, int tid) {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int n = n0 + (c >> 1), h = c & 1;
            const bool in = k0 < p.K && n < p.N;
            const int64_t blk = (int64_t)(k0 / 64) * slab_rows(p) + n;   // slab-major
            q[i] = bload16(rq, in ? (uint32_t)(blk * 32 + 16 * h) : OOB);
            s[i] = __builtin_bit_cast(float4v, bload16(rs, in ? (uint32_t)(blk * 16) : OOB));
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
                l0[b] = (f16)(s[i][0] * (float)(w0 & 0xF) - s[i][1]);
                l1[b] = (f16)(s[i][0] * (float)(w1 & 0xF) - s[i][1]);
                h0[b] = (f16)(s[i][2] * (float)((w0 >> 4) & 0xF) - s[i][3]);
                h1[b] = (f16)(s[i][2] * (float)((w1 >> 4) & 0xF) - s[i][3]);
            }
            *(half8v*)dst = l0;
            *(half8v*)(dst + 8) = l1;
            *(half8v*)(dst + 32) = h0;
            *(half8v*)(dst + 40) = h1;
        }
    }
};

template <int TM, int TN>
__device__ __forceinline__ void mma_slab(const f16* as, const f16* bs, float4v (&acc)[TM][TN], int arow,
                                         int brow, int kq) {
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
}

// PF = register stages in flight (1: the next slab is fetched while the
// current one is consumed; 2: two slabs ahead, for tiles with spare VGPRs).
template <int TM, int TN, int WT, int EPI, int PF>
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

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, ((int64_t)(p.M - 1) * p.lda + p.K) * 2);
    int64_t wq_bytes = (int64_t)p.N * p.K * 2, ws_bytes = 0;
    if constexpr (WT == GT_Q8_0) {
        const int64_t blocks = (int64_t)(p.K / 64 - 1) * slab_rows(p) + p.N;   // (slab, row) blocks reachable
        wq_bytes = blocks * 64;
        ws_bytes = blocks * 4;
    }
    if constexpr (WT == GT_Q4_K) {
        const int64_t blocks = (int64_t)(p.K / 64 - 1) * slab_rows(p) + p.N;
        wq_bytes = blocks * 32;
        ws_bytes = blocks * 16;
    }
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.Wq, wq_bytes);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(WT == GT_F16 ? p.Wq : p.Ws, WT == GT_F16 ? wq_bytes : ws_bytes);

    float4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = (float4v){0.f, 0.f, 0.f, 0.f};

    const int arow = wm * TM * 16 + (lane & 15), brow = wn * TN * 16 + (lane & 15);
    const int kq = (lane >> 4) * 8;
    const int nk = cdiv_dev(p.K, BK16);

    if constexpr (PF == 1) {
        ALoad16<BM> al;
        BLoad16<WT, BN> bl;
        al.load(ra, p, m0, 0, tid);
        bl.load(rq, rs, p, n0, 0, tid);
        al.store(As[0], tid);
        bl.store(Bs[0], tid);
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) {
            const int cur = kt & 1;
            if (kt + 1 < nk) {
                al.load(ra, p, m0, (kt + 1) * BK16, tid);
                bl.load(rq, rs, p, n0, (kt + 1) * BK16, tid);
            }
            mma_slab<TM, TN>(As[cur], Bs[cur], acc, arow, brow, kq);
            if (kt + 1 < nk) {
                al.store(As[cur ^ 1], tid);
                bl.store(Bs[cur ^ 1], tid);
            }
            __syncthreads();
        }
    } else {
        // two register stages in flight: slab s lives in stage s & 1
        ALoad16<BM> a0, a1;
        BLoad16<WT, BN> b0, b1;
        a0.load(ra, p, m0, 0, tid);
        b0.load(rq, rs, p, n0, 0, tid);
        if (nk > 1) {
            a1.load(ra, p, m0, BK16, tid);
            b1.load(rq, rs, p, n0, BK16, tid);
        }
        a0.store(As[0], tid);
        b0.store(Bs[0], tid);
        if (nk > 2) {
            a0.load(ra, p, m0, 2 * BK16, tid);
            b0.load(rq, rs, p, n0, 2 * BK16, tid);
        }
        __syncthreads();
        for (int kt = 0; kt < nk; kt += 2) {
            // phase 0: MFMAs on slab kt (LDS 0); slab kt+1 (stage 1) -> LDS 1; fetch slab kt+3
            mma_slab<TM, TN>(As[0], Bs[0], acc, arow, brow, kq);
            if (kt + 1 < nk) {
                a1.store(As[1], tid);
                b1.store(Bs[1], tid);
                if (kt + 3 < nk) {
                    a1.load(ra, p, m0, (kt + 3) * BK16, tid);
                    b1.load(rq, rs, p, n0, (kt + 3) * BK16, tid);
                }
            }
            __syncthreads();
            if (kt + 1 >= nk) break;
            // phase 1: MFMAs on slab kt+1 (LDS 1); slab kt+2 (stage 0) -> LDS 0; fetch slab kt+4
            mma_slab<TM, TN>(As[1], Bs[1], acc, arow, brow, kq);
            if (kt + 2 < nk) {
                a0.store(As[0], tid);
                b0.store(Bs[0], tid);
                if (kt + 4 < nk) {
                    a0.load(ra, p, m0, (kt + 4) * BK16, tid);
                    b0.load(rq, rs, p, n0, (kt + 4) * BK16, tid);
                }
            }
            __syncthreads();
        }
    }
    epilogue<EPI, f16, TM, TN>(p, acc, m0 + wm * TM * 16, n0 + wn * TN * 16, lane);
}

// ===========================================================================
// f16 path, LDS-DMA + 32x32x16 MFMA (K % 64 == 0; f16 or q8_0 weights).
//
// v_mfma_f32_32x32x16_f16 needs half the operand bytes per FLOP of the
// 16x16x32 form (each 16-byte A or B fragment feeds 32 columns or rows), which
// matters because LDS bandwidth, not the matrix core, bounds this kernel: 4
// waves in a 2x2 grid, each wave a (32*TM) x (32*TN) tile of 32x32 blocks.
//
// global_load_lds_dwordx4 moves 16 B per lane straight into LDS (lane L lands
// at base + 16 L), so a 3-stage LDS ring is kept full with no staging
// registers: slab kt+2 is in flight while slab kt is multiplied.  Tiles are
// stored with XOR-swizzled 16 B chunks (the swizzle is applied through each
// lane's source address).  A 16-byte LDS read is served 16 lanes at a time
// over 64 banks (256 B): with 128-byte rows two rows share a bank row, so the
// chunk is XORed with (row >> 1) & 7 and 16 consecutive fragment rows land on
// 16 distinct bank quads; 64-byte q8_0 rows (four per bank row) use
// (row >> 2) & 3.
// q8_0 weights stay int8 in LDS next to their f16 scales and are dequantised
// after the LDS read.
//
// K permutation (identical for A and B, so the contraction is unchanged): in
// substep s (0..3) of a 64-wide slab, lane half q = lane/32 holds
// k = 32q + 8s + [0..7].  A lane's 32 k-values are then one contiguous q8_0
// block: one scale per lane per slab and 32 contiguous weight bytes.
// ===========================================================================
constexpr int DMA_NS = 3;

template <int TM, int TN, int WT>
struct DmaCfg {
    static constexpr int BM = 64 * TM, BN = 64 * TN;      // 2x2 waves of (32 TM) x (32 TN)
    static constexpr int A_BYTES = BM * 128;
    static constexpr int B_BYTES = WT == GT_Q8_0 ? BN * 64 : WT == GT_Q4_K ? BN * 32 : BN * 128;
    static constexpr int S_BYTES = WT == GT_Q8_0 ? BN * 4 : WT == GT_Q4_K ? BN * 16 : 0;
    static constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
    static constexpr int B_DMA = B_BYTES % 4096 == 0 ? 16 : 4;         // bytes per lane per weight DMA
    static constexpr int A_INSTR = A_BYTES / 1024 / 4;                 // per wave
    static constexpr int B_INSTR = B_BYTES / (64 * B_DMA) / 4;
    // q8_0: every wave loads all scales (BN * 4 bytes); q4_K: the waves split
    // the {scale, min} pairs (BN * 16 bytes) in 256-byte pieces
    static constexpr int S_INSTR = WT == GT_Q8_0 ? (BN + 63) / 64 : WT == GT_Q4_K ? S_BYTES / 1024 : 0;
    static constexpr int PER_SLAB = A_INSTR + B_INSTR + S_INSTR;
    static_assert(A_BYTES % 4096 == 0 && B_BYTES % 1024 == 0, "tile must split into equal parts per wave");
};

// Buffer load of 4 bytes per lane straight into LDS: lane L's data lands at
// lds + 4 L; soff is wave-uniform (lds_dma16 in common.hpp moves 16 bytes).
__device__ __forceinline__ void lds_dma4(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, voff, soff, 0, 0);
}

// Per-lane source offsets of one wave's share of a K slab, computed once: in
// the K loop a slab is issued with the K offset in a scalar register and the
// LDS destination in m0, so issuing costs no vector ALU work.  Sources are
// buffer resources based at the tile's first row (offsets stay 32-bit); rows
// past M or N are clamped to the last valid one.
template <int TM, int TN, int WT>
struct DmaSrc {
    typedef DmaCfg<TM, TN, WT> C;
    __amdgpu_buffer_rsrc_t ra, rw, rs;
    uint32_t va[C::A_INSTR], vb[C::B_INSTR], vs[C::S_INSTR > 0 ? C::S_INSTR : 1];
    int wid, L;   // L: rows per slab block of a q8_0 weight

    __device__ __forceinline__ void init(const GemmParams& p, int m0, int n0, int wid_, int lane) {
        wid = wid_;
        const int mb = max(m0, 0);   // tiles of the fused conv-module epilogue start H rows early
        ra = make_rsrc((const f16*)p.A + (int64_t)mb * p.lda, ((int64_t)(p.M - mb - 1) * p.lda + p.K) * 2);
        L = slab_rows(p);
        if constexpr (WT == GT_Q8_0 || WT == GT_Q4_K) {
            // slab-major: a slab's rows n0.. are contiguous WB-byte blocks, slab stride L * WB
            constexpr int WB = WT == GT_Q8_0 ? 64 : 32;
            rw = make_rsrc((const uint8_t*)p.Wq + (int64_t)n0 * WB, ((int64_t)(p.K / 64 - 1) * L + (p.N - n0)) * WB);
        } else {
            rw = make_rsrc((const uint8_t*)p.Wq + n0 * (int64_t)p.K * 2, (p.N - n0) * (int64_t)p.K * 2);
        }
#pragma unroll
        for (int i = 0; i < C::A_INSTR; ++i) {
            const int slot = (wid * C::A_INSTR + i) * 64 + lane;   // 1 KB block = 8 rows of 128 B
            const int row = slot >> 3, c = (slot & 7) ^ ((row >> 1) & 7);
            const int m = min(max(m0 + row, 0), p.M - 1) - mb;
            va[i] = (uint32_t)(((int64_t)m * p.lda + 8 * c) * 2);
        }
        if constexpr (WT == GT_Q8_0) {
#pragma unroll
            for (int i = 0; i < C::B_INSTR; ++i) {
                const int slot = (wid * C::B_INSTR + i) * 64 + lane;   // 16 rows of 64 B
                const int row = slot >> 2, c = (slot & 3) ^ ((row >> 2) & 3);
                const int n = min(row, p.N - n0 - 1);
                vb[i] = (uint32_t)(n * 64 + 16 * c);
            }
            rs = make_rsrc((const uint8_t*)p.Ws + (int64_t)n0 * 4, ((int64_t)(p.K / 64 - 1) * L + (p.N - n0)) * 4);
#pragma unroll
            for (int i = 0; i < C::S_INSTR; ++i) {
                const int n = min(i * 64 + lane, p.N - n0 - 1);    // 4 B = the slab's 2 scales of a row
                vs[i] = (uint32_t)(n * 4);
            }
        } else if constexpr (WT == GT_Q4_K) {
            // 32 nibble bytes per row and slab, 16-byte chunk c stored at c ^ ((row >> 3) & 1)
#pragma unroll
            for (int i = 0; i < C::B_INSTR; ++i) {
                const int slot = (wid * C::B_INSTR + i) * 64 + lane;
                int row, off;
                if constexpr (C::B_DMA == 16) {
                    row = slot >> 1;
                    off = 16 * ((slot & 1) ^ ((row >> 3) & 1));
                } else {
                    row = slot >> 3;
                    off = 16 * (((slot >> 2) & 1) ^ ((row >> 3) & 1)) + 4 * (slot & 3);
                }
                const int n = min(row, p.N - n0 - 1);
                vb[i] = (uint32_t)(n * 32 + off);
            }
            // {d*sc, dmin*m} float pairs of the slab's two sub-blocks: 16 B per row, slab-major
            rs = make_rsrc((const uint8_t*)p.Ws + (int64_t)n0 * 16, ((int64_t)(p.K / 64 - 1) * L + (p.N - n0)) * 16);
#pragma unroll
            for (int i = 0; i < C::S_INSTR; ++i) {
                const int slot = (wid * C::S_INSTR + i) * 64 + lane;
                const int n = min(slot >> 2, p.N - n0 - 1);
                vs[i] = (uint32_t)(n * 16 + 4 * (slot & 3));
            }
        } else {
            rs = rw;
#pragma unroll
            for (int i = 0; i < C::B_INSTR; ++i) {
                const int slot = (wid * C::B_INSTR + i) * 64 + lane;
                const int row = slot >> 3, c = (slot & 7) ^ ((row >> 1) & 7);
                const int n = min(row, p.N - n0 - 1);
                vb[i] = (uint32_t)(((int64_t)n * p.K + 8 * c) * 2);
            }
        }
    }

    __device__ __forceinline__ void issue(uint8_t* st, int k0) const {
#pragma unroll
        for (int i = 0; i < C::A_INSTR; ++i) lds_dma16(ra, st + (wid * C::A_INSTR + i) * 1024, va[i], k0 * 2);
        uint8_t* bs = st + C::A_BYTES;
        const int kb = WT == GT_Q8_0 ? (k0 / 64) * L * 64 : WT == GT_Q4_K ? (k0 / 64) * L * 32 : k0 * 2;
#pragma unroll
        for (int i = 0; i < C::B_INSTR; ++i) {
            if constexpr (C::B_DMA == 16) lds_dma16(rw, bs + (wid * C::B_INSTR + i) * 1024, vb[i], kb);
            else lds_dma4(rw, bs + (wid * C::B_INSTR + i) * 256, vb[i], kb);
        }
        uint8_t* ss = bs + C::B_BYTES;
        if constexpr (WT == GT_Q8_0) {
#pragma unroll
            for (int i = 0; i < C::S_INSTR; ++i) lds_dma4(rs, ss + i * 256, vs[i], (k0 / 64) * L * 4);
        } else if constexpr (WT == GT_Q4_K) {
#pragma unroll
            for (int i = 0; i < C::S_INSTR; ++i) lds_dma4(rs, ss + (wid * C::S_INSTR + i) * 256, vs[i], (k0 / 64) * L * 16);
        }
    }
};

// B operand of one slab for one wave in two phases: load() issues the LDS
// reads of the raw weights (q8_0: 32 bytes and the block scale per lane and
// 32-block; q4_K: 32 nibble bytes and the {d*sc, dmin*m} pair; f16: the four
// 8-half fragments), convert() turns them into bf[j][s], the f16 fragment of
// substep s.  TM x TN: the workgroup tile in 64-blocks; WTN: the wave's 32-column
// blocks.
template <int TM, int TN, int WT, int WTN>
struct BSlab {
    typedef DmaCfg<TM, TN, WT> C;
    int4v raw[WTN][WT == GT_F16 ? 4 : 2];
    f16 dq[WTN];       // q8_0: the 32-block scale d
    float2v sc[WTN];   // q4_K: {d*sc, dmin*m}
    __device__ __forceinline__ void load(const uint8_t* st, int wn, int lane) {
        const int q = lane >> 5, r32 = lane & 31;
        const uint8_t* bs = st + C::A_BYTES;
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            const int row = wn * WTN * 32 + 32 * j + r32;
            if constexpr (WT == GT_Q8_0) {
                const int sw = (row >> 2) & 3;
                raw[j][0] = *(const int4v*)(bs + row * 64 + (((2 * q) ^ sw) << 4));
                raw[j][1] = *(const int4v*)(bs + row * 64 + (((2 * q + 1) ^ sw) << 4));
                dq[j] = *(const f16*)(bs + C::B_BYTES + row * 4 + q * 2);
            } else if constexpr (WT == GT_Q4_K) {
                const int sw = (row >> 3) & 1;
                raw[j][0] = *(const int4v*)(bs + row * 32 + (sw << 4));
                raw[j][1] = *(const int4v*)(bs + row * 32 + ((sw ^ 1) << 4));
                sc[j] = *(const float2v*)(bs + C::B_BYTES + row * 16 + q * 8);
            } else {
                const uint8_t* rp = bs + row * 128;
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) raw[j][s2] = *(const int4v*)(rp + (((4 * q + s2) ^ ((row >> 1) & 7)) << 4));
            }
        }
    }
    __device__ __forceinline__ void convert(half8v (&bf)[WTN][4], int lane) const {
        const int q = lane >> 5;
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            if constexpr (WT == GT_F16) {
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) bf[j][s2] = __builtin_bit_cast(half8v, raw[j][s2]);
            } else {
                half2v m2 = {}, nm2 = {};
                if constexpr (WT == GT_Q8_0) {
                    m2 = (half2v){dq[j], dq[j]};
                } else {
                    m2 = (half2v){(f16)sc[j].x, (f16)sc[j].x};
                    nm2 = (half2v){(f16)-sc[j].y, (f16)-sc[j].y};
                }
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) {
                    const uint32_t w0 = (uint32_t)(s2 < 2 ? raw[j][0][2 * s2] : raw[j][1][2 * (s2 - 2)]);
                    const uint32_t w1 = (uint32_t)(s2 < 2 ? raw[j][0][2 * s2 + 1] : raw[j][1][2 * (s2 - 2) + 1]);
                    half2v h0, h1, h2, h3;
                    if constexpr (WT == GT_Q8_0) {
                        i8x4_to_f16(w0, m2, h0, h1);
                        i8x4_to_f16(w1, m2, h2, h3);
                    } else {
                        nib4_to_f16(w0, q, m2, nm2, h0, h1);
                        nib4_to_f16(w1, q, m2, nm2, h2, h3);
                    }
                    bf[j][s2] = (half8v){h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
                }
            }
        }
    }
};

// One 64-deep slab of MFMAs for one wave: acc[i][j] += A block i x B block j.
// PF: issue every LDS read of the slab (B first, then all A fragments) before
// the dequantisation, so that the A reads land while the VALU converts B; the
// schedule barrier keeps the compiler from sinking the A reads to their MFMAs.
// Otherwise A fragments are read per substep (fewer registers).
template <int TM, int TN, int WT, int WTM, int WTN, bool PF>
__device__ __forceinline__ void mma32_slab(const uint8_t* st, float16v (&acc)[WTM][WTN], int wm, int wn,
                                           int lane) {
    const int q = lane >> 5, r32 = lane & 31;
    BSlab<TM, TN, WT, WTN> b;
    b.load(st, wn, lane);
    half8v bf[WTN][4];
    if constexpr (PF) {
        half8v af[4][WTM];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
            for (int i = 0; i < WTM; ++i) {
                const int row = wm * WTM * 32 + 32 * i + r32;
                af[s2][i] = *(const half8v*)(st + row * 128 + (((4 * q + s2) ^ ((row >> 1) & 7)) << 4));
            }
        __builtin_amdgcn_sched_barrier(0);
        b.convert(bf, lane);
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
            for (int i = 0; i < WTM; ++i)
#pragma unroll
                for (int j = 0; j < WTN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s2][i], bf[j][s2], acc[i][j], 0, 0, 0);
    } else {
        b.convert(bf, lane);
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll
            for (int i = 0; i < WTM; ++i) {
                const int row = wm * WTM * 32 + 32 * i + r32;
                const half8v af = *(const half8v*)(st + row * 128 + (((4 * q + s2) ^ ((row >> 1) & 7)) << 4));
#pragma unroll
                for (int j = 0; j < WTN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[j][s2], acc[i][j], 0, 0, 0);
            }
        }
    }
}

// Epilogue for the 32x32 accumulator layout: register r of a lane holds
// row 8*(r/4) + 4*(lane/32) + r%4, column lane%32 of its 32x32 block.
template <int EPI, typename ActT, int TM, int TN>
__device__ __forceinline__ void epilogue32(const GemmParams& p, float16v (&acc)[TM][TN], int mw, int nw,
                                           int lane) {
    const int lr = 4 * (lane >> 5), lc = lane & 31;
    if constexpr (EPI == EPI_GLU) {
        // pointwise_conv1 rows are interleaved in 32-row groups (a0..31, b0..31, ...):
        // block 2jj holds the GLU inputs a, block 2jj+1 the matching gates b.
        static_assert(TN % 2 == 0, "GLU needs an even number of 32-column blocks");
        const int half_n = p.N / 2;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int jj = 0; jj < TN / 2; ++jj)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = mw + 32 * i + 8 * (r >> 2) + lr + (r & 3);
                    const int na = nw + 64 * jj + lc;
                    const int og = nw / 2 + 32 * jj + lc;
                    if (m < p.M && og < half_n) {
                        const float a = acc[i][2 * jj][r] + (p.bias ? p.bias[na] : 0.f);
                        const float g = acc[i][2 * jj + 1][r] + (p.bias ? p.bias[na + 32] : 0.f);
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
                for (int r = 0; r < 16; ++r) {
                    const int m = mw + 32 * i + 8 * (r >> 2) + lr + (r & 3);
                    const int n = nw + 32 * j + lc;
                    if (m < p.M && n < p.N) epi_one<EPI, ActT>(p, m, n, acc[i][j][r]);
                }
    }
}

// Coalesced epilogue: each wave stages its finished tile (after the elementwise
// epilogue math) in its own LDS region, then writes rows out with 16-byte
// stores; the residual update reads and writes the f32 stream in 16-byte
// vectors too.  The accumulator layout alone would give 2- or 4-byte stores
// scattered over 8 rows per instruction.
// Coalesced form of the channel-major flatten epilogue (EPI_RELU_TR): GEMM row
// m = (b, t, f) with f fastest, column n = channel; output row (b, t) holds
// n * F + f.  A wave's rows cover whole (b, t) groups when 32 TM is a
// multiple of F, and then its 32 TN columns form one contiguous run of
// 32 TN * F outputs per (b, t): staged in LDS as [bt][f][n] (row pitch 32 TN
// + 1 keeps both the staging writes and the gathering reads conflict-free)
// and written with 16-byte stores.
template <int TM, int TN>
__device__ __forceinline__ void epilogue32_relu_tr(const GemmParams& p, float16v (&acc)[TM][TN], float* wsm,
                                                   int mw, int nw, int lane) {
    constexpr int WR = 32 * TM, WC = 32 * TN, LDN = WC + 1;
    const int F = p.trF, nbt = WR / F;
    const int lr = 4 * (lane >> 5), lc = lane & 31;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = nw + 32 * j + lc;
            const float bb = p.bias ? p.bias[min(n, p.N - 1)] : 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rr = 32 * i + 8 * (r >> 2) + lr + (r & 3);
                const float v = acc[i][j][r] + bb;
                wsm[rr * LDN + 32 * j + lc] = v > 0.f ? v : 0.f;   // rr = bt_local * F + f
            }
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    const int run = WC * F;                       // outputs per (b, t) in this wave
    for (int c = lane; c < nbt * (run / 8); c += 64) {
        const int btl = c / (run / 8), e0 = (c % (run / 8)) * 8;
        const int m_first = mw + btl * F;
        if (m_first >= p.M) continue;
        const int bt = m_first / F, t = bt % p.T, b = bt / p.T;
        const bool dead = p.valid && t >= p.valid[b];
        f16* dst = (f16*)p.Y + ((int64_t)bt * p.N + nw) * F + e0;
        half8v h;
        // element e0 + e is channel nl, frequency f of the run, advanced
        // incrementally (no division per element)
        int nl = e0 / F, f = e0 - nl * F;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h[e] = dead ? (f16)0.f : (f16)wsm[(btl * F + f) * LDN + nl];
            if (++f == F) {
                f = 0;
                ++nl;
            }
        }
        if (nw + (e0 + 7) / F < p.N) {
            *(half8v*)dst = h;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (nw + (e0 + e) / F < p.N) dst[e] = h[e];
        }
    }
}

// Per-column epilogue constants of one wave's 32 NJ output columns (column
// nw + 32 j + lane % 32 for block j): bias, folded-LayerNorm W*gamma, and for
// the LayerNorm-statistics epilogue the gamma quad of the lane's copy-out
// columns (and the gamma / beta quads of a LayerNorm applied to the residual).
// Loaded before the main loop so the epilogue does not wait for them.
template <int NJ>
struct EpiCols {
    float b[NJ], c1[NJ];
    float4v g, rg, rb;
    __device__ __forceinline__ void load(const GemmParams& p, int nw, int lane, bool fold, bool gamma) {
        const int lc = lane & 31;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int n = min(nw + 32 * j + lc, p.N - 1);
            b[j] = p.bias ? p.bias[n] : 0.f;
            c1[j] = fold ? p.fold_c1[n] : 0.f;
        }
        g = rg = rb = (float4v){0.f, 0.f, 0.f, 0.f};
        if (gamma) {
            const int n = nw + (lane % (8 * NJ)) * 4;   // the copy-out columns of RESID_LN
            if (n < p.N) {
                g = *(const float4v*)(p.ln_g + n);
                if (p.res_rows) {
                    rg = *(const float4v*)(p.res_g + n);
                    rb = *(const float4v*)(p.res_b + n);
                }
            }
        }
    }
};

// The residual stream's values under one wave's output tile, loaded into
// registers before the main loop so that the residual epilogue does not wait
// for them: chunk t of a lane is the float4 at row rr = (lane + 64 t) / CPR,
// column 4 ((lane + 64 t) % CPR) of the wave tile (the epilogue's own order).
// RS: also the rows' {mean, rstd} of a LayerNorm applied to the residual.
template <int WR, int CPR, bool RS = false>
struct ResidPre {
    static constexpr int NT = WR * CPR / 64;
    static_assert(NT * 64 == WR * CPR, "whole chunks per lane");
    float4v v[NT];
    float2v rs[RS ? NT : 1];
    // Raw buffer loads over the wave's rows (rows past M, and float4s reaching
    // past N, are out of range and read zero): one offset add and one load per
    // chunk, where guarded global loads took a branch and 64-bit address
    // arithmetic each (~1.5k cycles before the first DMA of the product).
    __device__ __forceinline__ void load(const GemmParams& p, int mw, int nw, int lane) {
        const int rows = min(WR, p.M - mw);   // valid rows of the wave tile (<= 0: none)
        const __amdgpu_buffer_rsrc_t ry =
            make_rsrc((const float*)p.Y + (int64_t)max(mw, 0) * p.ldy,
                      rows > 0 ? ((int64_t)(rows - 1) * p.ldy + p.N) * 4 : 0);
        __amdgpu_buffer_rsrc_t rr = ry;
        if constexpr (RS) rr = make_rsrc((const float2v*)p.res_rows + max(mw, 0), rows > 0 ? (int64_t)rows * 8 : 0);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int c = lane + 64 * t, r = c / CPR, n = nw + (c % CPR) * 4;
            const uint32_t off = r < rows && n + 3 < p.N ? (uint32_t)((r * p.ldy + n) * 4) : OOB;
            v[t] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(ry, off, 0, 0));
            if constexpr (RS) {
                if (p.res_rows) {
                    const uint32_t ro = r < rows ? (uint32_t)(r * 8) : OOB;
                    rs[t] = __builtin_bit_cast(float2v, __builtin_amdgcn_raw_buffer_load_b64(rr, ro, 0, 0));
                }
            }
        }
    }
};

// Step 2 of the LDS-staged epilogues: the wave's WR x WC output tile, staged
// as f32 rows of WC + 4 floats at wsm (rows from mw, columns from nw; GLU
// output columns from nw / 2), leaves by coalesced 16-byte stores, the
// residual updates reading the residual stream at the same granularity
// (xpre: those values from ResidPre, or null; xrs: with xpre, the rows'
// {mean, rstd} for a LayerNorm applied to the residual).
template <int EPI, int WR, int WC, int NJ>
__device__ __forceinline__ void epilogue_lds_out(const GemmParams& p, const float* wsm, int mw, int nw, int lane,
                                                 const EpiCols<NJ>& ec, const float4v* xpre, const float2v* xrs) {
    constexpr int LDW = WC + 4;
    const int ncol = EPI == EPI_GLU ? p.N / 2 : p.N;
    const int n0 = EPI == EPI_GLU ? nw / 2 : nw;
    if constexpr (EPI == EPI_RESID_LN) {
        // 8 lanes hold one row's 32-column group: residual update, x * gamma in
        // f16, and the group's mean and sum of squared deviations (two passes
        // over registers, shuffles within the 8 lanes)
        constexpr int CPR = WC / 4;
        static_assert(CPR % 8 == 0 && 64 % CPR == 0, "RESID_LN: whole 32-column groups per wave");
        const int G = p.N / 32;
        const int cc = (lane % CPR) * 4, n = n0 + cc;   // a lane's columns are the same on every row
        const float4v g = ec.g;
#pragma unroll
        for (int t = 0; t < WR * CPR / 64; ++t) {
            const int c = lane + 64 * t;
            const int rr = c / CPR;
            const int m = mw + rr;
            if (m < p.M && n < p.N) {   // uniform over the 8 lanes of a group (same row, N % 32 == 0)
                const float4v v = *(const float4v*)(wsm + rr * LDW + cc);
                float* dst = (float*)p.Y + (int64_t)m * p.ldy + n;
                float4v x = xpre ? xpre[t] : *(const float4v*)dst;
                if (p.res_rows) {   // the stream before a LayerNorm whose output was not stored
                    const float2v rs = xrs ? xrs[t] : ((const float2v*)p.res_rows)[m];
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[e] = ((x[e] - rs.x) * rs.y) * ec.rg[e] + ec.rb[e];
                }
                x += v;
                *(float4v*)dst = x;
                const half4v h = {(f16)(x[0] * g[0]), (f16)(x[1] * g[1]), (f16)(x[2] * g[2]), (f16)(x[3] * g[3])};
                *(half4v*)((f16*)p.ln_h + (int64_t)m * p.N + n) = h;
                const float mean = group_sum((x[0] + x[1]) + (x[2] + x[3]), 8) * (1.0f / 32.0f);
                float d2 = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) d2 += (x[e] - mean) * (x[e] - mean);
                d2 = group_sum(d2, 8);
                if ((lane & 7) == 0) ((float2v*)p.ln_stats)[(int64_t)m * G + n / 32] = (float2v){mean, d2};
            }
        }
    } else if constexpr (EPI == EPI_STORE_F32 || EPI == EPI_RESID) {
        constexpr int CPR = WC / 4;   // float4 chunks per row
        static_assert(WR * CPR % 64 == 0, "whole chunks per lane");
#pragma unroll
        for (int t = 0; t < WR * CPR / 64; ++t) {
            const int c = lane + 64 * t;
            const int rr = c / CPR, cc = (c % CPR) * 4;
            const int m = mw + rr, n = n0 + cc;
            if (m >= p.M) continue;
            const float4v v = *(const float4v*)(wsm + rr * LDW + cc);
            float* dst = (float*)p.Y + (int64_t)m * p.ldy + n;
            if (n + 3 < ncol) {
                if constexpr (EPI == EPI_RESID) *(float4v*)dst = (xpre ? xpre[t] : *(const float4v*)dst) + v;
                else *(float4v*)dst = v;
            } else {
                for (int e = 0; e < 4 && n + e < ncol; ++e) {
                    if constexpr (EPI == EPI_RESID) dst[e] += v[e];
                    else dst[e] = v[e];
                }
            }
        }
    } else {
        constexpr int CPR = WC / 8;   // 8-half chunks per row
        for (int c = lane; c < WR * CPR; c += 64) {
            const int rr = c / CPR, cc = (c % CPR) * 8;
            const int m = mw + rr, n = n0 + cc;
            if (m >= p.M) continue;
            const float4v v0 = *(const float4v*)(wsm + rr * LDW + cc);
            const float4v v1 = *(const float4v*)(wsm + rr * LDW + cc + 4);
            f16* dst = (f16*)p.Y + (int64_t)m * p.ldy + n;
            if (n + 7 < ncol) {
                const half8v h = {(f16)v0[0], (f16)v0[1], (f16)v0[2], (f16)v0[3],
                                  (f16)v1[0], (f16)v1[1], (f16)v1[2], (f16)v1[3]};
                *(half8v*)dst = h;
            } else {
                for (int e = 0; e < 8 && n + e < ncol; ++e) dst[e] = (f16)(e < 4 ? v0[e] : v1[e - 4]);
            }
        }
    }
}

// fold: ftab (LDS) holds {mean, rstd} of the workgroup tile's rows for a
// folded LayerNorm, indexed from the tile's first row; trow0 is this wave's
// first row within the tile.  (ftab is always a valid LDS address, so that its
// loads stay LDS loads.)
// xpre: the wave tile's residual values from ResidPre (RESID / RESID_LN), or null;
// xrs: with xpre, the rows' {mean, rstd} for a LayerNorm applied to the residual.
template <int EPI, int TM, int TN>
__device__ __forceinline__ void epilogue32_lds(const GemmParams& p, float16v (&acc)[TM][TN], float* wsm,
                                               int mw, int nw, int lane, const EpiCols<TN>& ec,
                                               bool fold = false, const float2v* ftab = nullptr, int trow0 = 0,
                                               const float4v* xpre = nullptr, const float2v* xrs = nullptr) {
    constexpr int WR = 32 * TM;
    constexpr int WC = EPI == EPI_GLU ? 16 * TN : 32 * TN;   // output columns of this wave
    constexpr int LDW = WC + 4;
    const int lr = 4 * (lane >> 5), lc = lane & 31;
    // 1) elementwise math in registers, staged as f32
    if constexpr (EPI == EPI_GLU) {
        static_assert(TN % 2 == 0, "GLU needs an even number of 32-column blocks");
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            float2v st[16];   // folded LayerNorm {mean, rstd} of this lane's 16 rows
            if (fold) {
#pragma unroll
                for (int r = 0; r < 16; ++r) st[r] = ftab[trow0 + 32 * i + 8 * (r >> 2) + lr + (r & 3)];
            }
#pragma unroll
            for (int jj = 0; jj < TN / 2; ++jj) {
                const float ba = ec.b[2 * jj], bg = ec.b[2 * jj + 1];
                const float ca = ec.c1[2 * jj], cg = ec.c1[2 * jj + 1];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int rr = 32 * i + 8 * (r >> 2) + lr + (r & 3);
                    const int m = mw + rr;
                    float xa = acc[i][2 * jj][r], xg = acc[i][2 * jj + 1][r];
                    if (fold) {
                        xa = st[r].y * (xa - st[r].x * ca);
                        xg = st[r].y * (xg - st[r].x * cg);
                    }
                    float o = (xa + ba) * sigmoid_dev(xg + bg);
                    if (p.valid && m < p.M) {
                        const int b = m / p.T, t = m - b * p.T;
                        if (t >= p.valid[b]) o = 0.f;
                    }
                    wsm[rr * LDW + 32 * jj + lc] = o;
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            float2v st[16];   // folded LayerNorm {mean, rstd} of this lane's 16 rows
            if (fold) {
#pragma unroll
                for (int r = 0; r < 16; ++r) st[r] = ftab[trow0 + 32 * i + 8 * (r >> 2) + lr + (r & 3)];
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const float bb = ec.b[j], c1 = ec.c1[j];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int rr = 32 * i + 8 * (r >> 2) + lr + (r & 3);
                    float v = acc[i][j][r];
                    if (fold) v = st[r].y * (v - st[r].x * c1);
                    v += bb;
                    if constexpr (EPI == EPI_SILU) v = silu_dev(v);
                    else if constexpr (EPI == EPI_RELU) v = v > 0.f ? v : 0.f;
                    else v = v * p.alpha;    // STORE, STORE_F32, RESID
                    wsm[rr * LDW + 32 * j + lc] = v;
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    epilogue_lds_out<EPI, WR, WC, TN>(p, wsm, mw, nw, lane, ec, xpre, xrs);
}

// Constants of the fused conv-module epilogue, loaded before the main loop:
// thread tid's tile row {time index, kept} (tid < BM) and the depthwise taps,
// bias and folded BatchNorm of its channel pair c, c + 1 (c = n0/2 + 2 (tid % CP)).
template <int BM, int CP>
struct DwPre {
    int2 rt;
    float2v wk[GLU_DW_K], db, sc, sh;
    __device__ __forceinline__ void load(const GemmParams& p, int m0, int n0, int tid) {
        static_assert(BM <= 256, "one tile row per thread");
        rt = make_int2(0, 0);
        const int m = m0 + tid;
        if (tid < BM && m >= 0 && m < p.M) {
            const int b = udiv_small(m, p.T), t = m - b * p.T;   // M < 2^22 (checked at launch)
            rt = make_int2(t, !p.valid || t < p.valid[b]);
        }
        const int c = min(n0 / 2 + 2 * (tid % CP), p.N / 2 - 2);
#pragma unroll
        for (int j = 0; j < GLU_DW_K; ++j)
            wk[j] = (float2v){p.dw_w[c * GLU_DW_K + j], p.dw_w[(c + 1) * GLU_DW_K + j]};
        db = p.dw_b ? (float2v){p.dw_b[c], p.dw_b[c + 1]} : (float2v){0.f, 0.f};
        sc = (float2v){p.dw_scale[c], p.dw_scale[c + 1]};
        sh = (float2v){p.dw_shift[c], p.dw_shift[c + 1]};
    }
};

// Conformer convolution module after pointwise_conv1, in one pass over the
// tile: GLU + pad mask (rows t >= valid -> 0) staged for the whole workgroup
// tile in LDS as f32 [64 TM rows][32 TN channels], then the depthwise conv
// over time (zero padding outside each item), its bias, the folded BatchNorm
// and SiLU for the tile's inner 64 TM - 2 H rows (conformer.cpp:55-157).
// m0 is the tile's first GEMM row (H rows before the first row written).
template <int TM, int TN>
__device__ __forceinline__ void epilogue32_glu_dw(const GemmParams& p, float16v (&acc)[TM][TN], float* G, int m0,
                                                  int n0, int wm, int wn, int tid, bool fold, const float2v* ftab,
                                                  const EpiCols<TN>& ec, const DwPre<64 * TM, 16 * TN>& dp) {
    static_assert(TN % 2 == 0, "GLU needs an even number of 32-column blocks");
    constexpr int BM = 64 * TM, CW = 32 * TN, LDG = CW + 2, K = GLU_DW_K, H = (K - 1) / 2;
    constexpr int CP = CW / 2, RG = 256 / CP, NR = BM - 2 * H, RPG = (NR + RG - 1) / RG;
    static_assert(256 % CP == 0, "channel pairs must divide the workgroup");
    const int lane = tid & 63, lr = 4 * (lane >> 5), lc = lane & 31;
    // 0) per tile row: time index and whether the GLU output is kept (row in
    //    [0, M) and t < valid), one division per row instead of per element
    int2* rtab = (int2*)(G + BM * LDG);
    if (tid < BM) rtab[tid] = dp.rt;
    __syncthreads();
    // 1) GLU + pad mask into LDS
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jj = 0; jj < TN / 2; ++jj) {
            const float ba = ec.b[2 * jj], bg = ec.b[2 * jj + 1];
            const float ca = ec.c1[2 * jj], cg = ec.c1[2 * jj + 1];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rr = wm * 32 * TM + 32 * i + 8 * (r >> 2) + lr + (r & 3);
                float xa = acc[i][2 * jj][r], xg = acc[i][2 * jj + 1][r];
                if (fold) {
                    const float2v st = ftab[rr];
                    xa = st.y * (xa - st.x * ca);
                    xg = st.y * (xg - st.x * cg);
                }
                float o = (xa + ba) * sigmoid_dev(xg + bg);
                if (!rtab[rr].y) o = 0.f;
                G[rr * LDG + wn * 16 * TN + 32 * jj + lc] = o;
            }
        }
    __syncthreads();
    // 2) depthwise conv: a thread owns 2 channels and RPG consecutive rows,
    //    with the K-row window in registers
    const int cp = tid % CP, g = tid / CP;
    const int cl = 2 * cp, c = n0 / 2 + cl;
    if (c >= p.N / 2) return;
    const float2v(&wk)[K] = dp.wk;
    const float2v db = dp.db, sc = dp.sc, sh = dp.sh;
    const int r0 = H + g * RPG;
    float2v win[RPG + K - 1];
#pragma unroll
    for (int q = 0; q < RPG + K - 1; ++q) {
        const int row = r0 - H + q;
        win[q] = row < BM ? *(const float2v*)(G + row * LDG + cl) : (float2v){0.f, 0.f};
    }
#pragma unroll
    for (int q = 0; q < RPG; ++q) {
        const int r = r0 + q, m = m0 + r;
        if (r < BM - H && m < p.M) {
            const int t = rtab[r].x;
            float2v a = {0.f, 0.f};
            if (t >= H && t < p.T - H) {
                // the whole window inside the item (all but 2 H frames of it)
#pragma unroll
                for (int j = 0; j < K; ++j) a += wk[j] * win[q + j];
            } else {
#pragma unroll
                for (int j = 0; j < K; ++j)
                    if ((unsigned)(t + j - H) < (unsigned)p.T) a += wk[j] * win[q + j];
            }
            const float2v y = (a + db) * sc + sh;
            const half2v h = {(f16)silu_dev(y[0]), (f16)silu_dev(y[1])};
            *(half2v*)((f16*)p.Y + (int64_t)m * p.ldy + c) = h;
        }
    }
}

// Folded LayerNorm row statistics of a tile.  The tile's rows hold G = N/32
// partials {mean, sum of squared deviations} each, BM * G * 8 contiguous bytes
// (rows clamped to [0, M)): prefetch() loads them as 16-byte chunks before the
// main loop (thread t takes chunks t, t + 256, ...; G/2 consecutive chunks per
// row, so a row's chunks sit in G/2 consecutive lanes of one wave), and
// finish() combines each row with shuffles (Chan's pairwise formula) into
// {mean, 1/sqrt(var + eps)} in LDS.
template <int BM, int NTH = 256>
struct FoldStats {
    static constexpr int MAXC = BM * 32 / 2 / NTH;   // chunks per thread for G <= 32
    float4v c[MAXC];
    __device__ __forceinline__ void prefetch(const GemmParams& p, int m0, int t) {
        const int lc = __builtin_ctz(p.fold_groups / 2), total = BM << lc;   // log2 chunks per row
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
            const int ch = t + NTH * i;
            if (ch < total) {
                const int r = ch >> lc, m = min(max(m0 + r, 0), p.M - 1);
                c[i] = *((const float4v*)p.fold_stats + ((int64_t)m << lc) + (ch & ((1 << lc) - 1)));
            } else {
                c[i] = (float4v){0.f, 0.f, 0.f, 0.f};
            }
        }
    }
    template <int CPR>
    __device__ __forceinline__ void finish_t(const GemmParams& p, float2v* tab, int t) const {
        constexpr int G = 2 * CPR, NC = BM * CPR / NTH > 0 ? BM * CPR / NTH : 1;
        static_assert(NC <= MAXC, "chunks");
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int ch = t + NTH * i;
            const float mean = group_sum(c[i][0] + c[i][2], CPR) * (1.0f / G);
            const float da = c[i][0] - mean, db = c[i][2] - mean;
            const float q = group_sum(c[i][1] + c[i][3] + 32.0f * (da * da + db * db), CPR);
            if (ch < BM * CPR && (ch & (CPR - 1)) == 0)
                tab[ch / CPR] = (float2v){mean, rsqrtf(q * (1.0f / (32.0f * G)) + p.fold_eps)};
        }
    }
    __device__ __forceinline__ void finish(const GemmParams& p, float2v* tab, int t) const {
        switch (p.fold_groups) {
        case 2: finish_t<1>(p, tab, t); break;
        case 4: finish_t<2>(p, tab, t); break;
        case 8: finish_t<4>(p, tab, t); break;
        case 16: finish_t<8>(p, tab, t); break;
        default: finish_t<16>(p, tab, t); break;
        }
    }
};

// KG = 2: eight waves in two groups of four; group g streams K slabs
// [g nk/2, (g+1) nk/2) through its own LDS ring, and the two partial tiles are
// summed in LDS (group 0 + group 1, a fixed order) before group 0 runs the
// epilogue.  For grids of about one tile per CU: two waves per SIMD instead of
// one.
// WL = wave layout: 0 = 2 x 2 waves of 32 TM x 32 TN each; 1 = four waves side
// by side along N, each 64 TM rows x 16 TN columns, so that no two waves
// dequantise the same weight rows; 2 = the 2 x 2 layout with the slab's LDS
// reads issued up front (as layout 1 does).
// WL = 3: layout 0 with the K range cut over p.ksplit workgroups per tile
// (split-K across workgroups, for grids far smaller than the chip).  Each
// workgroup writes its partial tile to p.sk_part and counts itself in
// p.sk_cnt[tile]; the last one to arrive sums the partials in split order (the
// same order whichever arrives last, so results are deterministic), resets the
// counter and runs the epilogue.
template <int TM, int TN, int WT, int EPI, int NS = DMA_NS, int KG = 1, int WL = 0>
__global__ __launch_bounds__(256 * KG, KG == 1 ? 2 : 1) void gemm_dma_kernel(GemmParams p) {
    constexpr bool SPLIT = WL == 3;
    typedef DmaCfg<TM, TN, WT> C;
    static_assert(WL != 1 || (TN % 2 == 0 && EPI != EPI_GLU && EPI != EPI_GLU_DW && EPI != EPI_RELU_TR &&
                              EPI != EPI_RELU2_F32),
                  "wave layout 1: even TN, LDS-staged non-GLU epilogues");
    constexpr int WTM = WL == 1 ? 2 * TM : TM, WTN = WL == 1 ? TN / 2 : TN;   // one wave's 32-blocks
    static_assert(NS == 2 || NS == 3, "LDS ring depth");
    static_assert(KG == 1 || (KG == 2 && (EPI == EPI_STORE || EPI == EPI_STORE_F32 || EPI == EPI_RESID ||
                                          EPI == EPI_SILU || EPI == EPI_RESID_LN)),
                  "K groups: LDS-staged epilogues only");
    __shared__ __attribute__((aligned(1024))) uint8_t smem_all[KG * NS * C::STAGE];
    prefetch_gemm_args(p);

    const int tid = threadIdx.x & 255, lane = tid & 63;
    const int wid_all = wave_id_uniform();
    const int kg = wid_all >> 2, wid = wid_all & 3;
    const int wm = WL == 1 ? 0 : wid >> 1, wn = WL == 1 ? wid : wid & 1;
    uint8_t* smem = smem_all + kg * NS * C::STAGE;
    // The fused conv-module epilogue needs DWH rows of GLU output either side
    // of the rows it writes: its tiles overlap by 2 DWH rows.
    constexpr int DWH = EPI == EPI_GLU_DW ? (GLU_DW_K - 1) / 2 : 0;
    constexpr int SM = C::BM - 2 * DWH;
    const int nbm = cdiv_dev(p.M, SM), nbn = cdiv_dev(p.N, C::BN);
    int bm, bn, tile = 0, split = 0;
    if constexpr (SPLIT) {
        // the splits of one tile are consecutive positions: usually on one XCD,
        // but they straddle two whenever an XCD's range of positions is not a
        // multiple of ksplit, so the handoff below is made coherent across XCDs
        const int k = xcd_tile(blockIdx.x, nbm * nbn * p.ksplit);
        tile = k / p.ksplit;
        split = k - tile * p.ksplit;
        xcd_rect(tile, nbm, nbn, p.xcd_gm, bm, bn);
    } else {
        xcd_tile_2d(blockIdx.x, nbm, nbn, p.xcd_gm, bm, bn);
    }
    const int m0 = bm * SM - DWH, n0 = bn * C::BN;

    float16v acc[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j) acc[i][j] = (float16v){};

    // folded LayerNorm: the row statistics' loads go out before the DMAs (oldest
    // in the vector-memory counter) and are combined after the main loop
    constexpr bool FOLD = EPI == EPI_STORE || EPI == EPI_SILU || EPI == EPI_GLU || EPI == EPI_GLU_DW;
    FoldStats<FOLD ? C::BM : 8> fst;
    if constexpr (FOLD) {
        if (p.fold_stats && kg == 0) fst.prefetch(p, m0, tid);
    }

    // residual epilogues: the tile's residual values are loaded now (behind the
    // statistics, ahead of the DMAs) and wait in registers for the epilogue
    constexpr int TAB = FOLD && KG == 1 ? C::BM * 8 : 0;
    constexpr bool whole = 4 * 32 * WTM * (32 * WTN + 4) * 4 + TAB <= KG * NS * C::STAGE;
    // Two K groups on a wave tile of two 32-row blocks share the end of the
    // tile: group g sums and runs the epilogue of row block g (the other
    // group's partial of it comes through LDS), so both groups' waves work in
    // the reduction and the epilogue instead of group 0's alone.
    constexpr bool KHALF = KG == 2 && WTM == 2 && !SPLIT && whole;
    constexpr int ER = KHALF ? 32 : 32 * WTM;   // rows of this wave's epilogue
    const int erow = wm * WTM * 32 + (KHALF ? kg * 32 : 0);   // its first row within the tile
    const bool epi_wave = KHALF || kg == 0;
    constexpr bool RPRE = (EPI == EPI_RESID || EPI == EPI_RESID_LN) && whole;
    ResidPre<RPRE ? ER : 64, RPRE ? 8 * WTN : 1, EPI == EPI_RESID_LN && RPRE> rpre;
    if constexpr (RPRE) {
        if (epi_wave) rpre.load(p, m0 + erow, n0 + wn * WTN * 32, lane);
    }
    // the epilogue's per-column (and conv-module per-channel) constants
    const bool fold = FOLD && p.fold_stats != nullptr;
    EpiCols<WTN> ecol;
    if (epi_wave) ecol.load(p, n0 + wn * WTN * 32, lane, fold, EPI == EPI_RESID_LN);
    DwPre<EPI == EPI_GLU_DW ? C::BM : 64, 16 * TN> dwpre;
    if constexpr (EPI == EPI_GLU_DW) dwpre.load(p, m0, n0, tid);

    // slabs of this group, its first K
    const int nk = SPLIT ? p.K / 64 / KG / p.ksplit : p.K / 64 / KG, kb = (split * KG + kg) * nk * 64;
    DmaSrc<TM, TN, WT> src;
    src.init(p, m0, n0, wid, lane);
    src.issue(smem, kb);
    if (NS == 3 && nk > 1) src.issue(smem + C::STAGE, kb + 64);
    int st = 0;
    for (int kt = 0; kt < nk; ++kt) {
        // this wave's DMAs for slab kt have landed (with 3 stages slab kt+1 may
        // still be in flight)
        if (NS == 3 && kt + 1 < nk) wait_vmcnt<C::PER_SLAB>();
        else wait_vmcnt<0>();
        // Every wave's part of slab kt is in LDS and stage (kt+NS-1)%NS is no
        // longer read.  A bare s_barrier: the DMA counter was bounded above, and
        // a fenced __syncthreads() would also drain the DMAs still in flight.
        __builtin_amdgcn_s_barrier();
        if (kt + NS - 1 < nk) {
            const int st2 = st + NS - 1 >= NS ? st - 1 : st + NS - 1;
            src.issue(smem + st2 * C::STAGE, kb + (kt + NS - 1) * 64);
        }
        mma32_slab<TM, TN, WT, WTM, WTN, WL == 1 || WL == 2>(smem + st * C::STAGE, acc, wm, wn, lane);
        st = st + 1 == NS ? 0 : st + 1;
    }
    // KHALF: the row block this wave finishes (its own partial plus the other
    // group's, the same two terms as group 0 + group 1: bit-identical)
    float16v fin[1][WTN];
    if constexpr (KHALF) {
        constexpr int R = WTN * 16;
        static_assert(8 * R * 64 * 4 <= KG * NS * C::STAGE, "partial tiles exceed LDS");
        // [wave][register / 4][lane] float4s: 16-byte accesses, 1 KB per instruction
        float4v* give = (float4v*)smem_all + wid_all * (R / 4) * 64 + lane;                      // region (kg, wid)
        const float4v* take = (const float4v*)smem_all + ((1 - kg) * 4 + wid) * (R / 4) * 64 + lane;   // (1-kg, wid)
        __syncthreads();
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float4v g;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * t + e;
                    g[e] = kg ? acc[0][j][r] : acc[1][j][r];
                    fin[0][j][r] = kg ? acc[1][j][r] : acc[0][j][r];
                }
                give[(j * 4 + t) * 64] = g;
            }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float4v o = take[(j * 4 + t) * 64];
#pragma unroll
                for (int e = 0; e < 4; ++e) fin[0][j][4 * t + e] += o[e];
            }
    } else if constexpr (KG == 2) {
        // lane-major [wave][register][lane] f32: conflict-free both ways
        constexpr int R = WTM * WTN * 16;
        static_assert(4 * R * 64 * 4 <= KG * NS * C::STAGE, "partial tile exceeds LDS");
        float* red = (float*)smem_all + wid * R * 64 + lane;
        __syncthreads();
        if (kg == 1) {
#pragma unroll
            for (int i = 0; i < WTM; ++i)
#pragma unroll
                for (int j = 0; j < WTN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) red[((i * WTN + j) * 16 + r) * 64] = acc[i][j][r];
        }
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int i = 0; i < WTM; ++i)
#pragma unroll
                for (int j = 0; j < WTN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] += red[((i * WTN + j) * 16 + r) * 64];
        }
    }
    if constexpr (SPLIT) {
        static_assert(!FOLD && EPI != EPI_GLU_DW, "split-K: no folded LayerNorm");
        // Partial tiles [tile][split][wave][register][lane].  Why the relaxed
        // accesses below suffice on gfx950 (the C++ model alone would ask for
        // release / acquire): every access to the partials and the counter is
        // an agent-scope atomic, which gfx950 performs at the device's point of
        // coherence (the store writes through the XCD's L2, the load does not
        // take a possibly stale L2 line), whichever XCD issues it.  A writer
        // (1) stores its partial, (2) waits with s_waitcnt vmcnt(0), which
        // returns only once those stores are acknowledged at that scope, and
        // only then (3) issues its counter increment; the last arriver's
        // increment is ordered after every writer's (one location, one
        // modification order), and its partial loads are issued only after the
        // increment has returned.  So each partial it loads was complete at the
        // coherence point before it was read.  An agent-scope release / acquire
        // fence would add a write-back and an invalidation of the whole L2 of
        // the XCD, evicting the weights every other workgroup is streaming
        // (57 us per launch against 7.7 - 14 us, measured); that is the only
        // thing it would add here, since no plain (cacheable) access carries
        // data between the workgroups.
        constexpr int R = WTM * WTN * 16;
        const int S = p.ksplit;
        float* part = p.sk_part + (int64_t)tile * S * (4 * R * 64) + wid * R * 64 + lane;
        if (kg == 0) {
#pragma unroll
            for (int i = 0; i < WTM; ++i)
#pragma unroll
                for (int j = 0; j < WTN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        __hip_atomic_store(part + (int64_t)split * (4 * R * 64) + ((i * WTN + j) * 16 + r) * 64,
                                           acc[i][j][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wait_vmcnt<0>();   // the partial has reached the device before the count
        }
        __shared__ int sk_last;
        __syncthreads();
        if (threadIdx.x == 0) {
            const int seen = __hip_atomic_fetch_add(p.sk_cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sk_last = seen == S - 1;
            // every split of this tile has counted: ready for the next launch
            if (seen == S - 1) __hip_atomic_store(p.sk_cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!sk_last) return;
        if (kg == 0) {
            // the sum in split order, whichever split arrived last
            float16v own[WTM][WTN];
#pragma unroll
            for (int i = 0; i < WTM; ++i)
#pragma unroll
                for (int j = 0; j < WTN; ++j) own[i][j] = acc[i][j];
            for (int t = 0; t < S; ++t) {
#pragma unroll
                for (int i = 0; i < WTM; ++i)
#pragma unroll
                    for (int j = 0; j < WTN; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const float v = t == split ? own[i][j][r]
                                                       : __hip_atomic_load(part + (int64_t)t * (4 * R * 64) +
                                                                               ((i * WTN + j) * 16 + r) * 64,
                                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            acc[i][j][r] = t == 0 ? v : acc[i][j][r] + v;
                        }
            }
        }
    }
    // folded LayerNorm: the tile's row statistics at the top of the LDS block
    // (published by the barrier before the staging below)
    float2v* ftab = (float2v*)(smem_all + KG * NS * C::STAGE) - C::BM;
    if constexpr (FOLD) {
        if (fold) {
            __syncthreads();
            if (kg == 0) fst.finish(p, ftab, tid);
        }
    }
    if constexpr (EPI == EPI_RELU2_F32) {
        epilogue32<EPI, f16, TM, TN>(p, acc, m0 + wm * TM * 32, n0 + wn * TN * 32, lane);
    } else if constexpr (EPI == EPI_GLU_DW) {
        static_assert(C::BM * (32 * TN + 2) * 4 + C::BM * 8 + C::BM * 8 <= NS * C::STAGE,
                      "conv staging exceeds LDS ring");
        __syncthreads();
        epilogue32_glu_dw<TM, TN>(p, acc, (float*)smem, m0, n0, wm, wn, tid, fold, ftab, ecol, dwpre);
    } else if constexpr (EPI == EPI_RELU_TR) {
        if ((32 * TM) % p.trF == 0 && (32 * TN * p.trF) % 8 == 0 && p.N % 8 == 0) {
            static_assert(4 * 32 * TM * (32 * TN + 1) * 4 <= NS * C::STAGE, "epilogue staging exceeds LDS ring");
            __syncthreads();
            float* wsm = (float*)smem + wid * (32 * TM) * (32 * TN + 1);
            epilogue32_relu_tr<TM, TN>(p, acc, wsm, m0 + wm * TM * 32, n0 + wn * TN * 32, lane);
        } else {
            epilogue32<EPI, f16, TM, TN>(p, acc, m0 + wm * TM * 32, n0 + wn * TN * 32, lane);
        }
    } else {
        // the LDS ring is free once every wave has finished its last slab; tiles
        // whose staging exceeds it leave in row halves
        // (the folded-LayerNorm row table sits above the staging area)
        static_assert(whole || (WTM % 2 == 0 && 4 * 16 * WTM * (32 * WTN + 4) * 4 + TAB <= KG * NS * C::STAGE),
                      "epilogue staging exceeds LDS ring");
        if constexpr (KHALF) {
            // eight waves' 32-row staging tiles (the size of four 64-row ones)
            __syncthreads();
            float* wsm = (float*)smem_all + wid_all * 32 * (32 * WTN + 4);
            epilogue32_lds<EPI, 1, WTN>(p, fin, wsm, m0 + erow, n0 + wn * WTN * 32, lane, ecol, fold, ftab, erow,
                                        RPRE ? rpre.v : nullptr,
                                        RPRE && EPI == EPI_RESID_LN && p.res_rows ? rpre.rs : nullptr);
        } else if constexpr (whole) {
            __syncthreads();
            float* wsm = (float*)smem + wid * (32 * WTM) * ((EPI == EPI_GLU ? 16 * WTN : 32 * WTN) + 4);
            if (kg == 0)
                epilogue32_lds<EPI, WTM, WTN>(p, acc, wsm, m0 + wm * WTM * 32, n0 + wn * WTN * 32, lane, ecol,
                                              fold, ftab, wm * WTM * 32, RPRE ? rpre.v : nullptr,
                                              RPRE && EPI == EPI_RESID_LN && p.res_rows ? rpre.rs : nullptr);
        } else {
            constexpr int TH = WTM / 2;
            float* wsm = (float*)smem + wid * (32 * TH) * ((EPI == EPI_GLU ? 16 * WTN : 32 * WTN) + 4);
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                float16v part[TH][WTN];
#pragma unroll
                for (int i = 0; i < TH; ++i)
#pragma unroll
                    for (int j = 0; j < WTN; ++j) part[i][j] = acc[hh * TH + i][j];
                __syncthreads();
                if (kg == 0)
                    epilogue32_lds<EPI, TH, WTN>(p, part, wsm, m0 + wm * WTM * 32 + hh * TH * 32,
                                                 n0 + wn * WTN * 32, lane, ecol, fold, ftab,
                                                 wm * WTM * 32 + hh * TH * 32);
            }
        }
    }
}

// ===========================================================================
// Register-B kernel (gemm_rb_kernel): only the activation tile goes through
// LDS; the weights stream from L2 straight into registers.
//
// NWV waves (4 or 8) side by side along N, each owning 32 WTM rows x 32 WTN
// columns of a (32 WTM) x (NWV 32 WTN) workgroup tile, one workgroup per CU.  A
// wave's weight columns are its own, so each weight is loaded and dequantised
// once per workgroup and never written to or read from LDS; the A tile (BM
// rows x 64 K per slab) arrives by global_load_lds DMA into an NS-stage ring
// and is read by every wave.  LDS bytes per slab: BM*128 written + NWV*BM*128
// read (four waves: 5/BN bytes per flop, the 128 x 128 LDS-B kernel moves
// about 2.4x that; eight waves of 32 columns read the A tile twice as often
// and run two waves per SIMD).
//
// Per slab k one barrier, then the slab k+NS-1 loads are issued (A DMA, B
// register loads; slabs past K read out of range and return zeros, so the
// wait counts never change), then the MFMAs of slab k run interleaved with the
// LDS reads of A(k+1) and the dequantisation of B(k+1) into the other half of
// the double-buffered fragments.  The lane's K order (k = 32q + 8s + e for lane
// half q and substep s) is the LDS-B kernel's: each lane's weight bytes of a
// slab are one contiguous 32-byte run of one q8_0 block.
//
// The weights are the MFMA's A operand and the activations its B operand, with
// A row rho of block j fed from weight column 32 j + tail_col(rho): lane l then
// ends with row 32 i + l % 32 of the tile at the 16 consecutive columns
// 32 j + 16 (l / 32) + r in register r, and the epilogue stores 16-byte pieces
// straight from registers (no LDS staging, one {mean, rstd} per row and lane).
// ===========================================================================

// One wave's raw weight registers for one 64-deep slab: WTN blocks of 32
// columns; lane (q = lane / 32, c = lane % 32) holds column c of each block
// over k = 32q .. 32q + 31 of the slab.
template <int WT, int WTN> struct BRaw;

template <int WTN> struct BRaw<GT_Q8_0, WTN> {
    int4v q[WTN][2];
    uint32_t d[WTN];
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rs, const uint32_t (&vq)[WTN],
                                         const uint32_t (&vs)[WTN], int soq, int sos) {
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            q[j][0] = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)vq[j], soq, 0);
            q[j][1] = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(vq[j] + 16), soq, 0);
            d[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)vs[j], sos, 0);
        }
    }
    __device__ __forceinline__ void convert_j(half8v (&bf)[4], int j, int) const {
        const f16 dh = __builtin_bit_cast(f16, (uint16_t)d[j]);
        const half2v m2 = {dh, dh};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            half2v h0, h1, h2, h3;
            i8x4_to_f16((uint32_t)q[j][s >> 1][2 * (s & 1)], m2, h0, h1);
            i8x4_to_f16((uint32_t)q[j][s >> 1][2 * (s & 1) + 1], m2, h2, h3);
            bf[s] = (half8v){h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
        }
    }
};

// q4_K: both lane halves load the column's 32 nibble bytes (half q takes the
// low (q = 0) or high (q = 1) nibbles) and their own {d*sc, dmin*m} pair.
template <int WTN> struct BRaw<GT_Q4_K, WTN> {
    int4v q[WTN][2];
    float2v s[WTN];
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rs, const uint32_t (&vq)[WTN],
                                         const uint32_t (&vs)[WTN], int soq, int sos) {
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            q[j][0] = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)vq[j], soq, 0);
            q[j][1] = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(vq[j] + 16), soq, 0);
            s[j] = __builtin_bit_cast(float2v, __builtin_amdgcn_raw_buffer_load_b64(rs, (int)vs[j], sos, 0));
        }
    }
    __device__ __forceinline__ void convert_j(half8v (&bf)[4], int j, int q_half) const {
        const half2v m2 = {(f16)s[j].x, (f16)s[j].x};
        const half2v nm2 = {(f16)-s[j].y, (f16)-s[j].y};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            half2v h0, h1, h2, h3;
            nib4_to_f16((uint32_t)q[j][t >> 1][2 * (t & 1)], q_half, m2, nm2, h0, h1);
            nib4_to_f16((uint32_t)q[j][t >> 1][2 * (t & 1) + 1], q_half, m2, nm2, h2, h3);
            bf[t] = (half8v){h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
        }
    }
};

// f16 weights, row-major [N][K]: the lane's 32 halves are 64 contiguous bytes.
template <int WTN> struct BRaw<GT_F16, WTN> {
    int4v q[WTN][4];
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t, const uint32_t (&vq)[WTN],
                                         const uint32_t (&)[WTN], int soq, int) {
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t) q[j][t] = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(vq[j] + 16 * t), soq, 0);
    }
    __device__ __forceinline__ void convert_j(half8v (&bf)[4], int j, int) const {
#pragma unroll
        for (int t = 0; t < 4; ++t) bf[t] = __builtin_bit_cast(half8v, q[j][t]);
    }
};

// f16 weights copied into the conv-module kernel's fragment order
// (glu_frag_prepare): per 64-deep slab and 32-column block, four 1 KB pieces
// [t][lane] of 16 bytes, lane (q, c) holding column c's halves
// k = 32 q + 8 t .. + 7 of the slab, so that each load instruction of a wave
// reads 1 KB contiguous (row-major f16 rows put 32 rows x 2 pieces in every
// instruction: four times the L1 work).  Not a GGML type.
constexpr int GT_F16F = 101;
template <int WTN> struct BRaw<GT_F16F, WTN> {
    int4v q[WTN][4];
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t, const uint32_t (&vq)[WTN],
                                         const uint32_t (&)[WTN], int soq, int) {
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t) q[j][t] = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(vq[j] + 1024 * t), soq, 0);
    }
    __device__ __forceinline__ void convert_j(half8v (&bf)[4], int j, int) const {
#pragma unroll
        for (int t = 0; t < 4; ++t) bf[t] = __builtin_bit_cast(half8v, q[j][t]);
    }
};

// Conv-module item tiles: the weight row (GEMM column) of wave column c
// (0 .. 31) of wave wid in column tile bn.  The weights hold 32-row groups of
// GLU inputs and gates alternately; the wave takes channels c0 .. c0 + 15
// (c0 = 64 bn + 16 wid): columns 0 .. 15 their inputs, 16 .. 31 their gates.
__device__ __forceinline__ int glu_wcol(int bn, int wid, int c) {
    const int c0 = 64 * bn + 16 * wid;
    return 2 * c0 - (c0 & 31) + (c & 15) + 32 * (c >> 4);
}

// Vector-memory instructions of one slab's weight loads per wave.
template <int WT, int WTN>
constexpr int rb_b_ops() { return WT == GT_F16 || WT == GT_F16F ? 4 * WTN : 3 * WTN; }

// Register-B epilogue: lane l holds row 32 i + l % 32 of the tile at columns
// nw + 32 j + 16 (l / 32) + r in acc[i][j][r].  y = alpha (acc + bias), with a
// folded LayerNorm alpha (rstd (acc - mean c1) + bias) as two FMAs
// (a = alpha rstd, nb = -a mean per row; c1 and alpha * bias per column from
// ctab), SiLU for EPI_SILU (alpha 1); f16 (or f32) pieces of 16 bytes by raw
// buffer stores, rows past M and columns past N out of range (N % 16 == 0).
template <int EPI, int WTM, int WTN>
__device__ __forceinline__ void epilogue_rb(const GemmParams& p, const float16v (&acc)[WTM][WTN], const float* ctab,
                                            int m0, int nw, int lane, float alpha, bool fold, const float2v* ftab) {
    constexpr int WC = 32 * WTN, ESZ = EPI == EPI_STORE_F32 ? 4 : 2;
    const int r32 = lane & 31, h = lane >> 5;
    const int rows = p.M - m0;   // >= 1
    const __amdgpu_buffer_rsrc_t ry =
        make_rsrc((const uint8_t*)p.Y + (int64_t)m0 * p.ldy * ESZ, ((int64_t)(rows - 1) * p.ldy + p.N) * ESZ);
    float4v cb[WTN][4], cc[WTN][4];
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            cb[j][t] = *(const float4v*)(ctab + 32 * j + 16 * h + 4 * t);
            cc[j][t] = fold ? *(const float4v*)(ctab + WC + 32 * j + 16 * h + 4 * t) : (float4v){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
    for (int i = 0; i < WTM; ++i) {
        const int row = 32 * i + r32;
        float a = alpha, nb = 0.f;
        if (fold) {
            const float2v st = ftab[row];
            a = alpha * st.y;
            nb = -a * st.x;
        }
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            const int n = nw + 32 * j + 16 * h;
            const uint32_t off = row < rows && n < p.N ? (uint32_t)((row * p.ldy + n) * ESZ) : OOB;
            float y[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float b = fold ? __builtin_fmaf(nb, cc[j][r >> 2][r & 3], cb[j][r >> 2][r & 3]) : cb[j][r >> 2][r & 3];
                float v = __builtin_fmaf(a, acc[i][j][r], b);
                if constexpr (EPI == EPI_SILU) v = silu_dev(v);
                y[r] = v;
            }
            if constexpr (EPI == EPI_STORE_F32) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float4v v4 = {y[4 * t], y[4 * t + 1], y[4 * t + 2], y[4 * t + 3]};
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(int4v, v4), ry, off + 16 * t, 0, 0);
                }
            } else {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    half8v hv;
#pragma unroll
                    for (int e = 0; e < 8; ++e) hv[e] = (f16)y[8 * t + e];
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(int4v, hv), ry, off + 16 * t, 0, 0);
                }
            }
        }
    }
}

// Register-B epilogue of the residual products (two K groups, each wave
// finishing one 32-row block): lane l holds row mb + l % 32 at columns
// nw + 32 j + 16 (l / 32) + r in acc[j][r].  alpha (acc + bias) is staged in
// LDS (wsm: 32 rows of 32 WTN + 4 floats, four 16-byte writes per lane and
// block) and leaves through the coalesced residual copy-out (epilogue_lds_out:
// x += (.), and for RESID_LN x * gamma and the 32-column group statistics),
// whose full-line stores and residual loads take a quarter of the requests of
// 16-byte pieces on 32 rows.  ctab: the wave's 32 WTN columns of alpha * bias.
template <int EPI, int WTN>
__device__ __forceinline__ void epilogue_rb_resid(const GemmParams& p, const float16v (&acc)[WTN], const float* ctab,
                                                  float* wsm, int mb, int nw, int lane, float alpha,
                                                  const EpiCols<WTN>& ec, const float4v* xpre, const float2v* xrs) {
    constexpr int WC = 32 * WTN, LDW = WC + 4;
    const int r32 = lane & 31, h = lane >> 5;
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
        const int c = 32 * j + 16 * h;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float4v b4 = *(const float4v*)(ctab + c + 4 * t);
            float4v v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __builtin_fmaf(alpha, acc[j][4 * t + e], b4[e]);
            *(float4v*)(wsm + r32 * LDW + c + 4 * t) = v;
        }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    epilogue_lds_out<EPI, 32, WC, WTN>(p, wsm, mb, nw, lane, ec, xpre, xrs);
}

// Register-B conv-module epilogue (item tiles of 128 rows x 64 channels: tile
// row r is frame tb + r of item `item`, the tile writes frames [tlo, thi)):
// K group kg holds the summed rows 64 kg +
// 32 ii + l % 32 in fin[ii], lane half l / 32 the inputs (0) or the gates (1)
// of the wave's 16 channels in registers 0 .. 15.  One lane-half swap per
// register pair hands each lane the input and the gate of channel
// 16 wid + 8 (l / 32) + e; the GLU (folded LayerNorm, bias, a * sigmoid(b))
// with the pad mask (frames t >= valid are zero, and with them the next
// item's rows) goes into G [128][LDG] f32 in LDS.  Then the depthwise conv
// over time (zero rows outside the item's valid frames: frames before tb are
// outside the item), its bias, the folded BatchNorm and SiLU for frames
// [tlo, thi): thread tid takes the channel pair 2 (tid % 32) and rows
// 8 (tid / 32) .. + 7, its 16-row window in registers, and stores f16 pairs
// (conformer.cpp:55-157).
template <int LDG, bool FOLD>
__device__ __forceinline__ void epilogue_rb_glu_dw(const GemmParams& p, const float16v (&fin)[2][1], const float* ctab,
                                                   const float2v* ftab, float* G, int m0, int item, int tb, int tlo,
                                                   int thi, int n0, int kg, int wid, int lane, int tid, float4v taps4,
                                                   const float2v (&dwc)[3]) {
    constexpr int K = GLU_DW_K, H = (K - 1) / 2, RPT = 8;
    // the tile's taps [64][K] past the GLU tile (thread tid < 144 brought 16 bytes)
    float* taps = G + 128 * LDG;
    if (tid < 64 * K / 4) ((float4v*)taps)[tid] = taps4;
    const int h = lane >> 5, r32 = lane & 31;
    const int T = p.T;
    const int vl = p.valid ? min(p.valid[item], T) : T;
    float4v bi[2], bg[2], ci[2], cg[2];   // input / gate bias, input / gate c1 of the lane's 8 channels
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        bi[t] = *(const float4v*)(ctab + 8 * h + 4 * t);
        bg[t] = *(const float4v*)(ctab + 16 + 8 * h + 4 * t);
        ci[t] = *(const float4v*)(ctab + 32 + 8 * h + 4 * t);
        cg[t] = *(const float4v*)(ctab + 48 + 8 * h + 4 * t);
    }
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int row = 64 * kg + 32 * ii + r32;
        // the pad mask as a bit mask (no branch around the sigmoid)
        const uint32_t keep = tb + row < vl ? 0xffffffffu : 0u;
        float a = 1.f, nb = 0.f;
        if constexpr (FOLD) {
            const float2v st = ftab[row];
            a = st.y;
            nb = -a * st.x;
        }
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(fin[ii][0][e]),
                                                             __float_as_uint(fin[ii][0][8 + e]), false, false);
            const float xa = __uint_as_float(sw[0]), xg = __uint_as_float(sw[1]);
            float va, vg;
            if constexpr (FOLD) {
                va = __builtin_fmaf(a, xa, __builtin_fmaf(nb, ci[e >> 2][e & 3], bi[e >> 2][e & 3]));
                vg = __builtin_fmaf(a, xg, __builtin_fmaf(nb, cg[e >> 2][e & 3], bg[e >> 2][e & 3]));
            } else {
                va = xa + bi[e >> 2][e & 3];
                vg = xg + bg[e >> 2][e & 3];
            }
            o[e] = __uint_as_float(__float_as_uint(va * sigmoid_dev(vg)) & keep);
        }
        float* gr = G + row * LDG + 16 * wid + 8 * h;
        *(float4v*)gr = (float4v){o[0], o[1], o[2], o[3]};
        *(float4v*)(gr + 4) = (float4v){o[4], o[5], o[6], o[7]};
    }
    __syncthreads();
    const int cl = 2 * (tid & 31), r0 = RPT * (tid >> 5), c = n0 / 2 + cl;
    float2v wk[K];
#pragma unroll
    for (int j = 0; j < K; ++j) wk[j] = (float2v){taps[cl * K + j], taps[(cl + 1) * K + j]};
    float2v win[RPT + K - 1];
#pragma unroll
    for (int q = 0; q < RPT + K - 1; ++q) {
        const int row = r0 - H + q;
        win[q] = row >= 0 && row < 128 ? *(const float2v*)(G + row * LDG + cl) : (float2v){0.f, 0.f};
    }
    // frames [tlo, thi): 4-byte stores at 32-bit offsets from the tile's
    // first row (other rows out of range)
    const __amdgpu_buffer_rsrc_t ry = make_rsrc((const f16*)p.Y + (int64_t)m0 * p.ldy, ((int64_t)(thi - tb) * p.ldy) * 2);
    const uint32_t off0 = (uint32_t)((r0 * p.ldy + c) * 2), ldb = (uint32_t)(p.ldy * 2);
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
        float2v acc = {0.f, 0.f};
#pragma unroll
        for (int j = 0; j < K; ++j) acc += wk[j] * win[q + j];
        const float2v y = (acc + dwc[0]) * dwc[1] + dwc[2];
        const half2v hv = {(f16)silu_dev(y[0]), (f16)silu_dev(y[1])};
        const int t = tb + r0 + q;
        const uint32_t off = t >= tlo && t < thi ? off0 + q * ldb : OOB;
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, hv), ry, off, 0, 0);
    }
}

// KG = 2: eight waves in two groups of four; group g streams K slabs
// [g nk, (g+1) nk) through its own ring, and after the main loop group g sums
// and finishes row block g of the 64-row tile (the other group's partial of
// it comes through LDS): two waves per SIMD for grids of about one tile per
// CU.  Used with the residual epilogues on 64 x 128 tiles.
// NWV = 8: eight waves side by side along N (one K group), two per SIMD, each
// reading its slab's activation fragments within the slab (a two-step
// buffer) instead of one slab ahead, which the registers of two waves per
// SIMD cannot hold; the other wave on the SIMD covers the LDS latency.
// EPI_GLU_DW (the conformer conv module after pointwise_conv1): one item of
// T <= 128 frames per 128-row tile, 64 channels (their 64 input and 64 gate
// columns) per tile, two K groups; the depthwise conv never crosses an item,
// so the tile needs no halo rows.
template <int WTM, int WTN, int WT, int EPI, int NS, bool FO = false, int KG = 1, int NWV = 4>
struct RbCfg {
    static constexpr int BM = 32 * WTM, BN = NWV * 32 * WTN, WC = 32 * WTN;
    static constexpr int NT = 64 * NWV * KG;                  // threads
    static constexpr bool GD = EPI == EPI_GLU_DW;             // item tiles, GLU + depthwise epilogue
    static constexpr bool SB = NWV == 8 || GD;                // fragments read within their slab
    static constexpr int A_STAGE = BM * 128;                  // f16 [BM][64]
    static constexpr int NA = A_STAGE / (NWV * 1024);         // 1 KB A DMAs per wave per slab
    static constexpr int NB = rb_b_ops<WT, WTN>();
    static constexpr int PER_SLAB = NA + NB;
    static constexpr int NR = 4;                              // weight register sets (>= NS - 1 in flight)
    static constexpr int U = 4;                               // loop unroll: every ring index static
    static constexpr bool RESID = EPI == EPI_RESID || EPI == EPI_RESID_LN;
    static constexpr bool FOLD = FO && (EPI == EPI_STORE || EPI == EPI_SILU || GD);
    static constexpr int NCA = RESID ? 1 : 2;                 // column constant arrays
    static constexpr int RING = KG * NS * A_STAGE;
    static constexpr int FOLD_BYTES = FOLD ? BM * 32 * 8 : 0; // {mean, M2} of up to 32 groups per row
    static constexpr int XCH = KG == 2 ? 8 * (WTM / 2) * 16 * WTN * 64 * 4 : 0;   // K-group exchange
    static constexpr int CTAB = NWV * KG * NCA * WC * 4;      // epilogue column constants
    static constexpr int LDG = 64 + 4;                        // GLU staging row (floats, GD)
    static constexpr int TAPS = GD ? 64 * GLU_DW_K * 4 : 0;   // the tile's depthwise taps (GD)
    static constexpr int STG = RESID ? 8 * 32 * (WC + 4) * 4 : GD ? BM * LDG * 4 + TAPS : 0;   // epilogue staging
    static constexpr int AFTER = XCH + CTAB + STG;            // the post-loop regions, from offset 0
    static constexpr int BODY = (RING > AFTER ? RING : AFTER) + FOLD_BYTES;
    // the row table {mean, rstd}: past the body, or (GD) over the start of the
    // fold statistics, once they are in registers
    static constexpr int FTAB = GD && FOLD ? BODY - FOLD_BYTES : BODY;
    static constexpr int LDS = GD && FOLD ? BODY : BODY + BM * 8;
    static_assert(A_STAGE % (NWV * 1024) == 0, "A slab splits into 1 KB DMAs per wave");
    static_assert(NWV == 4 || (NWV == 8 && KG == 1 && !RESID), "eight waves: one K group, store / SiLU");
    static_assert(!FOLD || AFTER <= RING, "the fold statistics sit past the ring");
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(KG == 1 || KG == 2, "K groups");
    static_assert(!RESID || (KG == 2 && WTM == 2), "residual epilogues: two K groups, one row block per group");
    static_assert(!GD || (KG == 2 && WTM == 4 && WTN == 1 && NWV == 4), "conv module: 128 x 128 item tiles, two K groups");
    static_assert(WT != GT_F16F || GD, "fragment-ordered f16 weights: conv-module kernel only");
    static_assert(RESID || GD || KG == 1, "store / SiLU epilogues: one K group");
    static_assert(!FOLD || KG == 1 || GD, "folded LayerNorm: one K group (or the conv module)");
};

template <int WTM, int WTN, int WT, int EPI, int NS, bool FO = false, int KG = 1, int NWV = 4>
__global__ __launch_bounds__(64 * NWV * KG, 1) void gemm_rb_kernel(GemmParams p) {
    typedef RbCfg<WTM, WTN, WT, EPI, NS, FO, KG, NWV> C;
    static_assert(NS >= 3 && NS <= 5, "ring depth");
    static_assert(EPI == EPI_STORE || EPI == EPI_STORE_F32 || EPI == EPI_SILU || C::RESID || C::GD,
                  "register-B kernel: store / SiLU / residual / conv-module epilogues");
    constexpr int BM = C::BM, NR = C::NR, WC = C::WC;
    constexpr bool GD = C::GD;
    __shared__ __attribute__((aligned(1024))) uint8_t smem_all[C::LDS];

    const int tid = threadIdx.x, lane = tid & 63, wid_all = wave_id_uniform();
    const int kg = KG == 2 ? wid_all >> 2 : 0, wid = KG == 2 ? wid_all & 3 : wid_all;
    const int q = lane >> 5, r32 = lane & 31;
    uint8_t* smem = smem_all + kg * NS * C::A_STAGE;   // this group's ring
    int bm, bn;
    // conv module: item tiles.  An item of T <= 128 frames is one row tile
    // (tile row r = frame r; the rest of the 128 rows belong to the next item
    // or lie past M and are masked); a longer item is cut into nti parts of at
    // most 120 output frames [tlo, thi), a part after the first starting 4
    // frames early (tile row r = frame tb + r) so that its 128 rows hold the
    // depthwise conv's halo on both sides.
    int item = 0, tb = 0, tlo = 0, thi = 0;
    if constexpr (GD) {
        constexpr int HALO = (GLU_DW_K - 1) / 2;
        const int T = p.T, nti = T <= 128 ? 1 : (T + 127 - 2 * HALO) / (128 - 2 * HALO);
        const int orows = udiv_small(T + nti - 1, nti);
        xcd_tile_2d(blockIdx.x, p.M / T * nti, cdiv_dev(p.N, C::BN), p.xcd_gm, bm, bn);
        item = udiv_small(bm, nti);
        const int part = bm - item * nti;
        tlo = part * orows;
        thi = min(tlo + orows, T);
        tb = part > 0 ? tlo - HALO : 0;
    } else {
        xcd_tile_2d(blockIdx.x, cdiv_dev(p.M, BM), cdiv_dev(p.N, C::BN), p.xcd_gm, bm, bn);
    }
    const int m0 = GD ? item * p.T + tb : bm * BM, n0 = bn * C::BN, nw = n0 + wid * WC;
    const int nkt = p.K / 64, nk = nkt / KG, kb = kg * nk;   // slabs: all, this group's, its first
    // weight column of the wave's column c (0 .. WC-1); conv module: lanes l
    // and l + 32 end with the input and the gate of the same 16 channels
    auto wcol = [&](int c) -> int {
        if constexpr (GD) return glu_wcol(bn, wid, c);
        else return nw + c;
    };

    // folded LayerNorm (FO: p.fold_stats is set) statistics of the tile's rows:
    // DMA into LDS first (the oldest vector-memory operations, complete by the
    // first slab's wait)
    constexpr bool fold = C::FOLD;
    if constexpr (fold) {
        const int lc = __builtin_ctz(p.fold_groups / 2), total = BM << lc;   // 16-byte chunks
        const __amdgpu_buffer_rsrc_t rf =
            make_rsrc((const float2v*)p.fold_stats + (int64_t)m0 * p.fold_groups,
                      ((int64_t)(p.M - m0) * p.fold_groups) * 8);
        uint8_t* fl = smem_all + C::BODY - C::FOLD_BYTES;
        for (int c0 = wid_all * 64; c0 < total; c0 += 64 * NWV * KG) {
            const int ch = c0 + lane, r = ch >> lc;
            const uint32_t off = ch < total ? (uint32_t)(min(r, p.M - 1 - m0) << (lc + 4)) + ((ch & ((1 << lc) - 1)) << 4)
                                            : OOB;
            lds_dma16(rf, fl + c0 * 16, off, 0);
        }
    }
    // the epilogue's column constants of column nw + lane + 64 t (written to
    // LDS after the main loop): alpha * bias, then the fold's c1 (store / SiLU)
    const float alpha = EPI == EPI_SILU || GD ? 1.f : p.alpha;
    constexpr int CPL = (WC + 63) / 64;
    float colv[C::NCA][CPL];
    // conv module: the depthwise bias and folded BatchNorm of this thread's
    // channel pair 64 bn + 2 (tid % 32) (the taps come through LDS later)
    float2v dwc[3];
    // residual epilogues: the wave's 32-row block of the residual stream (row
    // block kg of the tile) in the copy-out's layout, its rows' statistics
    // and the copy-out's columns of gamma, res_g, res_b, in registers before
    // the main loop
    constexpr bool RS = EPI == EPI_RESID_LN;
    ResidPre<C::RESID ? 32 : 64, C::RESID ? 8 * WTN : 1, RS> rpre;
    EpiCols<WTN> ecol;
    // issued right behind slab 0's loads, so that those go out first (ahead
    // of them the second K group's slab 0 waited ~2k cycles behind the first
    // group's operand loads); the first slab wait covers them (they are older
    // than slab 1's loads)
    auto load_epi_operands = [&]() {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            const int c = lane + 64 * t, n = wcol(c);
            const bool ok = c < WC && n < p.N;
            colv[0][t] = ok && p.bias ? p.bias[n] : 0.f;   // times alpha when written to LDS
            if constexpr (C::NCA == 2) colv[1][t] = fold && ok ? p.fold_c1[n] : 0.f;
        }
        if constexpr (C::RESID) {
            rpre.load(p, m0 + 32 * kg, nw, lane);
            ecol.load(p, nw, lane, false, RS);
        }
        if constexpr (GD) {
            const int c = n0 / 2 + 2 * (tid & 31);
            dwc[0] = p.dw_b ? (float2v){p.dw_b[c], p.dw_b[c + 1]} : (float2v){0.f, 0.f};
            dwc[1] = (float2v){p.dw_scale[c], p.dw_scale[c + 1]};
            dwc[2] = (float2v){p.dw_shift[c], p.dw_shift[c + 1]};
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // A: 64-column slabs of rows m0.., swizzled 16-byte chunks (as DmaSrc)
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc((const f16*)p.A + (int64_t)m0 * p.lda, ((int64_t)(p.M - m0 - 1) * p.lda + p.K) * 2);
    uint32_t va[C::NA];
#pragma unroll
    for (int i = 0; i < C::NA; ++i) {
        const int slot = (wid * C::NA + i) * 64 + lane;
        const int row = slot >> 3, c = (slot & 7) ^ ((row >> 1) & 7);
        const int m = min(m0 + row, p.M - 1) - m0;
        va[i] = (uint32_t)(((int64_t)m * p.lda + 8 * c) * 2);
    }
    // weights: per block j the lane's byte offset in slab 0 (columns past N: out of range)
    const int L = slab_rows(p);
    __amdgpu_buffer_rsrc_t rq = make_rsrc(p.Wq, 0), rs = rq;
    uint32_t vq[WTN], vs[WTN];
    if constexpr (WT == GT_Q8_0 || WT == GT_Q4_K) {
        constexpr int WB = WT == GT_Q8_0 ? 64 : 32, SB = WT == GT_Q8_0 ? 4 : 16;
        // a view into a larger weight keeps the allocation's slab stride L: its
        // last byte is in slab nk-1, row N-1
        rq = make_rsrc(p.Wq, ((int64_t)(nkt - 1) * L + p.N) * WB);
        rs = make_rsrc(p.Ws, ((int64_t)(nkt - 1) * L + p.N) * SB);
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            const int n = wcol(32 * j + tail_col(r32));
            vq[j] = n < p.N ? (uint32_t)(n * WB + (WT == GT_Q8_0 ? 32 * q : 0)) : OOB;
            vs[j] = n < p.N ? (uint32_t)(n * SB + (WT == GT_Q8_0 ? 2 * q : 8 * q)) : OOB;
        }
    } else if constexpr (WT == GT_F16F) {
        // [slab][block of 32 columns][t][lane] pieces; this wave's block is
        // 4 bn + wid (the fragment copy is in the kernel's column order)
        rq = make_rsrc(p.Wq, (int64_t)p.N * p.K * 2);
        vq[0] = (uint32_t)(((4 * bn + wid) * 256 + lane) * 16);
        vs[0] = 0;
    } else {
        rq = make_rsrc(p.Wq, (int64_t)p.N * p.K * 2);
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            const int n = wcol(32 * j + tail_col(r32));
            vq[j] = n < p.N ? (uint32_t)(((int64_t)n * p.K + 32 * q) * 2) : OOB;
            vs[j] = 0;
        }
    }
    // scalar offsets of the group's slab k (out of range past its last slab)
    auto soq = [&](int k) -> int {
        if (k >= nk) return (int)OOB;
        return WT == GT_Q8_0 ? (kb + k) * L * 64 : WT == GT_Q4_K ? (kb + k) * L * 32
             : WT == GT_F16F ? (kb + k) * p.N * 128 : (kb + k) * 128;
    };
    auto sos = [&](int k) -> int {
        if (k >= nk) return (int)OOB;
        return WT == GT_Q8_0 ? (kb + k) * L * 4 : WT == GT_Q4_K ? (kb + k) * L * 16 : 0;
    };
    auto issue_a = [&](int k) {
        uint8_t* st = smem + (k % NS) * C::A_STAGE + wid * C::NA * 1024;
        const int so = k < nk ? (kb + k) * 128 : (int)OOB;
#pragma unroll
        for (int i = 0; i < C::NA; ++i) lds_dma16(ra, st + i * 1024, va[i], so);
    };

    float16v acc[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j) acc[i][j] = (float16v){};

    BRaw<WT, WTN> braw[NR];
    half8v af[2][4][WTM], bf[2][WTN][4];
    auto read_a = [&](half8v (&a)[4][WTM], int k) {
        const uint8_t* st = smem + (k % NS) * C::A_STAGE;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < WTM; ++i) {
                const int row = 32 * i + r32;
                a[s][i] = *(const half8v*)(st + row * 128 + (((4 * q + s) ^ ((row >> 1) & 7)) << 4));
            }
    };

    if constexpr (C::SB) {
        // slabs 0 .. NS-2 in flight; per slab: wait for it, one barrier, issue
        // slab k+NS-1, dequantise slab k's weights, then its MFMAs with the A
        // fragments of step s+1 read under those of step s
#pragma unroll
        for (int k = 0; k < NS - 1; ++k) {
            issue_a(k);
            braw[k % NR].load(rq, rs, vq, vs, soq(k), sos(k));
            if (k == 0) load_epi_operands();
        }
        for (int k0 = 0; k0 < nk; k0 += C::U) {
#pragma unroll
            for (int u = 0; u < C::U; ++u) {
                const int k = k0 + u;
                __builtin_amdgcn_sched_barrier(0);
                wait_vmcnt<(NS - 2) * C::PER_SLAB>();   // slab k has landed
                __builtin_amdgcn_s_barrier();
                issue_a(k + NS - 1);
                braw[(u + NS - 1) % NR].load(rq, rs, vq, vs, soq(k + NS - 1), sos(k + NS - 1));
                half8v b1[WTN][4], a2[2][WTM];
#pragma unroll
                for (int j = 0; j < WTN; ++j) braw[u % NR].convert_j(b1[j], j, q);
                const uint8_t* st = smem + (k % NS) * C::A_STAGE;
                auto read_step = [&](half8v (&a)[WTM], int s2) {
#pragma unroll
                    for (int i = 0; i < WTM; ++i) {
                        const int row = 32 * i + r32;
                        a[i] = *(const half8v*)(st + row * 128 + (((4 * q + s2) ^ ((row >> 1) & 7)) << 4));
                    }
                };
                read_step(a2[0], 0);
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) {
                    if (s2 < 3) read_step(a2[(s2 + 1) & 1], s2 + 1);
#pragma unroll
                    for (int i = 0; i < WTM; ++i)
#pragma unroll
                        for (int j = 0; j < WTN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b1[j][s2], a2[s2 & 1][i], acc[i][j], 0, 0, 0);
                }
            }
        }
    } else {
        // prologue: slabs 0 .. NS-3 issued; once slab 0 has landed it goes into
        // registers and slab NS-2 is issued behind it (the loop starts with
        // slabs 1 .. NS-2 in flight).  Issuing slab NS-2 first kept every wave
        // issuing loads for ~0.9k cycles after slab 0 had arrived.
    #pragma unroll
        for (int k = 0; k < NS - 2; ++k) {
            issue_a(k);
            braw[k % NR].load(rq, rs, vq, vs, soq(k), sos(k));
            if (k == 0) load_epi_operands();
        }
        wait_vmcnt<(NS - 3) * C::PER_SLAB>();
        __builtin_amdgcn_s_barrier();
        read_a(af[0], 0);
    #pragma unroll
        for (int j = 0; j < WTN; ++j) braw[0].convert_j(bf[0][j], j, q);
        issue_a(NS - 2);
        braw[(NS - 2) % NR].load(rq, rs, vq, vs, soq(NS - 2), sos(NS - 2));

        // nk % U == 0 (checked on the host): the ring indices of slab k are u-static
        for (int k0 = 0; k0 < nk; k0 += C::U) {
    #pragma unroll
            for (int u = 0; u < C::U; ++u) {
                const int k = k0 + u;
                // No instruction crosses a slab boundary: the scheduler would
                // otherwise fill the slab's VALU slots with the next slab's
                // dequantisation, whose weights were loaded only one slab ago
                // (a wait on them that empties the read-ahead).
                __builtin_amdgcn_sched_barrier(0);
                // slab k+1 (A in LDS from every wave, B in this wave's registers) has landed
                wait_vmcnt<(NS - 3) * C::PER_SLAB>();
                __builtin_amdgcn_s_barrier();
                issue_a(k + NS - 1);
                braw[(u + NS - 1) % NR].load(rq, rs, vq, vs, soq(k + NS - 1), sos(k + NS - 1));
                const int cu = u & 1, nx = cu ^ 1;
                // the MFMAs of slab k, with the next slab's A reads and weight
                // dequantisation interleaved (one MFMA, then an LDS read or four VALU)
                read_a(af[nx], k + 1);
    #pragma unroll
                for (int j = 0; j < WTN; ++j) braw[(u + 1) % NR].convert_j(bf[nx][j], j, q);
    #pragma unroll
                for (int s = 0; s < 4; ++s)
    #pragma unroll
                    for (int i = 0; i < WTM; ++i)
    #pragma unroll
                        for (int j = 0; j < WTN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[cu][j][s], af[cu][s][i], acc[i][j], 0, 0, 0);
    #pragma unroll
                for (int g = 0; g < 4 * WTM * WTN; ++g) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    if (g < 4 * WTM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
                }
            }
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    // conv module: the tile's 64 x 9 depthwise taps ([channel][tap], contiguous
    // in dw_w) by 144 lanes, into LDS in the epilogue
    float4v taps4 = {0.f, 0.f, 0.f, 0.f};
    if constexpr (GD) {
        if (tid < 64 * GLU_DW_K / 4) taps4 = *((const float4v*)(p.dw_w + (int64_t)(n0 / 2) * GLU_DW_K) + tid);
    }

    // folded LayerNorm: {mean, rstd} of the tile's rows (past the body, or
    // over the start of the statistics once they are in registers)
    float2v* ftab = (float2v*)(smem_all + C::FTAB);
    if constexpr (fold) {
        // the table is built by every thread of the workgroup
        constexpr int FT = C::NT;
        FoldStats<BM, FT> fst;
        const int lc = __builtin_ctz(p.fold_groups / 2), total = BM << lc;
        if (tid < FT) {
#pragma unroll
            for (int i = 0; i < FoldStats<BM, FT>::MAXC; ++i) {
                const int ch = tid + FT * i;
                fst.c[i] = ch < total ? ((const float4v*)(smem_all + C::BODY - C::FOLD_BYTES))[ch]
                                      : (float4v){0.f, 0.f, 0.f, 0.f};
            }
        }
        if constexpr (C::FTAB != C::BODY) __syncthreads();   // the table overwrites the statistics
        if (tid < FT) fst.finish(p, ftab, tid);
        __syncthreads();
    }
    // two K groups: group g finishes row blocks HB g .. HB g + HB - 1; its
    // partial of the other group's blocks goes to that group, which adds it to
    // its own (lane-major [wave][register][lane] f32)
    constexpr int HB = KG == 2 ? WTM / 2 : 1;
    float16v fin[HB][WTN];
    if constexpr (KG == 2) {
        // [wave][register / 4][lane] float4s: 16-byte accesses, 1 KB per instruction
        constexpr int R = 16 * WTN * HB;
        float4v* give = (float4v*)smem_all + wid_all * (R / 4) * 64 + lane;
        const float4v* take = (const float4v*)smem_all + ((1 - kg) * 4 + wid) * (R / 4) * 64 + lane;
#pragma unroll
        for (int ii = 0; ii < HB; ++ii)
#pragma unroll
            for (int j = 0; j < WTN; ++j)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    float4v g;
#pragma unroll
                    for (int e = 0; e < 4; ++e) g[e] = kg ? acc[ii][j][4 * t + e] : acc[HB + ii][j][4 * t + e];
                    give[((ii * WTN + j) * 4 + t) * 64] = g;
                }
        __syncthreads();
#pragma unroll
        for (int ii = 0; ii < HB; ++ii)
#pragma unroll
            for (int j = 0; j < WTN; ++j)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float4v o = take[((ii * WTN + j) * 4 + t) * 64];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        fin[ii][j][4 * t + e] = (kg ? acc[HB + ii][j][4 * t + e] : acc[ii][j][4 * t + e]) + o[e];
                }
    }
    // this wave's column constants (the ring is free; past the exchange):
    // written and read by the wave alone
    float* ctab = (float*)(smem_all + C::XCH) + wid_all * C::NCA * WC;
    float* wsm = (float*)(smem_all + C::XCH + C::CTAB) + wid_all * 32 * (WC + 4);
#pragma unroll
    for (int a = 0; a < C::NCA; ++a)
#pragma unroll
        for (int t = 0; t < CPL; ++t)
            if (lane + 64 * t < WC) ctab[a * WC + lane + 64 * t] = a == 0 ? alpha * colv[a][t] : colv[a][t];
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    if constexpr (C::RESID)
        epilogue_rb_resid<EPI, WTN>(p, fin[0], ctab, wsm, m0 + 32 * kg, nw, lane, alpha, ecol, rpre.v,
                                    RS && p.res_rows ? rpre.rs : nullptr);
    else if constexpr (GD)
        epilogue_rb_glu_dw<C::LDG, fold>(p, fin, ctab, ftab, (float*)(smem_all + C::XCH + C::CTAB), m0, item, tb,
                                         tlo, thi, n0, kg, wid, lane, tid, taps4, dwc);
    else epilogue_rb<EPI, WTM, WTN>(p, acc, ctab, m0, nw, lane, alpha, fold, ftab);
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
                const int64_t blk = (int64_t)(k0 / 64) * slab_rows(p) + n;   // slab-major
                v = *(const int4v*)(W + blk * 64 + (k0 & 63) + 16 * h);
                s = (float)S[blk * 2 + ((k0 & 63) >> 5)];
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
        // 32-element sub-block k0: the low nibbles of its slab block's 32 bytes if
        // k0 % 64 == 0, else the high nibbles
        const int hi = (k0 & 32) ? 1 : 0;
        shift = hi * 4;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 1, h = c & 1;
            const int n = n0 + row;
            int4v v = {};
            float2v sc = {0.f, 0.f};
            if (c < BN * 2 && n < p.N && k0 < p.K) {
                const int64_t blk = (int64_t)(k0 / 64) * slab_rows(p) + n;   // slab-major
                v = *(const int4v*)(W + blk * 32 + 16 * h);
                sc = S[blk * 2 + hi];
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
    constexpr int PF = TM * TN >= 16 ? 1 : 2;
    const int tiles = cdiv(p.M, 32 * TM) * cdiv(p.N, 32 * TN);
    launch((gemm_f16_kernel<TM, TN, WT, EPI, PF>), dim3(tiles), dim3(256), 0, s, p);
    PKX_LAUNCH_CHECK();
}
template <int TM, int TN, int WT, int EPI>
static void run_f32(const GemmParams& p, hipStream_t s) {
    const int tiles = cdiv(p.M, 32 * TM) * cdiv(p.N, 32 * TN);
    launch((gemm_f32_kernel<TM, TN, WT, EPI>), dim3(tiles), dim3(256), 0, s, p);
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
// the LDS-DMA kernel also has the residual + LayerNorm-statistics epilogue
#define PKX_EPI_SWITCH_DMA(RUN, TM, TN, WT)                                     \
    switch (epi) {                                                              \
    case EPI_STORE: RUN<TM, TN, WT, EPI_STORE>(p, s); break;                    \
    case EPI_STORE_F32: RUN<TM, TN, WT, EPI_STORE_F32>(p, s); break;            \
    case EPI_SILU: RUN<TM, TN, WT, EPI_SILU>(p, s); break;                      \
    case EPI_RESID: RUN<TM, TN, WT, EPI_RESID>(p, s); break;                    \
    case EPI_GLU: RUN<TM, TN, WT, EPI_GLU>(p, s); break;                        \
    case EPI_RELU: RUN<TM, TN, WT, EPI_RELU>(p, s); break;                      \
    case EPI_RELU_TR: RUN<TM, TN, WT, EPI_RELU_TR>(p, s); break;                \
    case EPI_RELU2_F32: RUN<TM, TN, WT, EPI_RELU2_F32>(p, s); break;            \
    case EPI_RESID_LN: RUN<TM, TN, WT, EPI_RESID_LN>(p, s); break;              \
    default: throw std::invalid_argument("gemm: bad epilogue");                 \
    }

// Row/column band split of the tile grid over the 8 XCDs that minimises the
// L2-miss bytes gn*|A| + gm*|W| (each XCD reads its A band and its W band).
static int choose_xcd_gm(const GemmParams& p, int WT, int BM, int BN) {
    const int nbm = cdiv(p.M, BM), nbn = cdiv(p.N, BN);   // BM: output rows per tile
    const double a_bytes = (double)p.M * p.K * 2;
    const double w_bytes = (double)p.N * p.K * (WT == GT_Q8_0 ? 34.0 / 32 : WT == GT_Q4_K ? 0.75 : 2.0);
    int best = 1;
    double best_cost = 1e300;
    for (int gm : {1, 2, 4, 8}) {
        const int gn = 8 / gm;
        if (gm > nbm || gn > nbn) continue;
        const double cost = gn * a_bytes + gm * w_bytes;
        if (cost < best_cost) {
            best_cost = cost;
            best = gm;
        }
    }
    return best_cost < 1e300 ? best : 1;
}

template <int TM, int TN, int WT, int EPI, int NS = DMA_NS, int KG = 1, int WL = 0>
static void run_dma(const GemmParams& p, hipStream_t s) {
    if constexpr ((EPI == EPI_GLU || EPI == EPI_GLU_DW) && TN % 2 != 0) {
        throw std::logic_error("gemm: GLU epilogue dispatched to a 64-wide tile");
    } else {
        require(p.K % (64 * KG) == 0, "gemm: K must split into whole 64-wide slabs per K group");
        const int sm = 64 * TM - (EPI == EPI_GLU_DW ? GLU_DW_K - 1 : 0);   // output rows per tile
        const int tiles = cdiv(p.M, sm) * cdiv(p.N, 64 * TN);
        GemmParams q = p;
        q.xcd_gm = choose_xcd_gm(p, WT, sm, 64 * TN);
        launch((gemm_dma_kernel<TM, TN, WT, EPI, NS, KG, WL>), dim3(tiles), dim3(256 * KG), 0, s, q);
        PKX_LAUNCH_CHECK();
    }
}

template <int WTM, int WTN, int WT, int EPI, int NS, int KG = 1, int NWV = 4>
static void run_rb(const GemmParams& p, hipStream_t s) {
    typedef RbCfg<WTM, WTN, WT, EPI, NS, false, KG, NWV> C;
    constexpr bool can_fold = (EPI == EPI_STORE || EPI == EPI_SILU) && KG == 1;
    require(p.K % (64 * C::U * KG) == 0, "gemm: register-B kernel needs K % (256 x K groups) == 0");
    if (EPI == EPI_RESID_LN) require(p.N % 32 == 0, "gemm: register-B residual + LayerNorm statistics needs N % 32 == 0");
    require(p.N % 16 == 0, "gemm: register-B kernel needs N % 16 == 0 (16-column stores)");
    require((int64_t)p.M * p.ldy * (EPI == EPI_STORE_F32 || C::RESID ? 4 : 2) < ((int64_t)1 << 31),
            "gemm: register-B kernel output must stay below 2 GB (32-bit store offsets)");
    if (p.fold_stats) require(p.fold_groups <= 32, "gemm: register-B kernel folds at most 32 statistics groups");
    const int tiles = cdiv(p.M, C::BM) * cdiv(p.N, C::BN);
    GemmParams q = p;
    q.xcd_gm = choose_xcd_gm(p, WT, C::BM, C::BN);
    if (can_fold && p.fold_stats) launch((gemm_rb_kernel<WTM, WTN, WT, EPI, NS, can_fold, KG, NWV>), dim3(tiles), dim3(C::NT), 0, s, q);
    else launch((gemm_rb_kernel<WTM, WTN, WT, EPI, NS, false, KG, NWV>), dim3(tiles), dim3(C::NT), 0, s, q);
    PKX_LAUNCH_CHECK();
}

template <int TM, int TN, int WT>
static void f16_epi(int epi, const GemmParams& p, hipStream_t s) { PKX_EPI_SWITCH(run_f16, TM, TN, WT) }
template <int TM, int TN, int WT>
static void dma_epi(int epi, const GemmParams& p, hipStream_t s) { PKX_EPI_SWITCH_DMA(run_dma, TM, TN, WT) }
// a 2-stage ring: short-K products (a handful of slabs per tile) over many tiles
// fit three workgroups per CU instead of two
template <int TM, int TN, int WT, int EPI>
static void run_dma_ns2(const GemmParams& p, hipStream_t s) { run_dma<TM, TN, WT, EPI, 2>(p, s); }
template <int TM, int TN, int WT>
static void dma_epi_ns2(int epi, const GemmParams& p, hipStream_t s) { PKX_EPI_SWITCH_DMA(run_dma_ns2, TM, TN, WT) }
// the 2 x 2 wave layout with the slab's LDS reads issued up front
template <int TM, int TN, int WT, int EPI>
static void run_dma_pf(const GemmParams& p, hipStream_t s) { run_dma<TM, TN, WT, EPI, DMA_NS, 1, 2>(p, s); }
template <int TM, int TN, int WT>
static void dma_epi_pf(int epi, const GemmParams& p, hipStream_t s) { PKX_EPI_SWITCH_DMA(run_dma_pf, TM, TN, WT) }
// 128 x 128 tiles of quantised weights: the side-by-side wave layout (each
// weight row dequantised by one wave only) with the slab's LDS reads issued up
// front, for every epilogue that allows it
template <int WT>
static void dma_22q(int epi, const GemmParams& p, hipStream_t s) {
    switch (epi) {
    case EPI_STORE: run_dma<2, 2, WT, EPI_STORE, DMA_NS, 1, 1>(p, s); break;
    case EPI_STORE_F32: run_dma<2, 2, WT, EPI_STORE_F32, DMA_NS, 1, 1>(p, s); break;
    case EPI_SILU: run_dma<2, 2, WT, EPI_SILU, DMA_NS, 1, 1>(p, s); break;
    case EPI_RESID: run_dma<2, 2, WT, EPI_RESID, DMA_NS, 1, 1>(p, s); break;
    case EPI_RELU: run_dma<2, 2, WT, EPI_RELU, DMA_NS, 1, 1>(p, s); break;
    case EPI_RESID_LN: run_dma<2, 2, WT, EPI_RESID_LN, DMA_NS, 1, 1>(p, s); break;
    default: dma_epi<2, 2, WT>(epi, p, s); break;
    }
}
// Split-K across workgroups for the residual products of few rows and K >= 1024
// (a streaming step's FFN linear2: M = streams x chunk frames, 64 x 64 tiles in
// the tens): 64 x 64 tiles in two K groups, the K range cut over S workgroups
// per tile (S a power of two up to 8, each K group keeping at least one 64-deep
// slab) until the grid holds about one workgroup per CU.  On MI355X at M = 512,
// N = 512, K = 2048: 64 tiles x 4 splits, 1.4 us faster per launch; at K = 512
// (linear_out, pw2) and with two workgroups per CU it was slower.
template <int WT>
static bool dma_splitk(int epi, const GemmParams& p, hipStream_t s) {
    if (!p.sk_part || !p.sk_cnt || p.M > 512 || p.K < 1024 || (epi != EPI_RESID && epi != EPI_RESID_LN))
        return false;
    const int tiles = cdiv(p.M, 64) * cdiv(p.N, 64);
    const int cus = device_cu_count();
    int S = 1;
    while (S < 8 && 2 * S * tiles <= cus && p.K % (2 * S * 128) == 0) S *= 2;
    if (S == 1 || (int64_t)tiles * S * 64 * 64 > p.sk_part_floats || tiles > p.sk_cnt_n) return false;
    GemmParams q = p;
    q.ksplit = S;
    q.xcd_gm = choose_xcd_gm(p, WT, 64, 64);
    if (epi == EPI_RESID) launch((gemm_dma_kernel<1, 1, WT, EPI_RESID, DMA_NS, 2, 3>), dim3(tiles * S), dim3(512), 0, s, q);
    else launch((gemm_dma_kernel<1, 1, WT, EPI_RESID_LN, DMA_NS, 2, 3>), dim3(tiles * S), dim3(512), 0, s, q);
    PKX_LAUNCH_CHECK();
    return true;
}
// 128 x 64 tiles with two K groups (eight waves): products of K >= 1024 whose
// grid is about one tile per CU and that the register-B kernels do not take
// (pw2 with f16 weights at K = 1024; the split took 0.3 - 0.9 us off a
// 14 - 15 us launch of these shapes)
template <int WT>
static bool dma_kg2(int epi, const GemmParams& p, hipStream_t s) {
    if (p.K % 128 != 0 || p.K < 1024 || (int64_t)cdiv(p.M, 128) * cdiv(p.N, 64) > 256) return false;
    if (WT != GT_F16 && p.M <= 512) {
        switch (epi) {
        case EPI_RESID: run_dma<1, 1, WT, EPI_RESID, DMA_NS, 2, 0>(p, s); return true;
        case EPI_RESID_LN: run_dma<1, 1, WT, EPI_RESID_LN, DMA_NS, 2, 0>(p, s); return true;
        default: break;
        }
    }
    switch (epi) {
    case EPI_STORE: run_dma<2, 1, WT, EPI_STORE, DMA_NS, 2, WT == GT_F16 ? 0 : 2>(p, s); return true;
    case EPI_STORE_F32: run_dma<2, 1, WT, EPI_STORE_F32, DMA_NS, 2, WT == GT_F16 ? 0 : 2>(p, s); return true;
    case EPI_RESID: run_dma<2, 1, WT, EPI_RESID, DMA_NS, 2, WT == GT_F16 ? 0 : 2>(p, s); return true;
    case EPI_SILU: run_dma<2, 1, WT, EPI_SILU, DMA_NS, 2, WT == GT_F16 ? 0 : 2>(p, s); return true;
    case EPI_RESID_LN: run_dma<2, 1, WT, EPI_RESID_LN, DMA_NS, 2, WT == GT_F16 ? 0 : 2>(p, s); return true;
    default: return false;
    }
}
// Register-B kernel (128 x 256 tiles, one per CU, eight waves of 32 columns:
// two per SIMD; 4.56 -> 4.52 ms per step against four waves of 64 columns,
// same machine) for the wide quantised products: FFN linear1 (N = 4096),
// q/k/v (N = 3072) and the all-layer positional projection.  On MI355X at M = 2000, K = 1024 (q8_0): 25.7 against
// 27.8 us (FFN linear1), 25.0 against 27.7 (q/k/v, folded LayerNorm), 22.2
// against 24.9 (positional, M = 249, N = 24576) for the LDS-B 128 x 128 tiles.
// Taken when the grid is one round of the chip at least 70% full, or four
// rounds or more; in between (M = 3000: 384 tiles, a half-empty second round
// of long workgroups) the LDS-B kernels' finer tiles win (1.1B shape at batch
// 8 x 30 s: 14.44 against 13.82 ms per forward with the register-B kernel).
template <int WT>
static bool dma_rb(int epi, const GemmParams& p, hipStream_t s) {
    if (p.K % 256 != 0 || p.N < 2048 || p.N % 16 != 0 || (p.fold_stats && p.fold_groups > 32)) return false;
    if ((int64_t)p.M * p.ldy * (epi == EPI_STORE_F32 ? 4 : 2) >= ((int64_t)1 << 31)) return false;
    if (epi != EPI_STORE && epi != EPI_SILU && epi != EPI_STORE_F32) return false;
    const int64_t tiles = (int64_t)cdiv(p.M, 128) * cdiv(p.N, 256), cus = device_cu_count();
    if (!((tiles <= cus && tiles * 10 >= cus * 7) || tiles >= 4 * cus)) return false;
    switch (epi) {
    case EPI_STORE: run_rb<4, 1, WT, EPI_STORE, 4, 1, 8>(p, s); break;
    case EPI_SILU: run_rb<4, 1, WT, EPI_SILU, 4, 1, 8>(p, s); break;
    default: run_rb<4, 1, WT, EPI_STORE_F32, 4, 1, 8>(p, s); break;
    }
    return true;
}

// Register-B kernel with two K groups (64 x 128 tiles, eight waves, two per
// SIMD) for the quantised residual products whose grid of those tiles is about
// one round of the chip: N = 1024 at M = 2000 (FFN linear2 at K = 4096,
// attention output at K = 1024).  The LDS-B kernel's main loop there waits on
// its LDS reads (both operands from LDS, no read-ahead): on MI355X at
// M = 2000, N = 1024 (q8_0) 27.0 against 30.2 us at K = 4096 and 12.7 against
// 13.3 us at K = 1024.  f16 weights (pointwise_conv2) stream twice the bytes
// per slab from L2 and stay on the LDS-B kernel (16.4 against 13.6 us).
template <int WT>
static bool dma_rb_resid(int epi, const GemmParams& p, hipStream_t s) {
    if (epi != EPI_RESID && epi != EPI_RESID_LN) return false;
    if (p.K % 512 != 0 || p.N % 32 != 0 || p.ldy % 4 != 0) return false;
    if ((int64_t)p.M * p.ldy * 4 >= ((int64_t)1 << 31)) return false;
    const int64_t tiles = (int64_t)cdiv(p.M, 64) * cdiv(p.N, 128), cus = device_cu_count();
    if (!((tiles <= cus && tiles * 10 >= cus * 7) || tiles >= 4 * cus)) return false;
    if (epi == EPI_RESID) run_rb<2, 1, WT, EPI_RESID, 4, 2>(p, s);
    else run_rb<2, 1, WT, EPI_RESID_LN, 4, 2>(p, s);
    return true;
}

// The conv module (pointwise_conv1 + GLU + depthwise conv + BatchNorm + SiLU)
// on item tiles: one 128-row tile per item of T <= 128 frames and 64
// channels, so B x N / 128 workgroups (256 at B = 16, one per CU) and no
// halo rows; longer items in ceil(T / 120) parts with 4-row halos.  The
// register-B kernel in two K groups (128 x 128 tiles, eight waves, two per
// SIMD).  The LDS-B kernel's 64-row tiles writing 56 rows (576 of them at
// B = 16, T' = 125) run 2.25 rounds of the chip.
// f16 weights run from their fragment-order copy (p.wfrag) when one is given.
template <int WT>
static bool rb_glu_dw(const GemmParams& p, hipStream_t s) {
    if (p.M % p.T != 0 || p.N % 128 != 0 || p.K % 512 != 0) return false;
    require((int64_t)p.M * p.ldy * 2 < ((int64_t)1 << 31), "gemm: conv-module output must stay below 2 GB");
    constexpr int HALO = (GLU_DW_K - 1) / 2;
    const int nti = p.T <= 128 ? 1 : cdiv(p.T, 128 - 2 * HALO), orows = cdiv(p.T, nti);   // as in the kernel
    const int64_t tiles64 = (int64_t)(p.M / p.T) * nti * (p.N / 128);
    // one workgroup per CU: past two rounds of the chip the LDS-B kernel's
    // three co-resident workgroups per CU win (on MI355X, f16 weights:
    // 256 / 512 tiles 17.0 / 33.0 us against 23.7 / 37.7; 704 tiles at
    // d = 1408 58.5 against 46.2, 5632 tiles 437 against 401)
    if (tiles64 > 2 * (int64_t)device_cu_count()) return false;
    const int tiles = (int)tiles64;
    GemmParams q = p;
    q.xcd_gm = choose_xcd_gm(p, WT, orows, 128);
    auto go = [&](auto WTC) {
        constexpr int W = decltype(WTC)::value;
        constexpr int NT = RbCfg<4, 1, W, EPI_GLU_DW, 4, true, 2, 4>::NT;
        if (p.fold_stats) launch((gemm_rb_kernel<4, 1, W, EPI_GLU_DW, 4, true, 2, 4>), dim3(tiles), dim3(NT), 0, s, q);
        else launch((gemm_rb_kernel<4, 1, W, EPI_GLU_DW, 4, false, 2, 4>), dim3(tiles), dim3(NT), 0, s, q);
    };
    if (WT == GT_F16 && p.wfrag) {
        q.Wq = p.wfrag;
        go(std::integral_constant<int, GT_F16F>{});
    } else {
        go(std::integral_constant<int, WT>{});
    }
    PKX_LAUNCH_CHECK();
    return true;
}

// One 16-byte piece per thread: piece i = ((slab (N/32) + block) 4 + t) 64 +
// lane holds weight row glu_wcol(block / 4, block % 4, tail_col(lane % 32)),
// halves 64 slab + 32 (lane / 32) + 8 t .. + 7.
__global__ void glu_frag_kernel(const f16* __restrict__ w, int N, int K, f16* __restrict__ frag) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)N * K / 8) return;
    const int lane = (int)(i & 63), t = (int)((i >> 6) & 3);
    const int64_t sb = i >> 8;
    const int nblk = N / 32, blk = (int)(sb % nblk), slab = (int)(sb / nblk);
    const int n = glu_wcol(blk >> 2, blk & 3, tail_col(lane & 31));
    const int k = 64 * slab + 32 * (lane >> 5) + 8 * t;
    ((int4v*)frag)[i] = *(const int4v*)(w + (int64_t)n * K + k);
}

bool glu_frag_supported(int wtype, int N, int K) { return wtype == GT_F16 && N % 128 == 0 && K % 512 == 0; }
size_t glu_frag_bytes(int N, int K) { return (size_t)N * K * 2; }
void glu_frag_prepare(const void* w, int N, int K, void* frag, hipStream_t s) {
    require(glu_frag_supported(GT_F16, N, K), "glu_frag_prepare: f16 weights, N % 128 == 0, K % 512 == 0");
    const int64_t pieces = (int64_t)N * K / 8;
    launch(glu_frag_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, s, (const f16*)w, N, K, (f16*)frag);
    PKX_LAUNCH_CHECK();
}

template <int TM, int TN, int WT>
static void f32_epi(int epi, const GemmParams& p, hipStream_t s) { PKX_EPI_SWITCH(run_f32, TM, TN, WT) }
// tiles narrower than 64 columns per wave pair: every epilogue but GLU (which
// pairs 32-column input and gate groups inside a wave's 64 columns)
template <int TM, int TN, int WT>
static void f32_epi_narrow(int epi, const GemmParams& p, hipStream_t s) {
    switch (epi) {
    case EPI_STORE: run_f32<TM, TN, WT, EPI_STORE>(p, s); break;
    case EPI_STORE_F32: run_f32<TM, TN, WT, EPI_STORE_F32>(p, s); break;
    case EPI_SILU: run_f32<TM, TN, WT, EPI_SILU>(p, s); break;
    case EPI_RESID: run_f32<TM, TN, WT, EPI_RESID>(p, s); break;
    case EPI_RELU: run_f32<TM, TN, WT, EPI_RELU>(p, s); break;
    case EPI_RELU_TR: run_f32<TM, TN, WT, EPI_RELU_TR>(p, s); break;
    case EPI_RELU2_F32: run_f32<TM, TN, WT, EPI_RELU2_F32>(p, s); break;
    default: throw std::invalid_argument("gemm: bad epilogue");
    }
}
// shape 0: 64x128 tiles; 1: 32x64; 2: 32x32 (GLU keeps 64-column wave tiles: 32x128)
template <int WT>
static void f32_shape(int shape, int epi, const GemmParams& p, hipStream_t s) {
    if (shape == 0) f32_epi<2, 4, WT>(epi, p, s);
    else if (epi == EPI_GLU) f32_epi<1, 4, WT>(epi, p, s);
    else if (shape == 1) f32_epi_narrow<1, 2, WT>(epi, p, s);
    else f32_epi_narrow<1, 1, WT>(epi, p, s);
}

bool gemm_glu_dw_supported(Precision prec, int wtype, int N, int K) {
    return prec == PREC_F16 && N % 64 == 0 && K % 64 == 0 &&
           (wtype == GT_F16 || wtype == GT_Q8_0 || (wtype == GT_Q4_K && K % 256 == 0));
}

void launch_gemm(Precision prec, int wtype, int epi, const GemmParams& p, hipStream_t s) {
    require(p.M > 0 && p.N > 0 && p.K > 0, "gemm: empty shape");
    require(p.K % 8 == 0, "gemm: K must be a multiple of 8");
    require(p.lda >= p.K && p.lda % 8 == 0, "gemm: lda must be >= K and a multiple of 8 (16-byte rows)");
    if (wtype == GT_Q8_0) require(p.K % 32 == 0, "gemm: q8_0 needs K % 32 == 0");
    if (wtype == GT_Q4_K) require(p.K % 256 == 0, "gemm: q4_K needs K % 256 == 0");
    if (epi == EPI_GLU) require(p.N % 64 == 0, "gemm: GLU needs N % 64 == 0");
    if (epi == EPI_GLU_DW) {
        require(gemm_glu_dw_supported(prec, wtype, p.N, p.K) && p.ldy % 8 == 0,
                "gemm: fused conv-module epilogue needs the f16 path, N % 64 == 0, K % 64 == 0, ldy % 8 == 0");
        require(p.dw_w && p.dw_scale && p.dw_shift && p.T >= 1, "gemm: fused conv-module epilogue parameters");
        require(p.M < (1 << 22), "gemm: fused conv-module epilogue: fewer than 2^22 rows");
    }
    // the LDS-DMA kernel (f16 activations, K % 64 == 0) carries the LayerNorm folding
    const bool dma_ok = prec == PREC_F16 && p.K % 64 == 0 && p.ldy % 8 == 0 &&
                        (wtype == GT_F16 || wtype == GT_Q8_0 || wtype == GT_Q4_K);
    if (epi == EPI_RESID_LN)
        require(dma_ok && p.N % 32 == 0 && p.ln_g && p.ln_h && p.ln_stats,
                "gemm: residual + LayerNorm statistics needs the f16 path, N % 32 == 0 and its outputs");
    if (p.res_rows)
        require(epi == EPI_RESID_LN && p.res_g && p.res_b,
                "gemm: a LayerNorm on the residual goes with EPI_RESID_LN and needs its gamma and beta");
    if (p.fold_stats)
        require(dma_ok && p.fold_c1 && p.fold_groups >= 2 && p.fold_groups <= 32 &&
                    (p.fold_groups & (p.fold_groups - 1)) == 0 &&
                    (epi == EPI_STORE || epi == EPI_SILU || epi == EPI_GLU || epi == EPI_GLU_DW),
                "gemm: a folded LayerNorm needs the f16 path, 2..32 (a power of two) statistics groups and a STORE / SILU / GLU epilogue");
    if (epi == EPI_GLU_DW) {
        if (wtype == GT_F16 && rb_glu_dw<GT_F16>(p, s)) return;
        if (wtype == GT_Q8_0 && rb_glu_dw<GT_Q8_0>(p, s)) return;
        if (wtype == GT_Q4_K && rb_glu_dw<GT_Q4_K>(p, s)) return;
        // longer items: 64 x 128 tiles (56 output rows, 64 channels) on a
        // 2-stage ring, three workgroups per CU: the overlapping row tiles
        // outnumber two slots per CU
        switch (wtype) {
        case GT_F16: run_dma<1, 2, GT_F16, EPI_GLU_DW, 2>(p, s); break;
        case GT_Q8_0: run_dma<1, 2, GT_Q8_0, EPI_GLU_DW, 2>(p, s); break;
        default: run_dma<1, 2, GT_Q4_K, EPI_GLU_DW, 2>(p, s); break;
        }
        return;
    }
    const bool big = (int64_t)cdiv(p.M, 128) * cdiv(p.N, 128) >= 256;
    if (dma_ok) {
        // Tile shapes from sweeps over the encoder's shapes on MI355X (M = B*T' = 2000):
        // the register-B kernels take the wide quantised products and the quantised
        // N = 1024 residual products when their grids fit one round of the chip;
        // otherwise q8_0 and q4_K weights prefer 128x128 when the grid holds >= 384 of
        // them, 128x64 with two K groups for long K, 64x64 for grids too small to fill
        // the chip; f16 weights run best at 64x128 (pw2: 128x64, two K groups).  The
        // GLU epilogue pairs 64-column groups, so it needs a tile at least 128 wide.
        const int64_t t22 = (int64_t)cdiv(p.M, 128) * cdiv(p.N, 128);
        const int64_t t21 = (int64_t)cdiv(p.M, 128) * cdiv(p.N, 64);
        const bool glu = epi == EPI_GLU || epi == EPI_GLU_DW;
        if (wtype == GT_Q8_0 && dma_rb<GT_Q8_0>(epi, p, s)) return;
        if (wtype == GT_Q4_K && dma_rb<GT_Q4_K>(epi, p, s)) return;
        if (wtype == GT_Q8_0 && dma_rb_resid<GT_Q8_0>(epi, p, s)) return;
        if (wtype == GT_Q4_K && dma_rb_resid<GT_Q4_K>(epi, p, s)) return;
        if (wtype == GT_Q8_0 && dma_splitk<GT_Q8_0>(epi, p, s)) return;
        if (wtype == GT_Q4_K && dma_splitk<GT_Q4_K>(epi, p, s)) return;
        if (wtype == GT_F16 && dma_splitk<GT_F16>(epi, p, s)) return;
        if (wtype == GT_Q8_0 && dma_kg2<GT_Q8_0>(epi, p, s)) return;
        if (wtype == GT_Q4_K && dma_kg2<GT_Q4_K>(epi, p, s)) return;
        if (wtype == GT_F16 && dma_kg2<GT_F16>(epi, p, s)) return;
        if (wtype == GT_Q8_0) {
            if (t22 >= 384 || (glu && t22 >= 256)) dma_22q<GT_Q8_0>(epi, p, s);
            else if (glu) dma_epi<1, 2, GT_Q8_0>(epi, p, s);
            // few rows (a streaming step: M = streams x chunk frames): the most workgroups
            else if (p.M <= 512 && (int64_t)cdiv(p.M, 64) * cdiv(p.N, 64) <= 512) dma_epi<1, 1, GT_Q8_0>(epi, p, s);
            else if (t21 >= 128) dma_epi_pf<2, 1, GT_Q8_0>(epi, p, s);
            else dma_epi<1, 1, GT_Q8_0>(epi, p, s);
        } else if (wtype == GT_Q4_K) {
            if (t22 >= 384 || (glu && t22 >= 256)) dma_22q<GT_Q4_K>(epi, p, s);
            else if (glu) dma_epi<1, 2, GT_Q4_K>(epi, p, s);
            else if (t21 >= 128) dma_epi_pf<2, 1, GT_Q4_K>(epi, p, s);
            else dma_epi<1, 1, GT_Q4_K>(epi, p, s);
        } else if (p.K <= 256) {
            // the subsampling's pointwise convs (K = N = 256 channels, M in the
            // 10^4 - 10^5 pixels): 23% faster on the 2-stage ring
            dma_epi_ns2<1, 2, GT_F16>(epi, p, s);
        } else {
            dma_epi<1, 2, GT_F16>(epi, p, s);
        }
    } else if (prec == PREC_F16) {
        switch (wtype) {
        case GT_F16: big ? f16_epi<4, 4, GT_F16>(epi, p, s) : f16_epi<2, 4, GT_F16>(epi, p, s); break;
        case GT_Q8_0: big ? f16_epi<4, 4, GT_Q8_0>(epi, p, s) : f16_epi<2, 4, GT_Q8_0>(epi, p, s); break;
        case GT_Q4_K: big ? f16_epi<4, 4, GT_Q4_K>(epi, p, s) : f16_epi<2, 4, GT_Q4_K>(epi, p, s); break;
        default: throw std::invalid_argument("gemm(f16): weight type must be f16/q8_0/q4_K");
        }
    } else {
        // 64x128 tiles while they fill the chip; a single utterance (M = T' ~ 125)
        // gives only 8-32 of them, so smaller tiles buy workgroups there
        const int64_t t24 = (int64_t)cdiv(p.M, 64) * cdiv(p.N, 128);
        const int64_t t12 = (int64_t)cdiv(p.M, 32) * cdiv(p.N, 64);
        const int shape = t24 >= 256 ? 0 : t12 >= 256 ? 1 : 2;
        switch (wtype) {
        case GT_F32: f32_shape<GT_F32>(shape, epi, p, s); break;
        case GT_F16: f32_shape<GT_F16>(shape, epi, p, s); break;
        case GT_Q8_0: f32_shape<GT_Q8_0>(shape, epi, p, s); break;
        case GT_Q4_K: f32_shape<GT_Q4_K>(shape, epi, p, s); break;
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

// One wave per weight row n: c1 = g . w[n], c2 = b . w[n] + bias[n], with w the
// f16 value the GEMM's in-register dequantisation produces (device layouts:
// f16 [N][K]; q8_0 slab-major int8 [K/64][N][64] + f16 d [K/64][N][2],
// w = f16(q d); q4_K slab-major nibbles [K/64][N][32] + float2 {scale, min}
// [K/64][N][2], w = f16(q s16 - m16)).
__global__ void ln_fold_consts_kernel(int wtype, const uint8_t* Wq, const uint8_t* Ws, int N, int K, const float* g,
                                      const float* b, const float* bias, float* c1, float* c2) {
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (n >= N) return;
    float s1 = 0.f, s2 = 0.f;
    for (int k = lane; k < K; k += 64) {
        float w;
        if (wtype == GT_F16) {
            w = (float)((const f16*)Wq)[(int64_t)n * K + k];
        } else if (wtype == GT_Q8_0) {   // slab-major, N rows per slab block
            const int64_t blk = (int64_t)(k / 64) * N + n;
            const float q = (float)((const int8_t*)Wq)[blk * 64 + (k & 63)];
            const float d = (float)((const f16*)Ws)[blk * 2 + ((k & 63) >> 5)];
            w = (float)(f16)(q * d);
        } else {
            const int l = k % 64;
            const int64_t blk = (int64_t)(k / 64) * N + n;   // slab-major, N rows per slab block
            const uint8_t byte = Wq[blk * 32 + (l & 31)];
            const float q = (float)(l < 32 ? (byte & 0xF) : (byte >> 4));
            const float2v sm = ((const float2v*)Ws)[blk * 2 + (l >> 5)];
            w = (float)(f16)fmaf(q, (float)(f16)sm.x, (float)(f16)(-sm.y));
        }
        s1 += g[k] * w;
        s2 += b[k] * w;
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    if (lane == 0) {
        c1[n] = s1;
        c2[n] = s2 + (bias ? bias[n] : 0.f);
    }
}

void launch_ln_fold_consts(int wtype, const void* Wq, const void* Ws, int N, int K, const float* g,
                           const float* b, const float* bias, float* c1, float* c2, hipStream_t s) {
    require(wtype == GT_F16 || wtype == GT_Q8_0 || wtype == GT_Q4_K, "ln fold: weight type must be f16/q8_0/q4_K");
    require(N > 0 && K > 0 && g && b && c1 && c2, "ln fold: bad arguments");
    launch(ln_fold_consts_kernel, dim3(cdiv(N, 4)), dim3(256), 0, s, wtype, (const uint8_t*)Wq, (const uint8_t*)Ws,
           N, K, g, b, bias, c1, c2);
    PKX_LAUNCH_CHECK();
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

// Loads this file's code object on the current device (the runtime loads it
// at the first launch otherwise, taking device memory then).
void gemm_module_ready() {
    hipFuncAttributes a;
    PKX_HIP(hipFuncGetAttributes(&a, (const void*)dequant_f16_kernel));
}

void launch_dequantize(int wtype, const void* src, float* dst, int64_t n, hipStream_t s) {
    const int bs = 256;
    if (wtype == GT_Q8_0) {
        require(n % 32 == 0, "dequantize: q8_0 needs n % 32 == 0");
        launch(dequant_q8_0_kernel, dim3(cdiv(n, bs)), dim3(bs), 0, s, (const uint8_t*)src, dst, n / 32);
    } else if (wtype == GT_Q4_K) {
        require(n % 256 == 0, "dequantize: q4_K needs n % 256 == 0");
        launch(dequant_q4_k_kernel, dim3(cdiv(n, bs)), dim3(bs), 0, s, (const uint8_t*)src, dst, n / 256);
    } else if (wtype == GT_F16) {
        launch(dequant_f16_kernel, dim3(cdiv(n, bs)), dim3(bs), 0, s, (const f16*)src, dst, n);
    } else {
        throw std::invalid_argument("dequantize: unsupported type");
    }
    PKX_LAUNCH_CHECK();
}

}  // namespace pkx

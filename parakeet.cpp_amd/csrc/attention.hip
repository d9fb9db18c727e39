// Relative-position multi-head self-attention core (Transformer-XL style).
//
// Replaces, for every (item b, head h), the reference sequence
// relpos_attention.cpp:213-286: qu = q + pos_bias_u, qv = q + pos_bias_v,
// ac = qu.k^T, bd = qv.p^T, rel_shift(bd) (pad/reshape/view, :226-238),
// softmax(scale*(ac+bd) + key mask) (:252-278), attn.v, head merge, and the
// padded-query zeroing (:291-302).  The [T,T] score matrix is never stored:
// keys are streamed in tiles of 64 with an online softmax, and the shifted
// term uses the identity bd_shift[i][j] = bd[i][T-1-i+j]: for a 16-query x
// 64-key tile the needed positional rows form one band of 79 rows, computed
// as a 16x80 MFMA product into LDS and gathered along the diagonal.  Each
// wave's G rows and probabilities are private to it, so only the shared
// K / V / band staging needs block-wide barriers.
#include "attention.hpp"

#include <type_traits>

namespace pkx {

constexpr int AK = 64;   // keys per tile

// ---------------------------------------------------------------------------
// f16 MFMA kernel, key-split: 8 waves per block in two key groups.  Waves 0-3
// take the even 64-key tiles, waves 4-7 the odd ones, each wave the same 16
// query rows as its partner; the two online-softmax states are merged once at
// the end.  A 64-query block therefore keeps two waves per SIMD busy, and a
// short sequence (T' <= 128) costs each wave a single key tile.  K, V and the
// positional band are staged for both tiles of a step at once; their 16-byte
// chunks are XOR-swizzled within each 256-byte LDS line, so 16 consecutive
// rows read at one logical chunk hit 16 distinct bank quads without row
// padding.  P.V reads V with transposing LDS loads (ds_read_b64_tr_b16).
// ---------------------------------------------------------------------------
template <int DK>
struct KsSmem {
    static constexpr int AQ = 64;                   // queries per block
    static constexpr int NCH = DK / 8;              // 16-byte chunks per K / band row
    static constexpr int BROWS = AQ + 2 * AK;       // band rows per step (AQ + 2 AK - 1 used)
    static constexpr int LDG = 84;                  // G row (floats): row groups 4 apart land 16 banks apart
    static constexpr int LDP = AK + 8;              // probability row (halves)
    f16 k[2 * AK * DK];       // [group][key][DK]
    f16 vt[2 * AK * DK];      // V: [group][key][DK]
    f16 p[BROWS * DK];        // band rows of the step
    float g[8][16 * LDG];     // per wave: G, then its probabilities (f16)
};

// stored position of logical 16-byte chunk c in row r of a swizzled array
// with nch chunks per row (rows shorter than 256 bytes share an LDS line)
__device__ __forceinline__ int swz(int r, int c, int nch) { return c ^ ((r / (16 / nch)) % nch); }

template <int DK, bool LONG>
__global__ __launch_bounds__(512, 1) void relpos_attn_ks_kernel(AttnParams a) {
    static_assert(DK == 32 || DK == 64 || DK == 128, "head dim");
    typedef KsSmem<DK> S;
    constexpr int AQ = S::AQ, NCH = S::NCH, NT = 512, NKC = DK / 32, NDT = DK / 16;
    __shared__ __attribute__((aligned(16))) S sm;
    static_assert(sizeof(S) <= 160 * 1024, "LDS");

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int grp = w >> 2, wq = w & 3;
    const int T = a.T, P = 2 * T - 1;
    // work order (head, item, query block), query block fastest, each XCD a
    // contiguous run: the blocks of one item share K and V, those of one head
    // the positional band, in the XCD's L2
    const int nq = (T + AQ - 1) / AQ;
    const int wid = xcd_tile(blockIdx.x, nq * a.B * a.H);
    const int b = (wid / nq) % a.B, h = wid / (nq * a.B), i0 = (wid % nq) * AQ;
    const int vl = a.valid ? a.valid[b] : T;
    const int i0w = i0 + 16 * wq;
    const int lr = 4 * (lane >> 4), lc = lane & 15;
    const f16* q = (const f16*)a.q;
    const f16* k = (const f16*)a.k;
    const f16* v = (const f16*)a.v;
    const f16* pp = (const f16*)a.p;
    const int64_t rowq = (int64_t)b * T;
    const int nit = (vl + 2 * AK - 1) / (2 * AK);   // steps of 128 keys (<= 1 unless LONG)

    // K, V and the positional band of a step through registers (long
    // sequences: the next step's loads are in flight while this one is
    // computed); V keeps its own layout, P.V reads it with transposing loads
    constexpr int KCH = 2 * AK * NCH, PCH = S::BROWS * NCH;
    constexpr int KPT = LONG ? (KCH + NT - 1) / NT : 1, PPT = LONG ? (PCH + NT - 1) / NT : 1;
    half8v kreg[KPT], vreg[KPT], preg[PPT];
    auto load_kp = [&](int jb) {
        const int rlo = T - 1 - (i0 + AQ - 1) + jb;
#pragma unroll
        for (int u = 0; u < KPT; ++u) {
            const int c = tid + NT * u, r = c / NCH, j = jb + r;
            const bool in = c < KCH && j < T;
            kreg[u] = in ? *(const half8v*)(k + (rowq + j) * a.ldk + h * DK + (c % NCH) * 8) : (half8v){};
            vreg[u] = in ? *(const half8v*)(v + (rowq + j) * a.ldv + h * DK + (c % NCH) * 8) : (half8v){};
        }
#pragma unroll
        for (int u = 0; u < PPT; ++u) {
            const int c = tid + NT * u, pr = rlo + c / NCH;
            preg[u] = (c < PCH && pr >= 0 && pr < P) ? *(const half8v*)(pp + (int64_t)pr * a.ldp + h * DK + (c % NCH) * 8)
                                                     : (half8v){};
        }
    };
    auto store_kp = [&]() {
#pragma unroll
        for (int u = 0; u < KPT; ++u) {
            const int c = tid + NT * u, r = c / NCH;   // r: 0..127 = group * 64 + key
            if (c < KCH) {
                *(half8v*)(sm.k + r * DK + swz(r, c % NCH, NCH) * 8) = kreg[u];
                *(half8v*)(sm.vt + r * DK + swz(r, c % NCH, NCH) * 8) = vreg[u];
            }
        }
#pragma unroll
        for (int u = 0; u < PPT; ++u) {
            const int c = tid + NT * u, r = c / NCH;
            if (c < PCH) *(half8v*)(sm.p + r * DK + swz(r, c % NCH, NCH) * 8) = preg[u];
        }
    };
    // A single step (T' <= 128): K and the band go straight into LDS by DMA,
    // 16 bytes per lane, the swizzle applied through each lane's source
    // chunk; rows past T' or outside the band's 2T'-1 positions read past the
    // buffer's end (negative rows wrap above it) and arrive as zeros.
    auto dma_kp = [&]() {
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(k + rowq * a.ldk + h * DK, ((int64_t)(T - 1) * a.ldk + DK) * 2);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(v + rowq * a.ldv + h * DK, ((int64_t)(T - 1) * a.ldv + DK) * 2);
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(pp + h * DK, ((int64_t)(P - 1) * a.ldp + DK) * 2);
        const int rlo = T - 1 - (i0 + AQ - 1);
        constexpr int KI = KCH / 64, PI = PCH / 64;   // 1-KB instructions per array
        for (int ii = w; ii < KI; ii += 8) {
            const int o = ii * 1024 + 16 * lane, r = o / (DK * 2), t = (o % (DK * 2)) / 16;
            lds_dma16(rk, (uint8_t*)sm.k + ii * 1024, (uint32_t)((r * a.ldk + swz(r, t, NCH) * 8) * 2), 0);
        }
        // V in its own layout ([key][dim], swizzled like K); P.V reads it with
        // transposing LDS loads
        for (int ii = w; ii < KI; ii += 8) {
            const int o = ii * 1024 + 16 * lane, r = o / (DK * 2), t = (o % (DK * 2)) / 16;
            lds_dma16(rv, (uint8_t*)sm.vt + ii * 1024, (uint32_t)((r * a.ldv + swz(r, t, NCH) * 8) * 2), 0);
        }
        for (int ii = w; ii < PI; ii += 8) {
            const int o = ii * 1024 + 16 * lane, r = o / (DK * 2), t = (o % (DK * 2)) / 16;
            const int64_t off = ((int64_t)(rlo + r) * a.ldp + swz(r, t, NCH) * 8) * 2;
            lds_dma16(rp, (uint8_t*)sm.p + ii * 1024, off < 0 ? OOB : (uint32_t)off, 0);
        }
    };

    // the query rows and position biases first: they return ahead of the
    // staging loads issued next (vector memory returns in order).  The head's
    // biases [bias_u | bias_v] (2 DK floats) take one 16-byte load per lane
    // and reach the lanes that add them through the wave's G scratch: the
    // per-CU load path carries 1 KB per wave instead of 16.
    constexpr int BL = DK / 4;   // lanes per bias vector
    half8v qx[NKC];
    float4v bl = {0.f, 0.f, 0.f, 0.f};
    {
        const int i = i0w + lc;
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
            const int c0 = h * DK + 32 * kc + 8 * (lane >> 4);
            qx[kc] = i < T ? *(const half8v*)(q + (rowq + i) * a.ldq + c0) : (half8v){};
        }
        if (lane < 2 * BL) bl = *(const float4v*)((lane < BL ? a.bias_u : a.bias_v) + h * DK + 4 * (lane % BL));
    }
    if (nit > 0) {
        if constexpr (LONG) load_kp(0);
        else dma_kp();
    }
    float4v bq[NKC][4];   // bias_u, bias_u, bias_v, bias_v halves of each fragment's 8 columns
    {
        float4v* bs = (float4v*)sm.g[w];
        if (lane < 2 * BL) bs[lane] = bl;
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the wave's bias writes are done
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
            const int c4 = (32 * kc + 8 * (lane >> 4)) / 4;
            bq[kc][0] = bs[c4];
            bq[kc][1] = bs[c4 + 1];
            bq[kc][2] = bs[BL + c4];
            bq[kc][3] = bs[BL + c4 + 1];
        }
    }

    // Query fragments (A operand of v_mfma_f32_16x16x32_f16): row lane%16,
    // k = 32*kc + 8*(lane/16) + [0..7].  pos_bias_u/v added in f32.
    half8v qu[NKC], qv[NKC];
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float xf = (float)qx[kc][e];
            qu[kc][e] = (f16)(xf + bq[kc][e >> 2][e & 3]);
            qv[kc][e] = (f16)(xf + bq[kc][2 + (e >> 2)][e & 3]);
        }
    // scores in log2 units: exp(scale * x) = exp2(scale * log2(e) * x)
    const float sl2 = a.scale * 1.4426950408889634f;
    // chunk of each of this lane's query rows (chunked-limited window)
    int qch[4] = {0, 0, 0, 0};
    if (a.chunk > 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) qch[r] = (i0w + lr + r) / a.chunk;
    }

    float4v o[NDT];
#pragma unroll
    for (int d = 0; d < NDT; ++d) o[d] = (float4v){0.f, 0.f, 0.f, 0.f};
    float mrow[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    float lrow[4] = {0.f, 0.f, 0.f, 0.f};
    float* gw = sm.g[w];
    f16* probw = (f16*)gw;
    const f16* kt = sm.k + grp * AK * DK;
    const f16* vtt = sm.vt + grp * DK * AK;   // V of this group's keys ([key][dim], swizzled)
    const int pb = AQ - 16 - 16 * wq + AK * grp;   // this wave's first band row

    for (int s = 0; s < nit; ++s) {
        if constexpr (LONG) store_kp();
        __builtin_amdgcn_s_waitcnt(0);   // this wave's DMAs have landed
        __syncthreads();
        if constexpr (LONG) {
            if (s + 1 < nit) load_kp(2 * AK * (s + 1));
        }
        const int j0 = 2 * AK * s + AK * grp;
        if (j0 < vl) {
            // ---- ac = qu . k^T : 16 x 64 ----
            float4v sac[4];
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                sac[jt] = (float4v){0.f, 0.f, 0.f, 0.f};
                const int r = 16 * jt + lc;
#pragma unroll
                for (int kc = 0; kc < NKC; ++kc) {
                    const half8v kf = *(const half8v*)(kt + r * DK + swz(r, 4 * kc + (lane >> 4), NCH) * 8);
                    sac[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qu[kc], kf, sac[jt], 0, 0, 0);
                }
            }
            // ---- band product G = qv . p_band^T : 16 x 80 ----
#pragma unroll
            for (int gt = 0; gt < 5; ++gt) {
                float4v g = {0.f, 0.f, 0.f, 0.f};
                const int r = pb + 16 * gt + lc;
#pragma unroll
                for (int kc = 0; kc < NKC; ++kc) {
                    const half8v pf = *(const half8v*)(sm.p + r * DK + swz(r, 4 * kc + (lane >> 4), NCH) * 8);
                    g = __builtin_amdgcn_mfma_f32_16x16x32_f16(qv[kc], pf, g, 0, 0, 0);
                }
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) gw[(lr + rr) * S::LDG + 16 * gt + lc] = g[rr];
            }
            // the wave reads back only its own G rows
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();

            // ---- scores (rel_shift gather bd[i][j] = G[i][15 - i + j]), masks, online softmax ----
            const bool kmask = j0 + AK > vl, cmask = a.chunk > 0;
            int kch[4] = {0, 0, 0, 0};
            if (cmask) {
#pragma unroll
                for (int jt = 0; jt < 4; ++jt) kch[jt] = (j0 + 16 * jt + lc) / a.chunk;
            }
            float sc[4][4];
            float tmax[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
            for (int jt = 0; jt < 4; ++jt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int ii = lr + r, jj = 16 * jt + lc;
                    float sv = (sac[jt][r] + gw[ii * S::LDG + 15 - ii + jj]) * sl2;
                    if (kmask && j0 + jj >= vl) sv = -INFINITY;
                    if (cmask) {
                        const int dc = qch[r] - kch[jt];
                        if (dc < 0 || dc > a.left_chunks) sv = -INFINITY;
                    }
                    sc[jt][r] = sv;
                    tmax[r] = fmaxf(tmax[r], sv);
                }
            float corr[4], msub[4], tsum[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float mnew = fmaxf(mrow[r], row16_max(tmax[r]));
                msub[r] = mnew == -INFINITY ? 0.f : mnew;   // no -inf - -inf while every key so far is masked
                corr[r] = __builtin_amdgcn_exp2f(mrow[r] - msub[r]);
                mrow[r] = mnew;
                tsum[r] = 0.f;
            }
#pragma unroll
            for (int jt = 0; jt < 4; ++jt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = __builtin_amdgcn_exp2f(sc[jt][r] - msub[r]);
                    tsum[r] += e;
                    probw[(lr + r) * S::LDP + 16 * jt + lc] = (f16)e;
                }
#pragma unroll
            for (int r = 0; r < 4; ++r) lrow[r] = lrow[r] * corr[r] + group_sum(tsum[r], 16);
            if (s > 0) {
#pragma unroll
                for (int d = 0; d < NDT; ++d)
#pragma unroll
                    for (int r = 0; r < 4; ++r) o[d][r] *= corr[r];
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();

            // ---- o += prob . v : A = prob (16 x 64 keys), B = v^T rows ----
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                const half8v pf = *(const half8v*)(probw + lc * S::LDP + 32 * kc + 8 * (lane >> 4));
#pragma unroll
                for (int d = 0; d < NDT; ++d) {
                    // B[key][dim] for keys 32 kc + 8 (lane / 16) + 0..7, dim 16 d + lane % 16:
                    // in each 16-lane group, lane 4 j + q points at key j (and j + 4) and
                    // dims 16 d + 4 q .. + 3; the transposing load hands lane i the four
                    // keys' values of dim 16 d + i
                    const int kr = 32 * kc + 8 * (lane >> 4) + (lc >> 2);
                    const int dc = 16 * d + 4 * (lc & 3);             // first dim of the 8-byte piece
                    const int r0 = kr, r1 = kr + 4;
                    const f16* p0 = vtt + r0 * DK + swz(r0, dc / 8, NCH) * 8 + (dc & 7);
                    const f16* p1 = vtt + r1 * DK + swz(r1, dc / 8, NCH) * 8 + (dc & 7);
                    typedef __fp16 fp4 __attribute__((ext_vector_type(4)));
                    const half4v v0 = __builtin_bit_cast(half4v, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                                                     (__attribute__((address_space(3))) fp4*)p0));
                    const half4v v1 = __builtin_bit_cast(half4v, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                                                     (__attribute__((address_space(3))) fp4*)p1));
                    const half8v vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                    o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf, vf, o[d], 0, 0, 0);
                }
            }
        }
        if (s + 1 < nit) __syncthreads();   // the next step's staging overwrites K, V and the band
    }

    // ---- merge the two key groups: group 0 finishes rows r = 0, 1 of each
    // lane's four, group 1 rows 2, 3.  Each wave leaves the other half of its
    // state in its own G area (no other wave reads it: no barrier before),
    // as 16-byte chunks [chunk][lane]; after one barrier it finishes its half
    // from its partner's area and stages the output rows in the K area (free
    // once every wave is past its products) ----
    constexpr int MR4 = (NDT * 2 + 4) / 4;   // float4 per lane handed over: o of two rows, m and l
    static_assert(MR4 * 64 * 16 <= sizeof(sm.g[0]) && 4 * 16 * DK * 2 <= sizeof(sm.k), "merge areas");
    float4v* hand = (float4v*)sm.g[w] + lane;
    const float4v* take = (const float4v*)sm.g[w ^ 4] + lane;   // the partner: same query rows, other keys
    f16* stage = (f16*)sm.k + wq * 16 * DK;   // the 16 output rows of query block wq (f16, DK wide)
    auto give = [&](auto R) {
        constexpr int r0 = decltype(R)::value;
        float x[MR4 * 4];
#pragma unroll
        for (int d = 0; d < NDT; ++d) {
            x[2 * d] = o[d][r0];
            x[2 * d + 1] = o[d][r0 + 1];
        }
        x[2 * NDT] = mrow[r0];
        x[2 * NDT + 1] = mrow[r0 + 1];
        x[2 * NDT + 2] = lrow[r0];
        x[2 * NDT + 3] = lrow[r0 + 1];
#pragma unroll
        for (int c = 0; c < MR4; ++c) hand[c * 64] = (float4v){x[4 * c], x[4 * c + 1], x[4 * c + 2], x[4 * c + 3]};
    };
    auto keep = [&](auto R) {
        constexpr int r0 = decltype(R)::value;
        float y[MR4 * 4];
#pragma unroll
        for (int c = 0; c < MR4; ++c) {
            const float4v t = take[c * 64];
            y[4 * c] = t[0];
            y[4 * c + 1] = t[1];
            y[4 * c + 2] = t[2];
            y[4 * c + 3] = t[3];
        }
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const int r = r0 + rr;
            const float m1 = y[2 * NDT + rr], l1 = y[2 * NDT + 2 + rr];
            const float m = fmaxf(mrow[r], m1);
            const float c0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mrow[r] - m);
            const float c1 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - m);
            const float l = lrow[r] * c0 + l1 * c1;
            const int i = i0w + lr + r;
            const float inv = (i < vl && l > 0.f) ? 1.0f / l : 0.f;   // padded query rows are zero
#pragma unroll
            for (int d = 0; d < NDT; ++d)
                stage[(lr + r) * DK + 16 * d + lc] = (f16)((o[d][r] * c0 + y[2 * d + rr] * c1) * inv);
        }
    };
    if (grp == 0) give(std::integral_constant<int, 2>{});
    else give(std::integral_constant<int, 0>{});
    __syncthreads();
    if (grp == 0) keep(std::integral_constant<int, 0>{});
    else keep(std::integral_constant<int, 2>{});
    __syncthreads();
    // ---- store: wave (wq, grp) writes rows 8 grp .. 8 grp + 7 of block wq in 16-byte chunks ----
    f16* out = (f16*)a.out;
#pragma unroll
    for (int u = 0; u < (8 * NCH + 63) / 64; ++u) {
        const int c = lane + 64 * u, r = 8 * grp + c / NCH, i = i0w + r;
        if (c < 8 * NCH && i < T)
            *(half8v*)(out + (rowq + i) * a.ldo + h * DK + (c % NCH) * 8) = *(const half8v*)(stage + r * DK + (c % NCH) * 8);
    }
}

// ---------------------------------------------------------------------------
// f32 kernel (exact-precision path): one wave per query row, scores in LDS.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void relpos_attn_f32_kernel(AttnParams a, int dk) {
    extern __shared__ float smf[];
    float* qu = smf;            // [dk]
    float* qv = smf + dk;       // [dk]
    float* sc = smf + 2 * dk;   // [T]
    const int lane = threadIdx.x;
    const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int T = a.T;
    const int vl = a.valid ? a.valid[b] : T;
    const float* q = (const float*)a.q;
    const float* k = (const float*)a.k;
    const float* v = (const float*)a.v;
    const float* pp = (const float*)a.p;
    float* out = (float*)a.out;
    const int64_t rowq = (int64_t)b * T;
    float* orow = out + (rowq + i) * a.ldo + (int64_t)h * dk;
    if (i >= vl) {
        for (int c = lane; c < dk; c += 64) orow[c] = 0.f;
        return;
    }
    for (int c = lane; c < dk; c += 64) {
        const float x = q[(rowq + i) * a.ldq + (int64_t)h * dk + c];
        qu[c] = x + a.bias_u[h * dk + c];
        qv[c] = x + a.bias_v[h * dk + c];
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int j = lane; j < vl; j += 64) {
        const float* kr = k + (rowq + j) * a.ldk + (int64_t)h * dk;
        const float* pr = pp + (int64_t)(T - 1 - i + j) * a.ldp + (int64_t)h * dk;
        float ac = 0.f, bd = 0.f;
        for (int c = 0; c < dk; ++c) {
            ac += qu[c] * kr[c];
            bd += qv[c] * pr[c];
        }
        float s = (ac + bd) * a.scale;
        if (a.chunk > 0) {
            const int dc = i / a.chunk - j / a.chunk;
            if (dc < 0 || dc > a.left_chunks) s = -INFINITY;   // key i itself is always seen
        }
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    mx = wave_max(mx);
    float den = 0.f;
    for (int j = lane; j < vl; j += 64) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        den += e;
    }
    den = wave_sum(den);
    __syncthreads();
    const float inv = 1.0f / den;
    for (int c = lane; c < dk; c += 64) {
        float acc = 0.f;
        for (int j = 0; j < vl; ++j) acc += sc[j] * v[(rowq + j) * a.ldv + (int64_t)h * dk + c];
        orow[c] = acc * inv;
    }
}

void launch_relpos_attention(Precision prec, const AttnParams& a, hipStream_t s) {
    require(a.T > 0 && a.B > 0 && a.H > 0, "attention: empty shape");
    if (prec == PREC_F16) {
        // 64 queries per block, two key groups of four waves; sequences of at
        // most 128 frames take a single step whose K and band arrive by DMA
        const dim3 grid(cdiv(a.T, 64) * a.H * a.B);
        const bool lng = a.T > 2 * AK;
        if (a.dk == 128) {
            if (lng) launch(relpos_attn_ks_kernel<128, true>, grid, dim3(512), 0, s, a);
            else launch(relpos_attn_ks_kernel<128, false>, grid, dim3(512), 0, s, a);
        } else if (a.dk == 64) {
            if (lng) launch(relpos_attn_ks_kernel<64, true>, grid, dim3(512), 0, s, a);
            else launch(relpos_attn_ks_kernel<64, false>, grid, dim3(512), 0, s, a);
        } else if (a.dk == 32) {
            if (lng) launch(relpos_attn_ks_kernel<32, true>, grid, dim3(512), 0, s, a);
            else launch(relpos_attn_ks_kernel<32, false>, grid, dim3(512), 0, s, a);
        } else {
            throw std::invalid_argument("attention(f16): head dim must be 32, 64 or 128");
        }
    } else {
        const size_t smem = sizeof(float) * (2 * (size_t)a.dk + (size_t)a.T);
        require(smem <= 64 * 1024, "attention(f32): T too large for the LDS score row");
        launch(relpos_attn_f32_kernel, dim3(a.T, a.H, a.B), dim3(64), smem, s, a, a.dk);
    }
    PKX_LAUNCH_CHECK();
}

}  // namespace pkx

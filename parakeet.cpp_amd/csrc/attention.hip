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
// as an 80x16 MFMA product into LDS and gathered along the diagonal.  Each
// wave's G area is private to it, so only the shared K / V / band staging
// needs block-wide barriers.
#include "attention.hpp"

#include <algorithm>
#include <type_traits>

namespace pkx {

constexpr int AK = 64;   // keys per tile

// ---------------------------------------------------------------------------
// f16 MFMA kernel, key-split: 8 waves per block in two key groups.  Waves 0-3
// take the even 64-key tiles, waves 4-7 the odd ones, each wave the same 16
// query rows as its partner; the two online-softmax states are merged once at
// the end.  A 64-query block therefore keeps two waves per SIMD busy, and a
// short sequence (T' <= 128) costs each wave a single key tile.  The products
// are formed transposed (keys x queries, dims x queries): each lane holds
// the scores of one query, so the softmax reduces over its own registers and
// the three other lanes of that query, and its probabilities are already the
// B operand of O^T = V^T . P^T, with no pass through LDS.  K, V and the
// positional band are staged for both tiles of a step at once; their 16-byte
// chunks are XOR-swizzled within each 256-byte LDS line, so 16 consecutive
// rows read at one logical chunk hit 16 distinct bank quads without row
// padding.  V^T fragments come from V with transposing LDS loads
// (ds_read_b64_tr_b16).  A step's K, band and V arrive by DMA; the next
// step's are issued as soon as every wave has read the current ones.
// ---------------------------------------------------------------------------
template <int DK, int NQW, int NG>
struct KsSmem {
    static constexpr int NW = NQW * NG;             // waves: NQW query blocks of 16 x NG key groups
    static constexpr int AQ = 16 * NQW;             // queries per block
    static constexpr int NCH = DK / 8;              // 16-byte chunks per K / band row
    static constexpr int BROWS = AQ + NG * AK;      // band rows per step (AQ + NG AK - 1 used)
    // 1-KB DMA instructions for K (and for V) and for the band, each rounded
    // up to a multiple of the waves (rows past a step's own arrive unused)
    static constexpr int KI = (NG * AK * NCH / 64 + NW - 1) / NW * NW;
    static constexpr int PI = (BROWS * NCH / 64 + NW - 1) / NW * NW;
    static constexpr int LDG = 84;                  // G^T row (floats)
    f16 k[KI * 512];          // K: [group][key][DK]
    f16 vs[KI * 512];         // V: [group][key][DK]
    f16 p[PI * 512];          // band rows of the step
    float g[NW][16 * LDG];    // per wave: G^T as [query][band row]
};

// stored position of logical 16-byte chunk c in row r of a swizzled array
// with nch chunks per row (rows shorter than 256 bytes share an LDS line)
__device__ __forceinline__ int swz(int r, int c, int nch) { return c ^ ((r / (16 / nch)) % nch); }

// max / sum over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48);
// every lane of the four gets the same value
__device__ __forceinline__ float xg_max(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xg_sum(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// ds_read_b64_tr_b16 issued from inline assembly, and the wait for it: the
// compiler's own form of this load counts as possibly aliasing every LDS DMA
// in flight and would drain them all before it.  lds_tr_wait<N> waits until
// at most N LDS operations of the wave are outstanding (in-order completion,
// so the two loads named are done) and ties their registers to the wait.
// Invariant: between lds_tr_b64 and the lds_tr_wait that names its register,
// no instruction may read, copy, spill or overwrite that register (the data
// lands asynchronously; the compiler believes it valid at the load).  The
// destination is an in-out operand from a defined value, so the load and the
// wait are the register's only definitions, and each value is consumed right
// after its wait; the built code keeps the window clean (no VGPR copy or spill
// of a transposed-load destination between the load and its s_waitcnt, read
// from this file's gfx950 assembly).
__device__ __forceinline__ void lds_tr_b64(half4v& r, const f16* p) {
    const uint32_t off = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const f16*)p;
    r = (half4v){};
    asm volatile("ds_read_b64_tr_b16 %0, %1" : "+v"(r) : "v"(off));
}
template <int N> __device__ __forceinline__ void lds_tr_wait(half4v& x, half4v& y) {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(x), "+v"(y) : "n"(N));
}

// f(integral_constant<int, I>) for I = B .. E-1
template <int B, int E, typename F> __device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

template <int DK, int NQW, int NG>
__global__ __launch_bounds__(64 * NQW * NG, 1) void relpos_attn_ks_kernel(AttnParams a) {
    static_assert(DK == 32 || DK == 64 || DK == 128, "head dim");
    static_assert(NG == 1 || NG == 2, "key groups");
    typedef KsSmem<DK, NQW, NG> S;
    constexpr int AQ = S::AQ, NCH = S::NCH, NW = S::NW, NKC = DK / 32, NDT = DK / 16, SK = NG * AK;
    __shared__ __attribute__((aligned(16))) S sm;
    static_assert(sizeof(S) <= 160 * 1024, "LDS");

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = w / NQW, wq = w % NQW;
    const int T = a.T, P = 2 * T - 1;
    // work order (head, item, query block), query block fastest, each XCD a
    // contiguous run: the blocks of one item share K and V, those of one head
    // the positional band, in the XCD's L2
    const int nq = (T + AQ - 1) / AQ;
    const int wid = xcd_tile(blockIdx.x, nq * a.B * a.H);
    const int ib = udiv_small(wid, nq), h = udiv_small(ib, a.B);   // wid < 2^22 (checked at launch)
    const int b = ib - h * a.B, i0 = (wid - ib * nq) * AQ;
    const int vl = a.valid ? a.valid[b] : T;
    const int i0w = i0 + 16 * wq;
    const int lg = lane >> 4, lc = lane & 15;   // lane group; lane in group = this lane's query
    const f16* q = (const f16*)a.q;
    const f16* k = (const f16*)a.k;
    const f16* v = (const f16*)a.v;
    const f16* pp = (const f16*)a.p;
    const int64_t rowq = (int64_t)b * T;
    const int nit = (vl + SK - 1) / SK;   // steps of SK = NG x 64 keys

    // K, the band and V of a step go straight into LDS by DMA, 16 bytes per
    // lane, the swizzle applied through each lane's source chunk, the same
    // number of instructions from every wave; rows past T' or outside the
    // band's 2T'-1 positions read past the buffer's end (negative rows wrap
    // above it) and arrive as zeros.
    constexpr int KPW = S::KI / NW, PPW = S::PI / NW;   // DMA instructions per wave
    auto dma_rows = [&](__amdgpu_buffer_rsrc_t r, f16* dst, int64_t ld, int row0, int per_wave) {
        for (int u = 0; u < per_wave; ++u) {
            const int ii = w + NW * u;
            const int o = ii * 1024 + 16 * lane, rr = o / (DK * 2), t = (o % (DK * 2)) / 16;
            const int64_t off = ((int64_t)(row0 + rr) * ld + swz(rr, t, NCH) * 8) * 2;
            lds_dma16(r, (uint8_t*)dst + ii * 1024, off < 0 ? OOB : (uint32_t)off, 0);
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
            const int c0 = h * DK + 32 * kc + 8 * lg;
            qx[kc] = i < T ? *(const half8v*)(q + (rowq + i) * a.ldq + c0) : (half8v){};
        }
        if (lane < 2 * BL) bl = *(const float4v*)((lane < BL ? a.bias_u : a.bias_v) + h * DK + 4 * (lane % BL));
    }
    __builtin_amdgcn_sched_barrier(0);   // these loads stay ahead of the staging
    // issued whatever the item's length (an item with no valid frame still
    // waits for them below), so that the waits in between count a fixed
    // number of younger loads
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(k + rowq * a.ldk + h * DK, ((int64_t)(T - 1) * a.ldk + DK) * 2);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(pp + h * DK, ((int64_t)(P - 1) * a.ldp + DK) * 2);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(v + rowq * a.ldv + h * DK, ((int64_t)(T - 1) * a.ldv + DK) * 2);
    const int rlo = T - 1 - (i0 + AQ - 1);   // the band's first position at step 0
    auto dma_k = [&](int st) { dma_rows(rk, sm.k, a.ldk, SK * st, KPW); };          // K of step st
    auto dma_p = [&](int st) { dma_rows(rp, sm.p, a.ldp, rlo + SK * st, PPW); };    // its band
    auto dma_v = [&](int st) { dma_rows(rv, sm.vs, a.ldv, SK * st, KPW); };         // its V
    dma_k(0);
    float4v bq[NKC][4];   // bias_u, bias_u, bias_v, bias_v halves of each fragment's 8 columns
    {
        float4v* bs = (float4v*)sm.g[w];
        if (lane < 2 * BL) bs[lane] = bl;
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the wave's bias writes are done
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
            const int c4 = (32 * kc + 8 * lg) / 4;
            bq[kc][0] = bs[c4];
            bq[kc][1] = bs[c4 + 1];
            bq[kc][2] = bs[BL + c4];
            bq[kc][3] = bs[BL + c4 + 1];
        }
    }

    // Query fragments (B operand of v_mfma_f32_16x16x32_f16): query lane%16,
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
    // the step's band and V behind K: the query conversion above runs while
    // K is in flight instead of after the issue of all 112 KB
    dma_p(0);
    dma_v(0);
    // scores in log2 units: exp(scale * x) = exp2(scale * log2(e) * x)
    const float sl2 = a.scale * 1.4426950408889634f;
    // the keys this lane's query sees: [jlo, jhi), the valid frames and, with
    // a chunked-limited window, the chunks qc - left_chunks .. qc of the
    // query's chunk qc (j / chunk in that range <=> j in the interval)
    int jlo = 0, jhi = vl;
    if (a.chunk > 0) {
        const int qc = (i0w + lc) / a.chunk;
        jlo = max(0, (qc - a.left_chunks) * a.chunk);
        jhi = min(vl, (qc + 1) * a.chunk);
    }

    // O^T fragments: o[d][r] = output of query lane%16, dim 16 d + 4 (lane/16) + r
    float4v o[NDT];
#pragma unroll
    for (int d = 0; d < NDT; ++d) o[d] = (float4v){0.f, 0.f, 0.f, 0.f};
    float mrow = -INFINITY;   // running max of this lane's query (the same in its four lanes)
    float lrow = 0.f;         // this lane's part of the running denominator (its 16 keys per tile)
    float* gw = sm.g[w];
    const f16* kt = sm.k + grp * AK * DK;
    const f16* vst = sm.vs + grp * AK * DK;         // V of this group's keys ([key][dim], swizzled)
    const int pb = AQ - 16 - 16 * wq + AK * grp;   // this wave's first band row
    float4v sac[4];    // S^T: sac[jt][r] = score of this lane's query, key 16 jt + 4 (lane/16) + r
    half4v pr[4];      // its probabilities

    // ---- S^T = k . qu^T : 64 x 16 ----
    auto qk = [&]() {
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            sac[jt] = (float4v){0.f, 0.f, 0.f, 0.f};
            const int r = 16 * jt + lc;
#pragma unroll
            for (int kc = 0; kc < NKC; ++kc) {
                const half8v kf = *(const half8v*)(kt + r * DK + swz(r, 4 * kc + lg, NCH) * 8);
                sac[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qu[kc], sac[jt], 0, 0, 0);
            }
        }
    };
    // ---- band product G^T = p_band . qv^T : 80 x 16, into the wave's G area
    // as [query][band row] (one 16-byte write per lane and 16-row block) ----
    auto band = [&]() {
#pragma unroll
        for (int gt = 0; gt < 5; ++gt) {
            float4v g = {0.f, 0.f, 0.f, 0.f};
            const int r = pb + 16 * gt + lc;
#pragma unroll
            for (int kc = 0; kc < NKC; ++kc) {
                const half8v pf = *(const half8v*)(sm.p + r * DK + swz(r, 4 * kc + lg, NCH) * 8);
                g = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf, qv[kc], g, 0, 0, 0);
            }
            *(float4v*)(gw + lc * S::LDG + 16 * gt + 4 * lg) = g;
        }
        // the wave reads back only its own G area
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
    };
    // ---- scores (rel_shift gather bd[i][j] = G[i][15 - i + j]), masks, online softmax ----
    auto softmax = [&](int s, int j0) {
        float sc[4][4];
        float tmax = -INFINITY;
        const float* grow = gw + lc * S::LDG + 15 - lc + 4 * lg;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // the mask is added (x + -inf = -inf for the finite scores), not
                // selected: a select lets the compiler move each G read behind
                // a branch of its own
                const int j = j0 + 16 * jt + 4 * lg + r;
                const float sv = (sac[jt][r] + grow[16 * jt + r]) * sl2 + ((j < jlo || j >= jhi) ? -INFINITY : 0.f);
                sc[jt][r] = sv;
                tmax = fmaxf(tmax, sv);
            }
        const float mnew = fmaxf(mrow, xg_max(tmax));
        const float msub = mnew == -INFINITY ? 0.f : mnew;   // no -inf - -inf while every key so far is masked
        const float corr = __builtin_amdgcn_exp2f(mrow - msub);
        mrow = mnew;
        float tsum = 0.f;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(sc[jt][r] - msub);
                tsum += e;
                pr[jt][r] = (f16)e;
            }
        lrow = lrow * corr + tsum;
        if (s > 0) {
#pragma unroll
            for (int d = 0; d < NDT; ++d) o[d] *= corr;
        }
    };
    // ---- O^T += v^T . prob^T : per 32-key block kc, MFMA k slot 8 (lane/16) + e
    // stands for key 32 kc + 4 (lane/16) + e (e < 4) or 32 kc + 16 + 4 (lane/16)
    // + e - 4, the keys whose probabilities this lane holds ----
    auto pv = [&]() {
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            const half8v pf = {pr[2 * kc][0], pr[2 * kc][1], pr[2 * kc][2], pr[2 * kc][3],
                               pr[2 * kc + 1][0], pr[2 * kc + 1][1], pr[2 * kc + 1][2], pr[2 * kc + 1][3]};
            half4v v0[NDT], v1[NDT];
#pragma unroll
            for (int d = 0; d < NDT; ++d) {
                // A[dim][key] for dims 16 d + lane % 16: in each 16-lane group, lane
                // 4 j + q points at key base + j and dims 16 d + 4 q .. + 3; the
                // transposing load hands lane i the four keys' values of dim 16 d + i
                const int kr = 32 * kc + 4 * lg + (lc >> 2);
                const int dc = 16 * d + 4 * (lc & 3);
                const int r1 = kr + 16;
                lds_tr_b64(v0[d], vst + kr * DK + swz(kr, dc / 8, NCH) * 8 + (dc & 7));
                lds_tr_b64(v1[d], vst + r1 * DK + swz(r1, dc / 8, NCH) * 8 + (dc & 7));
            }
            auto mma = [&](auto D) {
                constexpr int d = decltype(D)::value;
                lds_tr_wait<2 * (NDT - 1 - d)>(v0[d], v1[d]);
                const half8v vf = {v0[d][0], v0[d][1], v0[d][2], v0[d][3], v1[d][0], v1[d][1], v1[d][2], v1[d][3]};
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf, o[d], 0, 0, 0);
            };
            static_for<0, NDT>(mma);
        }
    };

    // Steps of 128 keys.  In flight at the top of a step, oldest first: its
    // K, band and V.  The next step's K and band are issued once every wave
    // has its scores, its V once every wave is past P.V; each wait leaves the
    // younger DMAs in flight, and a bare s_barrier publishes every wave's
    // share.  The last step issues nothing and is peeled off, so that every
    // path through a step has the same loads in flight (the compiler's own
    // waits then stay out of the way).  An item with no valid frame still
    // waits for the first step's DMAs.
    auto step = [&](int s, auto MORE) {
        constexpr bool more = decltype(MORE)::value;
        const int j0 = SK * s + AK * grp;
        const bool act = j0 < vl;
        wait_vmcnt<PPW + KPW>();   // K
        __builtin_amdgcn_s_barrier();
        if (act) qk();
        wait_vmcnt<KPW>();         // the band
        __builtin_amdgcn_s_barrier();
        if (act) {
            band();
            softmax(s, j0);
        }
        if constexpr (more) {
            __builtin_amdgcn_s_barrier();   // K and the band are read
            dma_k(s + 1);
            dma_p(s + 1);
            wait_vmcnt<PPW + KPW>();        // V (the next K and band behind it)
        } else {
            wait_vmcnt<0>();
        }
        __builtin_amdgcn_s_barrier();
        if (act) pv();
        if constexpr (more) {
            __builtin_amdgcn_s_barrier();   // V is read
            dma_v(s + 1);
        }
    };
    const int nst = max(nit, 1);
    for (int s = 0; s + 1 < nst; ++s) step(s, std::true_type{});
    step(nst - 1, std::false_type{});

    // ---- two key groups: merged, group 0 finishing the dims of the first
    // NDT / 2 blocks d, group 1 the rest.  Each wave leaves the other half of
    // its state in its own G area (no other wave reads it: no barrier
    // before), as 16-byte chunks [chunk][lane]; after one barrier it finishes
    // its half from its partner's area.  Stores: 8 bytes per lane and block
    // (the four lanes of a query cover 32 contiguous bytes) ----
    lrow = xg_sum(lrow);
    const int i = i0w + lc;
    f16* orow = (f16*)a.out + (rowq + i) * a.ldo + h * DK + 4 * lg;
    if constexpr (NG == 1) {
        const float inv = (i < vl && lrow > 0.f) ? 1.0f / lrow : 0.f;   // padded query rows are zero
        if (i < T) {
#pragma unroll
            for (int d = 0; d < NDT; ++d) {
                half4v hv;
#pragma unroll
                for (int r = 0; r < 4; ++r) hv[r] = (f16)(o[d][r] * inv);
                *(half4v*)(orow + 16 * d) = hv;
            }
        }
    } else {
        constexpr int NH = NDT / 2;
        constexpr int MR4 = (4 * NH + 2 + 3) / 4;   // float4 per lane handed over: o of NH blocks, m and l
        static_assert(MR4 * 64 * 16 <= sizeof(sm.g[0]), "merge area");
        float4v* hand = (float4v*)sm.g[w] + lane;
        // the partner: same queries, other keys
        const float4v* take = (const float4v*)sm.g[grp == 0 ? w + NQW : w - NQW] + lane;
        auto give = [&](auto D0) {
            constexpr int d0 = decltype(D0)::value;
            float x[MR4 * 4];
#pragma unroll
            for (int e = 0; e < MR4 * 4; ++e) x[e] = 0.f;
#pragma unroll
            for (int dd = 0; dd < NH; ++dd)
#pragma unroll
                for (int r = 0; r < 4; ++r) x[4 * dd + r] = o[d0 + dd][r];
            x[4 * NH] = mrow;
            x[4 * NH + 1] = lrow;
#pragma unroll
            for (int c = 0; c < MR4; ++c)
                hand[c * 64] = (float4v){x[4 * c], x[4 * c + 1], x[4 * c + 2], x[4 * c + 3]};
        };
        auto keep = [&](auto D0) {
            constexpr int d0 = decltype(D0)::value;
            float y[MR4 * 4];
#pragma unroll
            for (int c = 0; c < MR4; ++c) {
                const float4v t = take[c * 64];
                y[4 * c] = t[0];
                y[4 * c + 1] = t[1];
                y[4 * c + 2] = t[2];
                y[4 * c + 3] = t[3];
            }
            const float m1 = y[4 * NH], l1 = y[4 * NH + 1];
            const float m = fmaxf(mrow, m1);
            const float c0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mrow - m);
            const float c1 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - m);
            const float l = lrow * c0 + l1 * c1;
            const float inv = (i < vl && l > 0.f) ? 1.0f / l : 0.f;   // padded query rows are zero
            if (i < T) {
#pragma unroll
                for (int dd = 0; dd < NH; ++dd) {
                    half4v hv;
#pragma unroll
                    for (int r = 0; r < 4; ++r) hv[r] = (f16)((o[d0 + dd][r] * c0 + y[4 * dd + r] * c1) * inv);
                    *(half4v*)(orow + 16 * (d0 + dd)) = hv;
                }
            }
        };
        if (grp == 0) give(std::integral_constant<int, NH>{});
        else give(std::integral_constant<int, 0>{});
        __syncthreads();
        if (grp == 0) keep(std::integral_constant<int, 0>{});
        else keep(std::integral_constant<int, NH>{});
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
        require(a.ldq % 8 == 0 && a.ldk % 8 == 0 && a.ldv % 8 == 0 && a.ldp % 8 == 0 && a.ldo % 4 == 0,
                "attention(f16): row strides must keep 16-byte input rows and 8-byte output pieces aligned");
        // 64 queries per block, two key groups of four waves, steps of 128 keys
        // staged by DMA (offsets within a head's band rows are 32-bit)
        require(((int64_t)(2 * a.T - 2) * a.ldp + a.dk) * 2 < ((int64_t)1 << 31) &&
                    ((int64_t)(a.T + 127) * std::max(a.ldk, a.ldv) + a.dk) * 2 < ((int64_t)1 << 31),
                "attention(f16): an item's key rows or a head's positional rows span 2 GiB or more");
        // Blocks run one per CU (LDS).  When the last round of 64-query
        // blocks would leave the chip partly idle, 96-query blocks of one key
        // group (six waves, 1.5x the work each) are taken if they need
        // fewer rounds by that measure (T' = 375 at batch 8: 384 -> 256).
        const int cus = device_cu_count();
        const int64_t nb64 = (int64_t)cdiv(a.T, 64) * a.H * a.B, nb96 = (int64_t)cdiv(a.T, 96) * a.H * a.B;
        require(nb64 < ((int64_t)1 << 22), "attention(f16): more than 2^22 query blocks");
        const bool wide = 3 * ((nb96 + cus - 1) / cus) < 2 * ((nb64 + cus - 1) / cus);
        auto go = [&](auto DKc) {
            constexpr int D = decltype(DKc)::value;
            if (wide) launch(relpos_attn_ks_kernel<D, 6, 1>, dim3(nb96), dim3(384), 0, s, a);
            else launch(relpos_attn_ks_kernel<D, 4, 2>, dim3(nb64), dim3(512), 0, s, a);
        };
        if (a.dk == 128) go(std::integral_constant<int, 128>{});
        else if (a.dk == 64) go(std::integral_constant<int, 64>{});
        else if (a.dk == 32) go(std::integral_constant<int, 32>{});
        else throw std::invalid_argument("attention(f16): head dim must be 32, 64 or 128");
    } else {
        const size_t smem = sizeof(float) * (2 * (size_t)a.dk + (size_t)a.T);
        require(smem <= 64 * 1024, "attention(f32): T too large for the LDS score row");
        launch(relpos_attn_f32_kernel, dim3(a.T, a.H, a.B), dim3(64), smem, s, a, a.dk);
    }
    PKX_LAUNCH_CHECK();
}

}  // namespace pkx

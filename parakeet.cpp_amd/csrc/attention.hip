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
// K / V^T / band staging needs block-wide barriers.
#include "attention.hpp"

namespace pkx {

// ---------------------------------------------------------------------------
// f16 MFMA kernel.  NW waves per block, 16 query rows per wave (AQ = 16 NW).
// ---------------------------------------------------------------------------
constexpr int AK = 64;   // keys per tile

template <int DK, int NW>
struct AttnSmem {
    static constexpr int AQ = 16 * NW;
    static constexpr int APB = (AQ + AK - 1 + 15) / 16 * 16;  // positional band rows per key tile
    static constexpr int LDK = DK + 8;   // K and P rows (halves)
    static constexpr int LDV = AK + 8;   // transposed V rows (halves)
    static constexpr int LDG = 80;       // band product (floats)
    static constexpr int LDP = AK + 8;   // probabilities (halves)
    f16 k[AK * LDK];
    f16 vt[DK * LDV];
    f16 p[APB * LDK];
    float g[NW][16 * LDG];
    f16 prob[NW][16 * LDP];
};

template <int DK, int NW>
__global__ __launch_bounds__(64 * NW, 1) void relpos_attn_f16_kernel(AttnParams a) {
    static_assert(DK % 32 == 0, "head dim must be a multiple of 32");
    typedef AttnSmem<DK, NW> S;
    constexpr int AQ = S::AQ, NT = 64 * NW;
    __shared__ __attribute__((aligned(16))) S sm;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int b = blockIdx.z, h = blockIdx.y, i0 = blockIdx.x * AQ;
    const int T = a.T, P = 2 * T - 1;
    const int vl = a.valid ? a.valid[b] : T;
    const int i0w = i0 + 16 * w;
    const float scale = a.scale;
    const f16* q = (const f16*)a.q;
    const f16* k = (const f16*)a.k;
    const f16* v = (const f16*)a.v;
    const f16* pp = (const f16*)a.p;
    const int64_t rowq = (int64_t)b * T;

    // Query fragments (A operand of v_mfma_f32_16x16x32_f16): row lane%16,
    // k = 32*kc + 8*(lane/16) + [0..7].  pos_bias_u/v added in f32.
    constexpr int NKC = DK / 32;
    half8v qu[NKC], qv[NKC];
    {
        const int i = i0w + (lane & 15);
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
            const int c0 = 32 * kc + 8 * (lane >> 4);
            half8v x = {};
            if (i < T) x = *(const half8v*)(q + (rowq + i) * a.ldq + h * DK + c0);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xf = (float)x[e];
                qu[kc][e] = (f16)(xf + a.bias_u[h * DK + c0 + e]);
                qv[kc][e] = (f16)(xf + a.bias_v[h * DK + c0 + e]);
            }
        }
    }

    constexpr int NDT = DK / 16;
    float4v o[NDT];
#pragma unroll
    for (int d = 0; d < NDT; ++d) o[d] = (float4v){0.f, 0.f, 0.f, 0.f};
    float mrow[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    float lrow[4] = {0.f, 0.f, 0.f, 0.f};
    const int lr = 4 * (lane >> 4), lc = lane & 15;

    // Staging of one key tile (K rows, V as 8x8 blocks, the positional band)
    // through registers: all of a tile's global loads are issued together, and
    // the next tile's loads are in flight while the current tile is computed.
    constexpr int KCH = AK * (DK / 8), VCH = (AK / 8) * (DK / 8), PCH = S::APB * (DK / 8);
    constexpr int KPT = (KCH + NT - 1) / NT, VPT = (VCH + NT - 1) / NT, PPT = (PCH + NT - 1) / NT;
    half8v kreg[KPT], vreg[VPT][8], preg[PPT];
    auto load_tile = [&](int j0) {
        const int rlo = T - 1 - (i0 + AQ - 1) + j0;
#pragma unroll
        for (int u = 0; u < KPT; ++u) {
            const int c = tid + NT * u, r = c / (DK / 8), col = (c % (DK / 8)) * 8, j = j0 + r;
            kreg[u] = (c < KCH && j < T) ? *(const half8v*)(k + (rowq + j) * a.ldk + h * DK + col) : (half8v){};
        }
#pragma unroll
        for (int u = 0; u < VPT; ++u) {
            const int c = tid + NT * u, kg = c % (AK / 8), dg = c / (AK / 8);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int j = j0 + 8 * kg + e;
                vreg[u][e] = (c < VCH && j < T) ? *(const half8v*)(v + (rowq + j) * a.ldv + h * DK + 8 * dg)
                                                : (half8v){};
            }
        }
#pragma unroll
        for (int u = 0; u < PPT; ++u) {
            const int c = tid + NT * u, r = c / (DK / 8), col = (c % (DK / 8)) * 8, pr = rlo + r;
            preg[u] = (c < PCH && pr >= 0 && pr < P) ? *(const half8v*)(pp + (int64_t)pr * a.ldp + h * DK + col)
                                                     : (half8v){};
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int u = 0; u < KPT; ++u) {
            const int c = tid + NT * u;
            if (c < KCH) *(half8v*)(sm.k + (c / (DK / 8)) * S::LDK + (c % (DK / 8)) * 8) = kreg[u];
        }
        // V^T: the 8 x 8 block is transposed in registers, keys contiguous
#pragma unroll
        for (int u = 0; u < VPT; ++u) {
            const int c = tid + NT * u, kg = c % (AK / 8), dg = c / (AK / 8);
            if (c < VCH) {
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    half8v col;
#pragma unroll
                    for (int e = 0; e < 8; ++e) col[e] = vreg[u][e][d];
                    *(half8v*)(sm.vt + (8 * dg + d) * S::LDV + 8 * kg) = col;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < PPT; ++u) {
            const int c = tid + NT * u;
            if (c < PCH) *(half8v*)(sm.p + (c / (DK / 8)) * S::LDK + (c % (DK / 8)) * 8) = preg[u];
        }
    };

    load_tile(0);
    for (int j0 = 0; j0 < vl; j0 += AK) {
        store_tile();
        __syncthreads();
        if (j0 + AK < vl) load_tile(j0 + AK);

        // ---- ac = qu . k^T : 16 x 64 per wave ----
        float4v sac[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            sac[jt] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < NKC; ++kc) {
                const half8v kf = *(const half8v*)(sm.k + (16 * jt + lc) * S::LDK + 32 * kc + 8 * (lane >> 4));
                sac[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qu[kc], kf, sac[jt], 0, 0, 0);
            }
        }
        // ---- band product G = qv . p_band^T : 16 x 80, band rows start at AQ - 16 - 16 w ----
        {
            const int pb = AQ - 16 - 16 * w;
#pragma unroll
            for (int gt = 0; gt < 5; ++gt) {
                float4v g = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kc = 0; kc < NKC; ++kc) {
                    const half8v pf = *(const half8v*)(sm.p + (pb + 16 * gt + lc) * S::LDK + 32 * kc + 8 * (lane >> 4));
                    g = __builtin_amdgcn_mfma_f32_16x16x32_f16(qv[kc], pf, g, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) sm.g[w][(lr + r) * S::LDG + 16 * gt + lc] = g[r];
            }
        }
        // each wave reads back only its own G rows: a wave-local barrier suffices
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();

        // ---- scores, rel_shift gather, key mask, online softmax ----
        float s[4][4];
        float tmax[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int ii = lr + r, jj = 16 * jt + lc;
                const float bd = sm.g[w][ii * S::LDG + 15 - ii + jj];   // bd[i][T-1-i+j]
                float sv = (sac[jt][r] + bd) * scale;
                if (j0 + jj >= vl) sv = -INFINITY;
                if (a.chunk > 0) {
                    const int dc = (i0w + ii) / a.chunk - (j0 + jj) / a.chunk;
                    if (dc < 0 || dc > a.left_chunks) sv = -INFINITY;
                }
                s[jt][r] = sv;
                tmax[r] = fmaxf(tmax[r], sv);
            }
#pragma unroll
        for (int r = 0; r < 4; ++r) tmax[r] = row16_max(tmax[r]);   // over the tile's 64 keys
        float corr[4], tsum[4];
        float msub[4];   // the running max, 0 while every key so far is masked (no -inf - -inf)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float mnew = fmaxf(mrow[r], tmax[r]);
            msub[r] = mnew == -INFINITY ? 0.f : mnew;
            corr[r] = __expf(mrow[r] - msub[r]);   // exp(-inf) = 0 on the first tile
            mrow[r] = mnew;
            tsum[r] = 0.f;
        }
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __expf(s[jt][r] - msub[r]);
                tsum[r] += e;
                sm.prob[w][(lr + r) * S::LDP + 16 * jt + lc] = (f16)e;
            }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            tsum[r] = group_sum(tsum[r], 16);
            lrow[r] = lrow[r] * corr[r] + tsum[r];
        }
#pragma unroll
        for (int d = 0; d < NDT; ++d)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[d][r] *= corr[r];
        // the probabilities are wave-private too
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();

        // ---- o += prob . v : A = prob (16 x 64 keys), B = v^T rows ----
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            const half8v pf = *(const half8v*)(sm.prob[w] + lc * S::LDP + 32 * kc + 8 * (lane >> 4));
#pragma unroll
            for (int d = 0; d < NDT; ++d) {
                const half8v vf = *(const half8v*)(sm.vt + (16 * d + lc) * S::LDV + 32 * kc + 8 * (lane >> 4));
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf, vf, o[d], 0, 0, 0);
            }
        }
        __syncthreads();   // the next tile's staging overwrites K, V^T and the band
    }

    // ---- normalise, zero padded query rows, merge heads into ctx[b*T+i][h*DK+c] ----
    f16* out = (f16*)a.out;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int i = i0w + lr + r;
        if (i >= T) continue;
        const float inv = (i < vl && lrow[r] > 0.f) ? 1.0f / lrow[r] : 0.f;
#pragma unroll
        for (int d = 0; d < NDT; ++d)
            out[(rowq + i) * a.ldo + h * DK + 16 * d + lc] = (f16)(o[d][r] * inv);
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
        // 32 queries (2 waves) per block: twice the blocks of a 64-query tiling
        // and an LDS footprint that lets two blocks share a CU.
        constexpr int NW = 4;
        const dim3 grid(cdiv(a.T, 16 * NW), a.H, a.B);
        if (a.dk == 128) {
            launch(relpos_attn_f16_kernel<128, NW>, grid, dim3(64 * NW), 0, s, a);
        } else if (a.dk == 64) {
            launch(relpos_attn_f16_kernel<64, NW>, grid, dim3(64 * NW), 0, s, a);
        } else if (a.dk == 32) {
            launch(relpos_attn_f16_kernel<32, NW>, grid, dim3(64 * NW), 0, s, a);
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

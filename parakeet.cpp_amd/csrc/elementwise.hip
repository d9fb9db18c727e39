// Memory-bound kernels of the encoder path (see elementwise.hpp for the
// reference ops each one replaces).  All are single passes over HBM with
// 16-byte (f32) / 8-byte (f16) vector accesses along the channel dim.
#include "elementwise.hpp"

#include <type_traits>

namespace pkx {

// ---------------------------------------------------------------------------
// LayerNorm: one wave per row, the row held in registers (NV float4 per lane).
// A wave past the last row returns as a whole, so every reducing wave has all
// 64 lanes active.
// ---------------------------------------------------------------------------
// gamma/beta are loaded by the caller before the row statistics are formed,
// so their memory latency overlaps the reductions instead of following them.
// Returns the row's {mean, rstd}.
template <int NV>
__device__ __forceinline__ float2v ln_row(float4v (&v)[NV], int lane, int D, const float4v (&gg)[NV],
                                          const float4v (&bb)[NV], float eps) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = (lane + 64 * i) * 4;
        if (c < D) s += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
    }
    const float mean = wave_sum_full(s) / (float)D;
    float s2 = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = (lane + 64 * i) * 4;
        if (c < D) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = v[i][e] - mean;
                v[i][e] = d;
                s2 += d * d;
            }
        }
    }
    const float rs = 1.0f / sqrtf(wave_sum_full(s2) / (float)D + eps);
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[i][e] = (v[i][e] * rs) * gg[i][e] + bb[i][e];
    return (float2v){mean, rs};
}

template <int NV>
__device__ __forceinline__ void ld_row4(float4v (&v)[NV], const float* src, int lane, int D) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = (lane + 64 * i) * 4;
        v[i] = c < D ? *(const float4v*)(src + c) : (float4v){0.f, 0.f, 0.f, 0.f};
    }
}

template <typename T> __device__ __forceinline__ void store4(T* p, const float4v& v);
template <> __device__ __forceinline__ void store4<float>(float* p, const float4v& v) { *(float4v*)p = v; }
template <> __device__ __forceinline__ void store4<f16>(f16* p, const float4v& v) {
    half4v h = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
    *(half4v*)p = h;
}

// MODE 0: y = LN(x); MODE 1: y_f32 = LN(x), y = LN2(y_f32); MODE 2: y_f32 = LN(x);
// MODE 3: y = silu(LN(x)); MODE 4: y = LN2(LN(x)) and LN's per-row {mean, rstd}
// in rows, x unchanged (the consumer of LN(x) recomputes it from the two).
template <int NV, typename OutT, int MODE>
__global__ __launch_bounds__(256) void layernorm_kernel(LnParams p) {
    constexpr bool TWO = MODE == 1 || MODE == 4;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.M) return;
    float4v v[NV], g1[NV], b1[NV], g2[TWO ? NV : 1], b2[TWO ? NV : 1];
    ld_row4<NV>(v, p.x + row * p.D, lane, p.D);
    ld_row4<NV>(g1, p.g, lane, p.D);
    ld_row4<NV>(b1, p.b, lane, p.D);
    if constexpr (TWO) {
        ld_row4<NV>(g2, p.g2, lane, p.D);
        ld_row4<NV>(b2, p.b2, lane, p.D);
    }
    const float2v st = ln_row<NV>(v, lane, p.D, g1, b1, p.eps);
    if constexpr (MODE == 4) {
        if (lane == 0) ((float2v*)p.rows)[row] = st;
        ln_row<NV>(v, lane, p.D, g2, b2, p.eps);
    }
    if constexpr (MODE == 1 || MODE == 2) {
        float* yr = p.y_f32 + row * p.D;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = (lane + 64 * i) * 4;
            if (c < p.D) *(float4v*)(yr + c) = v[i];
        }
        if constexpr (MODE == 2) return;
        else ln_row<NV>(v, lane, p.D, g2, b2, p.eps);
    }
    if constexpr (MODE == 3) {
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[i][e] = silu_dev(v[i][e]);
    }
    OutT* yo = (OutT*)p.y + row * p.D;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = (lane + 64 * i) * 4;
        if (c < p.D) store4<OutT>(yo + c, v[i]);
    }
}

template <int NV, typename OutT>
static void ln_go(const LnParams& p, hipStream_t s) {
    const dim3 grid(cdiv(p.M, 4));
    if (p.silu)
        launch((layernorm_kernel<NV, OutT, 3>), grid, dim3(256), 0, s, p);
    else if (p.y_f32 && p.y)
        launch((layernorm_kernel<NV, OutT, 1>), grid, dim3(256), 0, s, p);
    else if (p.y_f32)
        launch((layernorm_kernel<NV, OutT, 2>), grid, dim3(256), 0, s, p);
    else if (p.rows)
        launch((layernorm_kernel<NV, OutT, 4>), grid, dim3(256), 0, s, p);
    else
        launch((layernorm_kernel<NV, OutT, 0>), grid, dim3(256), 0, s, p);
}

template <typename OutT>
static void ln_nv(const LnParams& p, hipStream_t s) {
    const int nv = cdiv(p.D, 256);
    if (nv <= 1) ln_go<1, OutT>(p, s);
    else if (nv <= 2) ln_go<2, OutT>(p, s);
    else if (nv <= 4) ln_go<4, OutT>(p, s);
    else if (nv <= 8) ln_go<8, OutT>(p, s);
    else if (nv <= 16) ln_go<16, OutT>(p, s);
    else throw std::invalid_argument("layernorm: D > 4096");
}

void launch_layernorm(Precision prec, const LnParams& p, hipStream_t s) {
    require(p.D % 4 == 0, "layernorm: D must be a multiple of 4");
    require(!p.silu || (p.y && !p.y_f32), "layernorm: the SiLU output is the activation-type y only");
    require(!p.rows || (p.y && !p.y_f32 && !p.silu && p.g2 && p.b2),
            "layernorm: row statistics go with the two-LayerNorm activation output only");
    if (p.M == 0) return;
    if (prec == PREC_F16) ln_nv<f16>(p, s);
    else ln_nv<float>(p, s);
    PKX_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// Depthwise conv1d + bias (+ folded BatchNorm + SiLU) over [B][T][D]: padl
// zero frames precede each item ((K-1)/2 symmetric, K-1 causal,
// conformer.cpp:81-120).  BNSILU: y = silu((conv + b) * scale + shift) in the
// input type; otherwise y = conv + b in f32 (the LayerNorm conv norm follows
// in its own pass).  A block takes a 128-byte channel slice of TC frames: it
// stages those frames and their K-1 halo frames once in LDS (coalesced
// 16-byte rows, zeros outside the item), then each thread computes TC/32
// consecutive frames of one 16-byte channel vector from a window in
// registers.  LDS rows are padded to 160 bytes, so the 16 lanes of a read
// group (two row groups, four rows apart) hit 16 distinct bank quads.
// ---------------------------------------------------------------------------
template <typename T, typename OutT, int K, int TC, bool BNSILU>
__global__ __launch_bounds__(256) void dwconv_lds_kernel(const T* in, OutT* out, const float* w, const float* dwb,
                                                         const float* sc, const float* sh, int Tn, int D, int padl) {
    constexpr int VEC = 16 / sizeof(T);   // channels per 16-byte vector
    constexpr int CV = 8;                 // vectors per staged row (128 bytes)
    constexpr int RG = 256 / CV;          // row groups
    constexpr int RT = TC / RG;           // output frames per thread
    constexpr int NR = TC + K - 1;        // staged frames
    static_assert(TC % RG == 0, "frames per thread");
    __shared__ int4v tile[NR][CV + 2];
    const int cv = threadIdx.x % CV, rg = threadIdx.x / CV;
    const int cb = blockIdx.x * CV * VEC;   // the block's first channel
    const int t0 = blockIdx.y * TC, b = blockIdx.z;
    const T* base = in + (int64_t)b * Tn * D;
    constexpr int NL = (NR * CV + 255) / 256;   // staging loads per thread, all issued before the first store
    int4v x[NL];
#pragma unroll
    for (int u = 0; u < NL; ++u) {
        const int i = threadIdx.x + 256 * u, r = i / CV, v = i % CV;
        const int t = t0 - padl + r, c = cb + v * VEC;
        x[u] = (int4v){0, 0, 0, 0};
        if (i < NR * CV && t >= 0 && t < Tn && c < D) x[u] = *(const int4v*)(base + (int64_t)t * D + c);
    }
#pragma unroll
    for (int u = 0; u < NL; ++u) {
        const int i = threadIdx.x + 256 * u;
        if (i < NR * CV) tile[i / CV][i % CV] = x[u];
    }
    // the block's taps [CV VEC][K] and per-channel constants, one coalesced
    // pass into LDS (per-thread scalar loads of 8 channels x K taps would
    // take most of the kernel's time)
    constexpr int CB = CV * VEC;
    __shared__ float wsm[CB * K], csm[3][CB];
    for (int i = threadIdx.x; i < CB * K; i += 256) wsm[i] = cb * K + i < D * K ? w[cb * K + i] : 0.f;
    for (int i = threadIdx.x; i < CB; i += 256) {
        const int c = min(cb + i, D - 1);
        csm[0][i] = dwb ? dwb[c] : 0.f;
        csm[1][i] = BNSILU ? sc[c] : 1.f;
        csm[2][i] = BNSILU ? sh[c] : 0.f;
    }
    const int c0 = cb + cv * VEC;
    __syncthreads();
    if (c0 >= D) return;
    float wk[VEC][K], bias[VEC], scale[VEC], shift[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
#pragma unroll
        for (int k = 0; k < K; ++k) wk[e][k] = wsm[(cv * VEC + e) * K + k];
        bias[e] = csm[0][cv * VEC + e];
        scale[e] = csm[1][cv * VEC + e];
        shift[e] = csm[2][cv * VEC + e];
    }
    float win[RT + K - 1][VEC];
#pragma unroll
    for (int r = 0; r < RT + K - 1; ++r) {
        const int4v xr = tile[rg * RT + r][cv];
        const T* xv = (const T*)&xr;
#pragma unroll
        for (int e = 0; e < VEC; ++e) win[r][e] = (float)xv[e];
    }
    OutT* ob = out + (int64_t)b * Tn * D + c0;
#pragma unroll
    for (int tt = 0; tt < RT; ++tt) {
        const int t = t0 + rg * RT + tt;
        if (t >= Tn) break;
        OutT o[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < K; ++k) acc += wk[e][k] * win[tt + k][e];
            if constexpr (BNSILU) o[e] = to_act<OutT>(silu_dev((acc + bias[e]) * scale[e] + shift[e]));
            else o[e] = acc + bias[e];
        }
        OutT* dst = ob + (int64_t)t * D;
#pragma unroll
        for (int h = 0; h < (int)(sizeof(OutT) * VEC / 16); ++h) ((int4v*)dst)[h] = ((const int4v*)o)[h];
    }
}

template <typename ET, int K>
static void dw_go(const void* in, void* out, const float* w, const float* dwb, const float* sc,
                  const float* sh, int B, int Tn, int D, int padl, hipStream_t s) {
    // blocks of 64 frames x 128 bytes of channels (an encoder item of 125
    // frames and 1024 f16 channels: 2 x 16 blocks)
    constexpr int TC = 64, VEC = 16 / sizeof(ET);
    const dim3 grid(cdiv(D / VEC, 8), cdiv(Tn, TC), B);
    if (sc)
        launch((dwconv_lds_kernel<ET, ET, K, TC, true>), grid, dim3(256), 0, s, (const ET*)in, (ET*)out, w, dwb, sc,
               sh, Tn, D, padl);
    else
        launch((dwconv_lds_kernel<ET, float, K, TC, false>), grid, dim3(256), 0, s, (const ET*)in, (float*)out, w,
               dwb, sc, sh, Tn, D, padl);
}

template <typename ET>
static void dw_k(const void* in, void* out, const float* w, const float* dwb, const float* sc,
                 const float* sh, int B, int Tn, int D, int K, int padl, hipStream_t s) {
    switch (K) {
    case 3: dw_go<ET, 3>(in, out, w, dwb, sc, sh, B, Tn, D, padl, s); break;
    case 5: dw_go<ET, 5>(in, out, w, dwb, sc, sh, B, Tn, D, padl, s); break;
    case 7: dw_go<ET, 7>(in, out, w, dwb, sc, sh, B, Tn, D, padl, s); break;
    case 9: dw_go<ET, 9>(in, out, w, dwb, sc, sh, B, Tn, D, padl, s); break;
    case 15: dw_go<ET, 15>(in, out, w, dwb, sc, sh, B, Tn, D, padl, s); break;
    case 31: dw_go<ET, 31>(in, out, w, dwb, sc, sh, B, Tn, D, padl, s); break;
    default: throw std::invalid_argument("dwconv: unsupported kernel size");
    }
}

void launch_dwconv(Precision prec, const void* in, void* out, const float* w, const float* dw_bias,
                   const float* bn_scale, const float* bn_shift, int B, int T, int D, int K, bool causal,
                   hipStream_t s) {
    if (B == 0 || T == 0) return;
    require(D % 8 == 0, "dwconv: D must be a multiple of 8");
    require((bn_scale == nullptr) == (bn_shift == nullptr), "dwconv: BatchNorm scale and shift go together");
    const int padl = causal ? K - 1 : (K - 1) / 2;
    if (prec == PREC_F16) dw_k<f16>(in, out, w, dw_bias, bn_scale, bn_shift, B, T, D, K, padl, s);
    else dw_k<float>(in, out, w, dw_bias, bn_scale, bn_shift, B, T, D, K, padl, s);
    PKX_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// Subsampling convs (H = time, W = feature; ggml conv layout [W,H,C,N]).
// ---------------------------------------------------------------------------
// Depthwise 3x3 stride-2 conv (+bias) on a channels-last map [B][Ti][Fi][C],
// rows t >= vmask[b] read as zero; pl = zero padding before each axis (1
// symmetric, 2 causal, subsampling.cpp:81-99).  A thread owns 8 channels (16-byte loads
// and stores, 32 threads cover 256 channels contiguously) and a set of output
// columns of one output row; the 3x3 window loads hit L1/L2 for the 2.25x
// overlap between neighbouring outputs.
template <typename T>
__global__ __launch_bounds__(256) void sub_dwconv_kernel(const T* in, const int* vmask, const float* w,
                                                         const float* bias, T* out, int Ti, int Fi,
                                                         int C, int To, int Fo, int pl) {
    constexpr int V = 16 / sizeof(T);                  // channels per thread
    const int to = blockIdx.x, b = blockIdx.y;
    const int groups = C / V, lanes_f = blockDim.x / groups;
    const int g = threadIdx.x % groups, c0 = g * V;
    if ((int)threadIdx.x >= groups * lanes_f) return;
    const int vlim = vmask ? vmask[b] : Ti;
    float wk[V][9], bb[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
        bb[e] = bias[c0 + e];
#pragma unroll
        for (int q = 0; q < 9; ++q) wk[e][q] = w[(c0 + e) * 9 + q];
    }
    for (int fo = threadIdx.x / groups; fo < Fo; fo += lanes_f) {
        float acc[V];
#pragma unroll
        for (int e = 0; e < V; ++e) acc[e] = bb[e];
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) {
            const int ti = 2 * to - pl + kh;
            if (ti < 0 || ti >= Ti || ti >= vlim) continue;
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) {
                const int fi = 2 * fo - pl + kw;
                if (fi < 0 || fi >= Fi) continue;
                const T* src = in + (((int64_t)b * Ti + ti) * Fi + fi) * C + c0;
                T x[V];
                *(int4v*)x = *(const int4v*)src;
#pragma unroll
                for (int e = 0; e < V; ++e) acc[e] += wk[e][kh * 3 + kw] * (float)x[e];
            }
        }
        T y[V];
#pragma unroll
        for (int e = 0; e < V; ++e) y[e] = to_act<T>(acc[e]);
        *(int4v*)(out + (((int64_t)b * To + to) * Fo + fo) * C + c0) = *(const int4v*)y;
    }
}

// First two subsampling stages fused: conv0 (1 -> C, 3x3, stride 2, pad 1)
// + bias + ReLU, the stage mask on its output rows, then the depthwise 3x3
// stride-2 conv + bias, written as [B][T2][F2][C].  The conv0 map (the
// largest tensor of the encoder: B x T/2 x F/2 x C) never leaves registers.
// A block takes one item and two output rows t2, t2+1; those need conv0 rows
// t1 = 2 t2 - 1 .. 2 t2 + 3 and mel rows 4 t2 - 3 .. 4 t2 + 7, which are
// staged in LDS (zero-padded, masked at t >= valid0).  One thread per channel
// walks the feature axis with a sliding 3-column window of conv0 values, so
// each conv0 value is computed once per block (the row shared by the two
// output rows included).  pl = zero padding before each axis: 1 symmetric
// (the rows and columns above), 2 causal (subsampling.cpp:81-99: conv0 rows
// 2 t2 - 2 .. 2 t2 + 2, mel rows 4 t2 - 6 .. 4 t2 + 4).
template <typename T>
__global__ __launch_bounds__(256) void sub_stage1_kernel(const float* mel, const int* valid0, const int* valid1,
                                                         const float* w0, const float* b0, const float* w2,
                                                         const float* b2, T* out, int F, int Tn, int C, int T1,
                                                         int F1, int T2, int F2, int pl) {
    extern __shared__ float mp[];                 // [11][4 F2 + 5]: mel columns 2 - 3 pl .. 4 F2 + 4 - 3 pl
    // f16 output: the mel tile is staged as f16 (rows of FPH halves, even so
    // that column pairs are 4-byte aligned) and conv0 runs as packed f16
    // products with f32 accumulation (v_dot2_f32_f16); a second tile holds
    // vertical pairs (rows j, j + 1 of one column) for the kw = 2 taps
    constexpr bool H = std::is_same<T, f16>::value;
    const int b = blockIdx.y, t2a = 2 * blockIdx.x;
    const int FP = 4 * F2 + 5, FPH = FP + 1;
    f16* mh = (f16*)mp;
    half2v* mv = (half2v*)(mh + 11 * FPH);        // [10][FP]
    const int v0 = valid0 ? valid0[b] : Tn;
    const int v1 = valid1 ? valid1[b] : T1;
    // time fastest across the threads: mel is [B][F][T], so 11 consecutive
    // threads read one feature's 44 contiguous bytes
    for (int idx = threadIdx.x; idx < 11 * FP; idx += blockDim.x) {
        const int j = idx % 11, q = idx / 11, fi = q - (3 * pl - 2);
        const int t = 4 * t2a - 3 * pl + j;
        float v = 0.f;
        if (t >= 0 && t < Tn && t < v0 && fi >= 0 && fi < F) v = mel[((int64_t)b * F + fi) * Tn + t];
        if constexpr (H) mh[j * FPH + q] = (f16)v;
        else mp[j * FP + q] = v;
    }
    __syncthreads();
    if constexpr (H) {
        for (int idx = threadIdx.x; idx < 10 * FP; idx += blockDim.x) {
            const int j = idx / FP, q = idx % FP;
            mv[idx] = (half2v){mh[j * FPH + q], mh[(j + 1) * FPH + q]};
        }
        __syncthreads();
    }
    bool rowok[5];
#pragma unroll
    for (int r = 0; r < 5; ++r) {
        const int t1 = 2 * t2a - pl + r;
        rowok[r] = t1 >= 0 && t1 < T1 && t1 < v1;
    }
    const bool has_b = t2a + 1 < T2;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        float k0[9], k2[9];
#pragma unroll
        for (int e = 0; e < 9; ++e) {
            k0[e] = w0[c * 9 + e];
            k2[e] = w2[c * 9 + e];
        }
        const float bc0 = b0[c], bc2 = b2[c];
        // f16 taps: (kw 0, kw 1) of each row, (kh 0, kh 1) at kw 2, and kw 2 of kh 2
        half2v w01[3], w2v;
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) w01[kh] = (half2v){(f16)k0[kh * 3], (f16)k0[kh * 3 + 1]};
        w2v = (half2v){(f16)k0[2], (f16)k0[5]};
        const float w22 = (float)(f16)k0[8];
        float prev[5];
#pragma unroll
        for (int r = 0; r < 5; ++r) prev[r] = 0.f;    // conv0 column f1 = -pl is padding
        for (int f2 = 0; f2 < F2; ++f2) {
            // mel columns 4 f2 + 2 - 3 pl .. 4 f2 + 6 - 3 pl (LDS columns 4 f2 .. 4 f2 + 4)
            float ca[5], cb[5];                       // conv0 columns f1 = 2 f2 - pl + 1, 2 f2 - pl + 2
            const int f1a = 2 * f2 - pl + 1;
            const bool fa = f1a >= 0 && f1a < F1, fb = f1a + 1 >= 0 && f1a + 1 < F1;
            if constexpr (H) {
                half2v p01[11], p23[11], v2[5], v4[5];
                f16 m4[11];
#pragma unroll
                for (int j = 0; j < 11; ++j) {
                    const f16* row = mh + j * FPH + 4 * f2;
                    p01[j] = *(const half2v*)row;
                    p23[j] = *(const half2v*)(row + 2);
                    m4[j] = row[4];
                }
#pragma unroll
                for (int r = 0; r < 5; ++r) {   // rows 2 r, 2 r + 1 at columns 4 f2 + 2 and 4 f2 + 4
                    v2[r] = mv[2 * r * FP + 4 * f2 + 2];
                    v4[r] = mv[2 * r * FP + 4 * f2 + 4];
                }
#pragma unroll
                for (int r = 0; r < 5; ++r) {
                    float sa = bc0, sb = bc0;
#pragma unroll
                    for (int kh = 0; kh < 3; ++kh) {
                        sa = __builtin_amdgcn_fdot2(p01[2 * r + kh], w01[kh], sa, false);
                        sb = __builtin_amdgcn_fdot2(p23[2 * r + kh], w01[kh], sb, false);
                    }
                    sa = __builtin_amdgcn_fdot2(v2[r], w2v, sa, false);
                    sb = __builtin_amdgcn_fdot2(v4[r], w2v, sb, false);
                    sa += w22 * (float)p23[2 * r + 2][0];
                    sb += w22 * (float)m4[2 * r + 2];
                    // ReLU and the masks (row, column; uniform over the block)
                    ca[r] = rowok[r] && fa ? fmaxf(sa, 0.f) : 0.f;
                    cb[r] = rowok[r] && fb ? fmaxf(sb, 0.f) : 0.f;
                }
            } else {
                float m[11][5];
#pragma unroll
                for (int j = 0; j < 11; ++j)
#pragma unroll
                    for (int q = 0; q < 5; ++q) m[j][q] = mp[j * FP + 4 * f2 + q];
#pragma unroll
                for (int r = 0; r < 5; ++r) {
                    float sa = bc0, sb = bc0;
#pragma unroll
                    for (int kh = 0; kh < 3; ++kh)
#pragma unroll
                        for (int kw = 0; kw < 3; ++kw) {
                            sa += k0[kh * 3 + kw] * m[2 * r + kh][kw];
                            sb += k0[kh * 3 + kw] * m[2 * r + kh][2 + kw];
                        }
                    ca[r] = (rowok[r] && fa && sa > 0.f) ? sa : 0.f;
                    cb[r] = (rowok[r] && fb && sb > 0.f) ? sb : 0.f;
                }
            }
            float oa = bc2, ob = bc2;
#pragma unroll
            for (int kh = 0; kh < 3; ++kh) {
                oa += k2[kh * 3] * prev[kh] + k2[kh * 3 + 1] * ca[kh] + k2[kh * 3 + 2] * cb[kh];
                ob += k2[kh * 3] * prev[2 + kh] + k2[kh * 3 + 1] * ca[2 + kh] + k2[kh * 3 + 2] * cb[2 + kh];
            }
            out[(((int64_t)b * T2 + t2a) * F2 + f2) * C + c] = to_act<T>(oa);
            if (has_b) out[(((int64_t)b * T2 + t2a + 1) * F2 + f2) * C + c] = to_act<T>(ob);
#pragma unroll
            for (int r = 0; r < 5; ++r) prev[r] = cb[r];
        }
    }
}

void launch_sub_stage1(Precision prec, const float* mel, const int* valid0, const int* valid1, const float* w0,
                       const float* b0, const float* w2, const float* b2, void* out, int B, int F, int T, int C,
                       hipStream_t s, bool causal) {
    const int T1 = sub_stage_len(T, causal), F1 = sub_stage_len(F, causal);
    const int T2 = sub_stage_len(T1, causal), F2 = sub_stage_len(F1, causal);
    const int pl = causal ? 2 : 1;
    const dim3 grid(cdiv(T2, 2), B);
    const int bs = C >= 256 ? 256 : ((C + 63) / 64) * 64;
    // 4 F2 + 5 >= F + 2 covers the zero padding; f32 tile [11][FP], f16 tile
    // [11][FP + 1] followed by the vertical pairs [10][FP]
    const uint32_t FP = 4 * F2 + 5;
    const uint32_t shm = prec == PREC_F16 ? 11u * (FP + 1) * 2u + 10u * FP * 4u : 11u * FP * 4u;
    if (prec == PREC_F16)
        launch(sub_stage1_kernel<f16>, grid, dim3(bs), shm, s, mel, valid0, valid1, w0, b0, w2, b2, (f16*)out, F, T,
               C, T1, F1, T2, F2, pl);
    else
        launch(sub_stage1_kernel<float>, grid, dim3(bs), shm, s, mel, valid0, valid1, w0, b0, w2, b2, (float*)out,
               F, T, C, T1, F1, T2, F2, pl);
    PKX_LAUNCH_CHECK();
}

void launch_sub_dwconv(Precision prec, const void* in, const int* vmask, const float* w,
                       const float* bias, void* out, int B, int Ti, int Fi, int C, hipStream_t s, bool causal) {
    const int To = sub_stage_len(Ti, causal), Fo = sub_stage_len(Fi, causal), pl = causal ? 2 : 1;
    require(C % 8 == 0 && C <= 2048, "subsampling: channels must be a multiple of 8 and at most 2048");
    const dim3 grid(To, B);
    const int bs = 256;
    if (prec == PREC_F16)
        launch(sub_dwconv_kernel<f16>, grid, dim3(bs), 0, s, (const f16*)in, vmask, w, bias, (f16*)out, Ti, Fi, C, To,
               Fo, pl);
    else
        launch(sub_dwconv_kernel<float>, grid, dim3(bs), 0, s, (const float*)in, vmask, w, bias, (float*)out, Ti, Fi,
               C, To, Fo, pl);
    PKX_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// Relative positional table in f64 (positions +(T-1) .. -(T-1)).
// ---------------------------------------------------------------------------
template <typename T>
__global__ void rel_pos_kernel(T* out, int Tn, int D) {
    const int half = D / 2;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t P = 2 * (int64_t)Tn - 1;
    if (idx >= P * half) return;
    const int p = (int)(idx / half), i = (int)(idx % half);
    const double factor = -(log(10000.0) / (double)D);
    const double div = exp((double)(2 * i) * factor);
    const double a = (double)((Tn - 1) - p) * div;
    out[(int64_t)p * D + 2 * i] = to_act<T>((float)sin(a));
    out[(int64_t)p * D + 2 * i + 1] = to_act<T>((float)cos(a));
}

void launch_rel_pos_encoding(Precision prec, void* out, int T, int D, hipStream_t s) {
    require(D % 2 == 0, "pos_enc: D must be even");
    const int64_t n = (2 * (int64_t)T - 1) * (D / 2);
    if (prec == PREC_F16)
        launch(rel_pos_kernel<f16>, dim3(cdiv(n, 256)), dim3(256), 0, s, (f16*)out, T, D);
    else
        launch(rel_pos_kernel<float>, dim3(cdiv(n, 256)), dim3(256), 0, s, (float*)out, T, D);
    PKX_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// Heads: log-softmax + argmax, split argmax.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void argmax_merge(float& bv, int& bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
    }
}
__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        argmax_merge(bv, bi, ov, oi);
    }
}

__global__ __launch_bounds__(256) void log_softmax_argmax_kernel(const float* x, float* y, int32_t* am,
                                                                 int64_t M, int V) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const float* xr = x + row * V;
    float* yr = y + row * V;
    float mx = -INFINITY;
    for (int v = lane; v < V; v += 64) mx = fmaxf(mx, xr[v]);
    mx = wave_max(mx);
    float sum = 0.f;
    for (int v = lane; v < V; v += 64) sum += expf(xr[v] - mx);
    const float lse = logf(wave_sum(sum));
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int v = lane; v < V; v += 64) {
        const float lp = (xr[v] - mx) - lse;
        yr[v] = lp;
        argmax_merge(bv, bi, lp, v);
    }
    wave_argmax(bv, bi);
    if (lane == 0) am[row] = bi;
}

__global__ __launch_bounds__(256) void split_argmax_kernel(const float* x, int64_t M, int nt, int nd,
                                                           int32_t* tok, int32_t* dur) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const float* xr = x + row * (nt + nd);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int v = lane; v < nt; v += 64) argmax_merge(bv, bi, xr[v], v);
    wave_argmax(bv, bi);
    float dv = -INFINITY;
    int di = 0x7fffffff;
    for (int v = lane; v < nd; v += 64) argmax_merge(dv, di, xr[nt + v], v);
    wave_argmax(dv, di);
    if (lane == 0) {
        tok[row] = bi;
        dur[row] = di;
    }
}

void launch_log_softmax_argmax(const float* logits, float* logprobs, int32_t* argmax, int64_t M,
                               int V, hipStream_t s) {
    if (M == 0) return;
    launch(log_softmax_argmax_kernel, dim3(cdiv(M, 4)), dim3(256), 0, s, logits, logprobs, argmax, M, V);
    PKX_LAUNCH_CHECK();
}

// Loads this file's code object on the current device (the runtime loads it
// at the first launch otherwise, taking device memory then).
void elementwise_module_ready() {
    hipFuncAttributes a;
    PKX_HIP(hipFuncGetAttributes(&a, (const void*)split_argmax_kernel));
}

void launch_split_argmax(const float* logits, int64_t M, int n_tok, int n_dur, int32_t* tok,
                         int32_t* dur, hipStream_t s) {
    if (M == 0) return;
    launch(split_argmax_kernel, dim3(cdiv(M, 4)), dim3(256), 0, s, logits, M, n_tok, n_dur, tok, dur);
    PKX_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// Cast / add
// ---------------------------------------------------------------------------
template <typename T>
__global__ void cast_f32_kernel(const float* x, T* y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = to_act<T>(x[i]);
}
__global__ void add_f32_kernel(float* x, const float* y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] += y[i];
}
void launch_cast_f32(Precision prec, const float* x, void* y, int64_t n, hipStream_t s) {
    if (n == 0) return;
    if (prec == PREC_F16)
        launch(cast_f32_kernel<f16>, dim3(cdiv(n, 256)), dim3(256), 0, s, x, (f16*)y, n);
    else
        launch(cast_f32_kernel<float>, dim3(cdiv(n, 256)), dim3(256), 0, s, x, (float*)y, n);
    PKX_LAUNCH_CHECK();
}
void launch_add_f32(float* x, const float* y, int64_t n, hipStream_t s) {
    if (n == 0) return;
    launch(add_f32_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, x, y, n);
    PKX_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// [B][T][D] -> per-item [D][valid[b]] (32x32 LDS tile transpose).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void compact_cf_kernel(const float* x, int Tn, int D, const int* valid,
                                                         const int64_t* offs, float* out) {
    __shared__ float tile[32][33];
    const int b = blockIdx.z, t0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
    const int vb = valid[b];
    if (t0 >= vb) return;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const int t = t0 + r, c = c0 + tx;
        tile[r][tx] = (t < vb && c < D) ? x[((int64_t)b * Tn + t) * D + c] : 0.f;
    }
    __syncthreads();
    float* ob = out + offs[b];
    for (int r = ty; r < 32; r += 8) {
        const int c = c0 + r, t = t0 + tx;
        if (c < D && t < vb) ob[(int64_t)c * vb + t] = tile[tx][r];
    }
}

void launch_compact_channels_first(const float* x, int B, int T, int D, const int* valid,
                                   const int64_t* offs, float* out, hipStream_t s) {
    const dim3 grid(cdiv(T, 32), cdiv(D, 32), B);
    launch(compact_cf_kernel, grid, dim3(256), 0, s, x, T, D, valid, offs, out);
    PKX_LAUNCH_CHECK();
}

}  // namespace pkx

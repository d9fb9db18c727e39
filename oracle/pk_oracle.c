/*
 * pk_oracle.c -- CPU restatement of the parakeet.cpp encoder path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker + "port" CPU baseline); the
 * product library never links it.  See pk_oracle.h for the layout contract.
 * Each function cites the reference file:line whose graph it restates.
 *
 * Arithmetic conventions (the reference's ggml kernels are absent):
 *   - dot products: f32 products summed in f32 lane partials (ggml's SIMD
 *     sgemm accumulates the same way), OpenMP over output rows;
 *   - LayerNorm statistics in f64 with an f32 mean (ggml_norm_f32);
 *   - softmax / log-softmax statistics in f64;
 *   - BatchNorm fold in f32 exactly as conformer.cpp:144-147.
 */
#include "pk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0;

void orc_set_threads(int n) {
    g_threads = n;
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* binary16                                                                  */
/* ------------------------------------------------------------------------ */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    float f;
    if (ex == 0) {
        /* zero or subnormal: man * 2^-24, exact in f32 */
        f = (float)man * 5.9604644775390625e-8f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);       /* NaN */
    if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);      /* >= 2^16 -> inf */
    if (ax < 0x38800000u) {
        /* below 2^-14: subnormal result, mantissa = RNE(|f| * 2^24) (exact scale) */
        float af;
        memcpy(&af, &ax, 4);
        return (uint16_t)(sign | (uint16_t)rintf(af * 16777216.0f));
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;       /* carries into inf correctly */
    return (uint16_t)(sign | h);
}

/* ------------------------------------------------------------------------ */
/* Block formats (docs/quantization.md; ggml v0.13.0 block_q8_0 / block_q4_K) */
/* ------------------------------------------------------------------------ */

#define QK8_0 32
#define Q8_0_BYTES 34
#define QK_K 256
#define Q4_K_BYTES 144

int64_t orc_row_bytes(int type, int64_t ne0) {
    switch (type) {
    case ORC_F32: return ne0 * 4;
    case ORC_F16: return ne0 * 2;
    case ORC_Q8_0: return (ne0 % QK8_0) ? 0 : (ne0 / QK8_0) * Q8_0_BYTES;
    case ORC_Q4_K: return (ne0 % QK_K) ? 0 : (ne0 / QK_K) * Q4_K_BYTES;
    default: return 0;
    }
}

static uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static void wr_u16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* 6-bit scale/min of sub-block j from the 12 packed bytes. */
static void q4k_scale_min(int j, const uint8_t* q, int* sc, int* mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

int orc_dequantize(int type, const void* src, float* dst, int64_t n) {
    const uint8_t* s = (const uint8_t*)src;
    if (type == ORC_F32) { memcpy(dst, src, (size_t)n * 4); return 0; }
    if (type == ORC_F16) {
        for (int64_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(rd_u16(s + 2 * i));
        return 0;
    }
    if (type == ORC_Q8_0) {
        if (n % QK8_0) return 1;
        for (int64_t b = 0; b < n / QK8_0; ++b) {
            const uint8_t* blk = s + b * Q8_0_BYTES;
            float d = orc_f16_to_f32(rd_u16(blk));
            for (int j = 0; j < QK8_0; ++j) dst[b * QK8_0 + j] = (float)(int8_t)blk[2 + j] * d;
        }
        return 0;
    }
    if (type == ORC_Q4_K) {
        if (n % QK_K) return 1;
        for (int64_t b = 0; b < n / QK_K; ++b) {
            const uint8_t* blk = s + b * Q4_K_BYTES;
            float d = orc_f16_to_f32(rd_u16(blk));
            float dmin = orc_f16_to_f32(rd_u16(blk + 2));
            const uint8_t* scales = blk + 4;
            const uint8_t* qs = blk + 16;
            float* y = dst + b * QK_K;
            for (int c = 0; c < 4; ++c) {          /* 64-element chunk: two sub-blocks */
                int sc, mn;
                q4k_scale_min(2 * c, scales, &sc, &mn);
                float d1 = d * (float)sc, m1 = dmin * (float)mn;
                q4k_scale_min(2 * c + 1, scales, &sc, &mn);
                float d2 = d * (float)sc, m2 = dmin * (float)mn;
                for (int l = 0; l < 32; ++l) y[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0xF) - m1;
                for (int l = 0; l < 32; ++l) y[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - m2;
            }
        }
        return 0;
    }
    return 2;
}

/* ggml's quantisers (ggml v0.13.0 ggml-quants.c, the published algorithms
 * ggml_quantize_chunk runs for parakeet-cli quantize, examples/cli/main.cpp:
 * 322-426).  Compiled without FMA contraction. */
static int nearest_int(float fval) {
    /* round to nearest, ties to even, via the 1.5 * 2^23 magic constant */
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

/* make_qkx2_quants: affine (scale, min) fit of n values to [0, nmax] by
 * weighted least squares over nstep+1 candidate scales; returns the scale,
 * *the_min = -min. */
__attribute__((optimize("fp-contract=off")))
static float make_qkx2_quants(int n, int nmax, const float* x, const float* weights, uint8_t* L,
                              float* the_min, uint8_t* Laux, float rmin, float rdelta, int nstep) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_mad = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)(l < 0 ? 0 : l > nmax ? nmax : l);
        float diff = scale * L[i] + min - x[i];
        diff = diff * diff;
        best_mad += weights[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : l > nmax ? nmax : l;
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                mad += weights[i] * diff;
            }
            if (mad < best_mad) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_mad = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

static void get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

/* quantize_row_q4_K_ref for one 256-value super-block */
__attribute__((optimize("fp-contract=off")))
static void quantize_q4_k_block(const float* x, uint8_t* blk) {
    uint8_t L[QK_K], Laux[32], sc[12];
    float weights[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = make_qkx2_quants(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    memset(sc, 0, sizeof sc);
    for (int j = 0; j < 8; ++j) {
        uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
        uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
        ls = ls < 63 ? ls : 63;
        lm = lm < 63 ? lm : 63;
        if (j < 4) {
            sc[j] = ls;
            sc[j + 4] = lm;
        } else {
            sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
            sc[j - 0] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    const uint16_t dh = orc_f32_to_f16(max_scale / 63.f), mh = orc_f32_to_f16(max_min / 63.f);
    for (int j = 0; j < 8; ++j) {
        uint8_t s, m;
        get_scale_min_k4(j, sc, &s, &m);
        const float d = orc_f16_to_f32(dh) * s;
        if (!d) continue;
        const float dm = orc_f16_to_f32(mh) * m;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest_int((x[32 * j + ii] + dm) / d);
            L[32 * j + ii] = (uint8_t)(l < 0 ? 0 : l > 15 ? 15 : l);
        }
    }
    wr_u16(blk, dh);
    wr_u16(blk + 2, mh);
    memcpy(blk + 4, sc, 12);
    uint8_t* q = blk + 16;
    for (int j = 0; j < QK_K; j += 64) {
        for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
        q += 32;
    }
}

/* quantize_row_q8_0_ref */
__attribute__((optimize("fp-contract=off")))
static void quantize_q8_0_block(const float* v, uint8_t* blk) {
    float amax = 0.f;
    for (int j = 0; j < QK8_0; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / ((1 << 7) - 1);
    const float id = d ? 1.0f / d : 0.0f;
    wr_u16(blk, orc_f32_to_f16(d));
    for (int j = 0; j < QK8_0; ++j) blk[2 + j] = (uint8_t)(int8_t)roundf(v[j] * id);
}

int orc_quantize(int type, const float* x, void* dst, int64_t n) {
    uint8_t* o = (uint8_t*)dst;
    if (type == ORC_F32) { memcpy(dst, x, (size_t)n * 4); return 0; }
    if (type == ORC_F16) {
        for (int64_t i = 0; i < n; ++i) wr_u16(o + 2 * i, orc_f32_to_f16(x[i]));
        return 0;
    }
    if (type == ORC_Q8_0) {
        if (n % QK8_0) return 1;
        for (int64_t b = 0; b < n / QK8_0; ++b) quantize_q8_0_block(x + b * QK8_0, o + b * Q8_0_BYTES);
        return 0;
    }
    if (type == ORC_Q4_K) {
        if (n % QK_K) return 1;
        for (int64_t b = 0; b < n / QK_K; ++b) quantize_q4_k_block(x + b * QK_K, o + b * Q4_K_BYTES);
        return 0;
    }
    return 2;
}

/* ------------------------------------------------------------------------ */
/* Positional encoding: pos_enc.cpp:10-34                                    */
/* ------------------------------------------------------------------------ */

void orc_rel_pos_encoding(int T, int d, float* out) {
    const int P = 2 * T - 1, half = d / 2;
    const double factor = -(log(10000.0) / (double)d);
    double* div = (double*)malloc(sizeof(double) * (size_t)half);
    for (int i = 0; i < half; ++i) div[i] = exp((double)(2 * i) * factor);
    for (int p = 0; p < P; ++p) {
        const double pos = (double)((T - 1) - p);
        for (int i = 0; i < half; ++i) {
            const double a = pos * div[i];
            out[(size_t)p * d + 2 * i] = (float)sin(a);
            out[(size_t)p * d + 2 * i + 1] = (float)cos(a);
        }
    }
    free(div);
}

/* ------------------------------------------------------------------------ */
/* LayerNorm: conformer.cpp:300-307 (ggml_norm + mul + add)                  */
/* ------------------------------------------------------------------------ */

void orc_layer_norm(const float* x, int64_t M, int D, const float* g,
                    const float* b, float eps, float* y) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        const float* xr = x + m * D;
        float* yr = y + m * D;
        double sum = 0.0;
        for (int i = 0; i < D; ++i) sum += xr[i];
        const float mean = (float)(sum / D);
        double sum2 = 0.0;
        for (int i = 0; i < D; ++i) {
            const float v = xr[i] - mean;
            yr[i] = v;
            sum2 += (double)(v * v);
        }
        const float scale = 1.0f / sqrtf((float)(sum2 / D) + eps);
        for (int i = 0; i < D; ++i) {
            float t = yr[i] * scale;
            t = t * g[i];
            yr[i] = t + b[i];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Linear: y = x . W^T + b  (ggml_mul_mat(W, x) + ggml_add)                  */
/* ------------------------------------------------------------------------ */

typedef float v8f __attribute__((vector_size(32)));

static inline v8f ld8(const float* p) { v8f v; memcpy(&v, p, 32); return v; }
static inline float hsum8(v8f v) {
    return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
}

void orc_linear(const float* x, int64_t M, int K, const float* W, int N,
                const float* bias, float* y) {
    const int K8 = K & ~7;
    const int64_t Mb = (M + 1) / 2;
    const int Nb = (N + 3) / 4;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t mb = 0; mb < Mb; ++mb) {
        for (int nb = 0; nb < Nb; ++nb) {
            const int64_t m0 = 2 * mb;
            const int n0 = 4 * nb;
            const int mc = (M - m0) < 2 ? (int)(M - m0) : 2;
            const int nc = (N - n0) < 4 ? (N - n0) : 4;
            const float* xr[2];
            const float* wr[4];
            for (int i = 0; i < 2; ++i) xr[i] = x + (size_t)(m0 + (i < mc ? i : 0)) * K;
            for (int j = 0; j < 4; ++j) wr[j] = W + (size_t)(n0 + (j < nc ? j : 0)) * K;
            v8f acc[2][4];
            for (int i = 0; i < 2; ++i)
                for (int j = 0; j < 4; ++j) acc[i][j] = (v8f){0, 0, 0, 0, 0, 0, 0, 0};
            for (int k = 0; k < K8; k += 8) {
                const v8f a0 = ld8(xr[0] + k), a1 = ld8(xr[1] + k);
                for (int j = 0; j < 4; ++j) {
                    const v8f w = ld8(wr[j] + k);
                    acc[0][j] += a0 * w;
                    acc[1][j] += a1 * w;
                }
            }
            for (int i = 0; i < mc; ++i)
                for (int j = 0; j < nc; ++j) {
                    float s = hsum8(acc[i][j]);
                    for (int k = K8; k < K; ++k) s += xr[i][k] * wr[j][k];
                    if (bias) s += bias[n0 + j];
                    y[(size_t)(m0 + i) * N + n0 + j] = s;
                }
        }
    }
}

static float silu_f(float v) { return (float)((double)v / (1.0 + exp(-(double)v))); }
static float sigmoid_f(float v) { return (float)(1.0 / (1.0 + exp(-(double)v))); }

static float* fbuf(size_t n) { return (float*)malloc(n * sizeof(float)); }

/* ------------------------------------------------------------------------ */
/* Rel-pos MHSA: relpos_attention.cpp:162-306                                */
/* ------------------------------------------------------------------------ */

void orc_relpos_attention(const orc_layer* L, const float* x, int B, int T,
                          const float* pe, const int* valid, float* out) {
    const int D = L->D, H = L->H, dk = D / H, P = 2 * T - 1;
    const int64_t M = (int64_t)B * T;
    const float scale = 1.0f / sqrtf((float)dk);
    const int chunk = L->att_limited ? L->att_right + 1 : 1;   /* relpos_attention.cpp:30-38 */
    const int left_chunks = L->att_limited ? L->att_left / chunk : 0;
    float* q = fbuf((size_t)M * D);
    float* k = fbuf((size_t)M * D);
    float* v = fbuf((size_t)M * D);
    float* p = fbuf((size_t)P * D);
    float* ctx = fbuf((size_t)M * D);
    orc_linear(x, M, D, L->wq, D, L->bq, q);                  /* :191 */
    orc_linear(x, M, D, L->wk, D, L->bk, k);                  /* :192 */
    orc_linear(x, M, D, L->wv, D, L->bv, v);                  /* :193 */
    orc_linear(pe, P, D, L->wpos, D, NULL, p);                /* :194, no bias */

#pragma omp parallel
    {
        double* sc = (double*)malloc(sizeof(double) * (size_t)T);
        float* qu = fbuf((size_t)dk);
        float* qv = fbuf((size_t)dk);
#pragma omp for collapse(3) schedule(static)
        for (int b = 0; b < B; ++b)
            for (int h = 0; h < H; ++h)
                for (int i = 0; i < T; ++i) {
                    const int vl = valid ? valid[b] : T;
                    float* cr = ctx + ((size_t)b * T + i) * D + (size_t)h * dk;
                    if (i >= vl) {                            /* :291-302 query mask */
                        for (int c = 0; c < dk; ++c) cr[c] = 0.f;
                        continue;
                    }
                    const float* qr = q + ((size_t)b * T + i) * D + (size_t)h * dk;
                    for (int c = 0; c < dk; ++c) {            /* :213-220 */
                        qu[c] = qr[c] + L->pos_bias_u[h * dk + c];
                        qv[c] = qr[c] + L->pos_bias_v[h * dk + c];
                    }
                    double mx = -INFINITY;
                    for (int j = 0; j < T; ++j) {
                        if (j >= vl) { sc[j] = -INFINITY; continue; }   /* :252-277 key mask */
                        if (L->att_limited) {                 /* :252-270 chunked-limited window */
                            const int diff = i / chunk - j / chunk;
                            if (diff < 0 || diff > left_chunks) { sc[j] = -INFINITY; continue; }
                        }
                        const float* kr = k + ((size_t)b * T + j) * D + (size_t)h * dk;
                        /* rel_shift (:226-238): bd_shift[i][j] = bd[i][T-1-i+j] */
                        const float* pr = p + (size_t)(T - 1 - i + j) * D + (size_t)h * dk;
                        float ac = 0.f, bd = 0.f;
                        for (int c = 0; c < dk; ++c) { ac += qu[c] * kr[c]; bd += qv[c] * pr[c]; }
                        const float s = (ac + bd) * scale;    /* softmax(scale*scores + mask) */
                        sc[j] = s;
                        if (s > mx) mx = s;
                    }
                    double den = 0.0;
                    for (int j = 0; j < vl; ++j) { sc[j] = exp(sc[j] - mx); den += sc[j]; }
                    for (int c = 0; c < dk; ++c) {
                        double acc = 0.0;
                        for (int j = 0; j < vl; ++j)
                            acc += sc[j] * v[((size_t)b * T + j) * D + (size_t)h * dk + c];
                        cr[c] = (float)(acc / den);
                    }
                }
        free(sc);
        free(qu);
        free(qv);
    }
    orc_linear(ctx, M, D, L->wo, D, L->bo, out);              /* :305 */
    free(q); free(k); free(v); free(p); free(ctx);
}

/* ------------------------------------------------------------------------ */
/* Conv module: conformer.cpp:38-164 (symmetric or causal depthwise pad,    */
/* batch_norm or layer_norm between the depthwise conv and SiLU)             */
/* ------------------------------------------------------------------------ */

void orc_conv_module(const orc_layer* L, const float* c, int B, int T,
                     const int* valid, float* out) {
    const int D = L->D, K = L->K, pad = L->conv_causal ? K - 1 : (K - 1) / 2;   /* :100-116 */
    const int64_t M = (int64_t)B * T;
    float* y = fbuf((size_t)M * 2 * D);
    float* g = fbuf((size_t)M * D);
    float* n = fbuf((size_t)M * D);
    float* bsc = fbuf((size_t)D);
    float* bsh = fbuf((size_t)D);
    orc_linear(c, M, D, L->pw1_w, 2 * D, L->pw1_b, y);        /* :48-53 */
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {                          /* :55-80 GLU + pad mask */
        const int b = (int)(m / T), t = (int)(m % T);
        const int vl = valid ? valid[b] : T;
        for (int ch = 0; ch < D; ++ch) {
            const float a = y[m * 2 * D + ch], gate = y[m * 2 * D + D + ch];
            g[m * D + ch] = (t < vl) ? a * sigmoid_f(gate) : 0.f;
        }
    }
    for (int ch = 0; ch < D && !L->conv_ln; ++ch) {            /* :134-154 BN fold */
        bsc[ch] = L->bn_g[ch] / sqrtf(L->bn_var[ch] + 1e-5f);
        bsh[ch] = L->bn_b[ch] - L->bn_mean[ch] * bsc[ch];
    }
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t)
            for (int ch = 0; ch < D; ++ch) {                   /* :81-124 depthwise, :157 SiLU */
                float acc = 0.f;
                for (int kk = 0; kk < K; ++kk) {
                    const int ts = t + kk - pad;
                    if (ts < 0 || ts >= T) continue;
                    acc += L->dw_w[ch * K + kk] * g[((size_t)b * T + ts) * D + ch];
                }
                if (L->dw_b) acc += L->dw_b[ch];
                if (L->conv_ln) {                              /* normalised below */
                    n[((size_t)b * T + t) * D + ch] = acc;
                    continue;
                }
                float nv = acc * bsc[ch];
                nv = nv + bsh[ch];
                n[((size_t)b * T + t) * D + ch] = silu_f(nv);
            }
    if (L->conv_ln) {                                          /* :128-133 norm over channels, SiLU */
        orc_layer_norm(n, M, D, L->bn_g, L->bn_b, 1e-5f, n);
        for (int64_t i = 0; i < M * D; ++i) n[i] = silu_f(n[i]);
    }
    orc_linear(n, M, D, L->pw2_w, D, L->pw2_b, out);          /* :158-162 */
    free(y); free(g); free(n); free(bsc); free(bsh);
}

/* ------------------------------------------------------------------------ */
/* Conformer layer: conformer.cpp:285-353                                    */
/* ------------------------------------------------------------------------ */

static void ffn(const float* xin, int64_t M, int D, int FF, const float* w1,
                const float* b1, const float* w2, const float* b2, float* out) {
    float* h = fbuf((size_t)M * FF);
    orc_linear(xin, M, D, w1, FF, b1, h);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M * FF; ++i) h[i] = silu_f(h[i]);
    orc_linear(h, M, FF, w2, D, b2, out);
    free(h);
}

void orc_conformer_layer(const orc_layer* L, const float* x, int B, int T,
                         const float* pe, const int* valid, float* out,
                         float* conv_out) {
    const int D = L->D;
    const int64_t M = (int64_t)B * T, MD = M * D;
    const float eps = 1e-5f;
    float* r = fbuf((size_t)MD);
    float* t1 = fbuf((size_t)MD);
    float* t2 = fbuf((size_t)MD);
    /* Stage A: r = x + 0.5*FFN1(LN(x)) */
    orc_layer_norm(x, M, D, L->ff1_ln_g, L->ff1_ln_b, eps, t1);
    ffn(t1, M, D, L->FF, L->ff1_w1, L->ff1_b1, L->ff1_w2, L->ff1_b2, t2);
    for (int64_t i = 0; i < MD; ++i) r[i] = x[i] + t2[i] * 0.5f;
    /* Stage B: r += MHSA(LN(r)) */
    orc_layer_norm(r, M, D, L->att_ln_g, L->att_ln_b, eps, t1);
    orc_relpos_attention(L, t1, B, T, pe, valid, t2);
    for (int64_t i = 0; i < MD; ++i) r[i] += t2[i];
    /* Stage C: r += conv(LN(r)) */
    orc_layer_norm(r, M, D, L->conv_ln_g, L->conv_ln_b, eps, t1);
    orc_conv_module(L, t1, B, T, valid, t2);
    if (conv_out) memcpy(conv_out, t2, (size_t)MD * sizeof(float));
    for (int64_t i = 0; i < MD; ++i) r[i] += t2[i];
    /* Stage D: r += 0.5*FFN2(LN(r)); out = LN(r) */
    orc_layer_norm(r, M, D, L->ff2_ln_g, L->ff2_ln_b, eps, t1);
    ffn(t1, M, D, L->FF, L->ff2_w1, L->ff2_b1, L->ff2_w2, L->ff2_b2, t2);
    for (int64_t i = 0; i < MD; ++i) r[i] += t2[i] * 0.5f;
    orc_layer_norm(r, M, D, L->out_ln_g, L->out_ln_b, eps, out);
    free(r); free(t1); free(t2);
}

/* ------------------------------------------------------------------------ */
/* Subsampling: subsampling.cpp:25-46, :48-240, :242-386                     */
/* ------------------------------------------------------------------------ */

/* all_paddings = 2 (symmetric) or 3 (causal: 2 before, 1 after), k 3, s 2 */
int orc_subsampled_len_c(int T, int causal) {
    int t = T;
    for (int s = 0; s < 3; ++s) t = (t + (causal ? 3 : 2) - 3) / 2 + 1;
    return t;
}

int orc_valid_out_len_c(int T, int in_valid, int causal) {
    int v = in_valid >= 0 ? in_valid : T - 1;
    for (int s = 0; s < 3; ++s) v = (v + (causal ? 3 : 2) - 3) / 2 + 1;
    return v;
}

int orc_subsampled_len(int T) { return orc_subsampled_len_c(T, 0); }
int orc_valid_out_len(int T, int in_valid) { return orc_valid_out_len_c(T, in_valid, 0); }

/* 3x3 stride-2 depthwise conv (pad pl before each axis) over a channels-last
 * [Ti][Fi][C] map, reading rows t >= vmask as zero; output channels-last
 * [To][Fo][C] + bias. */
static void dw3x3s2(const float* in, int Ti, int Fi, int C, int vmask, int pl,
                    const float* w, const float* bias, float* out, int To, int Fo) {
    for (int t = 0; t < To; ++t)
        for (int f = 0; f < Fo; ++f)
            for (int c = 0; c < C; ++c) {
                float acc = 0.f;
                for (int kh = 0; kh < 3; ++kh) {
                    const int ti = 2 * t - pl + kh;
                    if (ti < 0 || ti >= Ti || ti >= vmask) continue;
                    for (int kw = 0; kw < 3; ++kw) {
                        const int fi = 2 * f - pl + kw;
                        if (fi < 0 || fi >= Fi) continue;
                        acc += w[c * 9 + kh * 3 + kw] * in[((size_t)ti * Fi + fi) * C + c];
                    }
                }
                out[((size_t)t * Fo + f) * C + c] = acc + bias[c];
            }
}

int orc_subsampling(const orc_subsampling_w* S, const float* mel, int B, int F,
                    int T, const int* valid_in, int stage_masks, float* out,
                    int* valid_out) {
    const int C = S->C, D = S->D;
    /* causal (subsampling.cpp:81-99): pad 2 before / 1 after on time and
     * feature axes, per-stage input time masks on every path (:100-147, :283-300) */
    const int cz = S->causal, pl = cz ? 2 : 1, ap = cz ? 3 : 2;
    if (cz) stage_masks = 1;
    const int T1 = (T + ap - 3) / 2 + 1, F1 = (F + ap - 3) / 2 + 1;
    const int T2 = (T1 + ap - 3) / 2 + 1, F2 = (F1 + ap - 3) / 2 + 1;
    const int T3 = (T2 + ap - 3) / 2 + 1, F3 = (F2 + ap - 3) / 2 + 1;
    float* flat = fbuf((size_t)B * T3 * C * F3);
    for (int b = 0; b < B; ++b) {
        const int v0 = valid_in ? valid_in[b] : T - 1;
        const int v1 = (v0 + ap - 3) / 2 + 1, v2 = (v1 + ap - 3) / 2 + 1;
        const int vo = orc_valid_out_len_c(T, valid_in ? valid_in[b] : -1, cz);
        valid_out[b] = vo > T3 ? T3 : vo;
        const int m0 = stage_masks ? v0 : T, m1 = stage_masks ? v1 : T1, m2 = stage_masks ? v2 : T2;
        const float* mb = mel + (size_t)b * F * T;
        float* a1 = fbuf((size_t)T1 * F1 * C);
        float* a2 = fbuf((size_t)T2 * F2 * C);
        float* a2p = fbuf((size_t)T2 * F2 * C);
        float* a3 = fbuf((size_t)T3 * F3 * C);
        float* a3p = fbuf((size_t)T3 * F3 * C);
        /* conv.0: Conv2d(1->C, 3x3, s2, p1) + bias + ReLU (:143-157); H=time, W=feat */
#pragma omp parallel for collapse(2) schedule(static)
        for (int t = 0; t < T1; ++t)
            for (int f = 0; f < F1; ++f)
                for (int c = 0; c < C; ++c) {
                    float acc = 0.f;
                    for (int kh = 0; kh < 3; ++kh) {
                        const int ti = 2 * t - pl + kh;
                        if (ti < 0 || ti >= T || ti >= m0) continue;
                        for (int kw = 0; kw < 3; ++kw) {
                            const int fi = 2 * f - pl + kw;
                            if (fi < 0 || fi >= F) continue;
                            acc += S->w0[c * 9 + kh * 3 + kw] * mb[(size_t)fi * T + ti];
                        }
                    }
                    acc += S->b0[c];
                    a1[((size_t)t * F1 + f) * C + c] = acc > 0.f ? acc : 0.f;
                }
        /* conv.2 depthwise + bias, conv.3 pointwise + bias + ReLU (:159-192) */
        dw3x3s2(a1, T1, F1, C, m1, pl, S->w2, S->b2, a2, T2, F2);
        orc_linear(a2, (int64_t)T2 * F2, C, S->w3, C, S->b3, a2p);
        for (size_t i = 0; i < (size_t)T2 * F2 * C; ++i) a2p[i] = a2p[i] > 0.f ? a2p[i] : 0.f;
        /* conv.5 depthwise + bias, conv.6 pointwise + bias + ReLU */
        dw3x3s2(a2p, T2, F2, C, m2, pl, S->w5, S->b5, a3, T3, F3);
        orc_linear(a3, (int64_t)T3 * F3, C, S->w6, C, S->b6, a3p);
        for (size_t i = 0; i < (size_t)T3 * F3 * C; ++i) a3p[i] = a3p[i] > 0.f ? a3p[i] : 0.f;
        /* flatten channel-major per time step (idx c*F'+f, :194-202) + mask (:204-230) */
        for (int t = 0; t < T3; ++t)
            for (int c = 0; c < C; ++c)
                for (int f = 0; f < F3; ++f)
                    flat[((size_t)b * T3 + t) * C * F3 + (size_t)c * F3 + f] =
                        (t < valid_out[b]) ? a3p[((size_t)t * F3 + f) * C + c] : 0.f;
        free(a1); free(a2); free(a2p); free(a3); free(a3p);
    }
    orc_linear(flat, (int64_t)B * T3, C * F3, S->wout, D, S->bout, out);  /* :232-236 */
    free(flat);
    return T3;
}

/* ------------------------------------------------------------------------ */
/* Encoder: encoder.cpp:97-167                                               */
/* ------------------------------------------------------------------------ */

int orc_encoder_forward(const orc_subsampling_w* S, const orc_layer* layers,
                        int n_layers, int xscaling, const float* mel, int B,
                        int F, int T, const int* valid_in, int stage_masks,
                        float* out, int* valid_out, float* capture) {
    const int D = S->D;
    const int Tp = orc_subsampled_len_c(T, S->causal);
    const size_t MD = (size_t)B * Tp * D;
    float* x = fbuf(MD);
    float* y = fbuf(MD);
    orc_subsampling(S, mel, B, F, T, valid_in, stage_masks, x, valid_out);
    if (xscaling) {                                            /* :123 / :186 */
        const float s = sqrtf((float)D);
        for (size_t i = 0; i < MD; ++i) x[i] *= s;
    }
    float* pe = fbuf((size_t)(2 * Tp - 1) * D);
    orc_rel_pos_encoding(Tp, D, pe);
    for (int l = 0; l < n_layers; ++l) {
        orc_conformer_layer(&layers[l], x, B, Tp, pe, valid_out, y, NULL);
        if (capture) memcpy(capture + (size_t)l * MD, y, MD * sizeof(float));
        float* tmp = x; x = y; y = tmp;
    }
    memcpy(out, x, MD * sizeof(float));
    free(x); free(y); free(pe);
    return Tp;
}

/* ------------------------------------------------------------------------ */
/* Cache-aware streaming encoder: streaming_encoder.cpp:29-96 (state),       */
/* :98-338 (one layer with its caches), :340-462 (step)                      */
/* ------------------------------------------------------------------------ */

struct orc_stream {
    const orc_subsampling_w* S;
    const orc_layer* layers;
    int n_layers, xscaling, F, D, K;
    int cache_len, drop_extra, valid_out_len;
    int step, clc_len;
    float* cache_ch;   /* [L][cache_len][D]: norm_self_att outputs of earlier frames */
    float* cache_t;    /* [L][K-1][D]: GLU outputs of earlier frames */
};

orc_stream* orc_stream_new(const orc_subsampling_w* S, const orc_layer* layers, int n_layers,
                           int xscaling, int F, int cache_len, int drop_extra, int valid_out_len) {
    orc_stream* st = (orc_stream*)calloc(1, sizeof(orc_stream));
    st->S = S; st->layers = layers; st->n_layers = n_layers; st->xscaling = xscaling;
    st->F = F; st->D = S->D; st->K = layers[0].K;
    st->cache_len = cache_len; st->drop_extra = drop_extra; st->valid_out_len = valid_out_len;
    st->cache_ch = fbuf((size_t)n_layers * cache_len * st->D);
    st->cache_t = fbuf((size_t)n_layers * (st->K - 1) * st->D);
    orc_stream_reset(st);
    return st;
}

void orc_stream_free(orc_stream* st) {
    if (!st) return;
    free(st->cache_ch); free(st->cache_t); free(st);
}

void orc_stream_reset(orc_stream* st) {                       /* :72-79 zeros */
    st->step = 0; st->clc_len = 0;
    memset(st->cache_ch, 0, sizeof(float) * (size_t)st->n_layers * st->cache_len * st->D);
    memset(st->cache_t, 0, sizeof(float) * (size_t)st->n_layers * (st->K - 1) * st->D);
}

int orc_stream_chunk_len(const orc_stream* st, int n) {      /* :350-366 */
    const int drop = st->step != 0 ? st->drop_extra : 0;
    const int tc = orc_subsampled_len_c(n, 1) - drop;
    return tc < 0 ? 0 : tc;
}

/* One conformer layer of the chunk x [Tc][D] with its caches; out [Tc][D]. */
static void stream_layer(const orc_layer* L, const float* x, int Tc, const float* pe, int CL, int clc,
                         float* cache_ch, float* cache_t, float* out) {
    const int D = L->D, H = L->H, dk = D / H, K = L->K, LP = K - 1, FF = L->FF;
    const int Tk = CL + Tc, P = 2 * Tk - 1;
    const size_t MD = (size_t)Tc * D;
    const float scale = 1.0f / sqrtf((float)dk);
    float* r = fbuf(MD);
    float* t1 = fbuf(MD);
    float* t2 = fbuf(MD);
    float* ain = fbuf(MD);
    /* stage A (:139-144): r = x + 0.5 FFN1(LN(x)); attn_in = norm_self_att(r) */
    orc_layer_norm(x, Tc, D, L->ff1_ln_g, L->ff1_ln_b, 1e-5f, t1);
    ffn(t1, Tc, D, FF, L->ff1_w1, L->ff1_b1, L->ff1_w2, L->ff1_b2, t2);
    for (size_t i = 0; i < MD; ++i) r[i] = x[i] + t2[i] * 0.5f;
    orc_layer_norm(r, Tc, D, L->att_ln_g, L->att_ln_b, 1e-5f, ain);
    /* stage B (:146-245): K/V over [cache ; attn_in], Q over attn_in */
    float* kv = fbuf((size_t)Tk * D);
    memcpy(kv, cache_ch, sizeof(float) * (size_t)CL * D);
    memcpy(kv + (size_t)CL * D, ain, sizeof(float) * MD);
    float* q = fbuf(MD);
    float* k = fbuf((size_t)Tk * D);
    float* v = fbuf((size_t)Tk * D);
    float* p = fbuf((size_t)P * D);
    float* ctx = fbuf(MD);
    orc_linear(ain, Tc, D, L->wq, D, L->bq, q);
    orc_linear(kv, Tk, D, L->wk, D, L->bk, k);
    orc_linear(kv, Tk, D, L->wv, D, L->bv, v);
    orc_linear(pe, P, D, L->wpos, D, NULL, p);
    /* mask (:196-222): leading cache_len - clc keys empty; chunked-limited
     * window over key kj and query cache_len + qi */
    const int chunk = L->att_right + 1, left_chunks = chunk > 0 ? L->att_left / chunk : 0;
    const int empty = CL - clc;
    double* sc = (double*)malloc(sizeof(double) * (size_t)Tk);
    for (int h = 0; h < H; ++h)
        for (int i = 0; i < Tc; ++i) {
            const float* qr = q + (size_t)i * D + (size_t)h * dk;
            double mx = -INFINITY;
            for (int j = 0; j < Tk; ++j) {
                const int cq = (CL + i) / chunk, ck = j / chunk, diff = cq - ck;
                if (j < empty || diff < 0 || diff > left_chunks) { sc[j] = -INFINITY; continue; }
                /* rel_shift of a [Tc][P] score block (:180-190): column Tc-1-i+j */
                const float* kr = k + (size_t)j * D + (size_t)h * dk;
                const float* pr = p + (size_t)(Tc - 1 - i + j) * D + (size_t)h * dk;
                float ac = 0.f, bd = 0.f;
                for (int c = 0; c < dk; ++c) {
                    ac += (qr[c] + L->pos_bias_u[h * dk + c]) * kr[c];
                    bd += (qr[c] + L->pos_bias_v[h * dk + c]) * pr[c];
                }
                sc[j] = (double)((ac + bd) * scale);
                if (sc[j] > mx) mx = sc[j];
            }
            double den = 0.0;
            for (int j = 0; j < Tk; ++j) { sc[j] = exp(sc[j] - mx); den += sc[j]; }
            for (int c = 0; c < dk; ++c) {
                double acc = 0.0;
                for (int j = 0; j < Tk; ++j) acc += sc[j] * v[(size_t)j * D + (size_t)h * dk + c];
                ctx[(size_t)i * D + (size_t)h * dk + c] = (float)(acc / den);
            }
        }
    free(sc);
    orc_linear(ctx, Tc, D, L->wo, D, L->bo, t2);
    for (size_t i = 0; i < MD; ++i) r[i] += t2[i];
    /* next attention cache (:247-266): the last CL rows of [cache ; attn_in] */
    memcpy(cache_ch, kv + (size_t)Tc * D, sizeof(float) * (size_t)CL * D);
    /* stage C (:268-330): conv module over [conv cache ; GLU] */
    orc_layer_norm(r, Tc, D, L->conv_ln_g, L->conv_ln_b, 1e-5f, t1);
    float* y = fbuf((size_t)Tc * 2 * D);
    orc_linear(t1, Tc, D, L->pw1_w, 2 * D, L->pw1_b, y);
    float* dwin = fbuf((size_t)(LP + Tc) * D);
    memcpy(dwin, cache_t, sizeof(float) * (size_t)LP * D);
    for (int t = 0; t < Tc; ++t)
        for (int ch = 0; ch < D; ++ch)
            dwin[(size_t)(LP + t) * D + ch] = y[(size_t)t * 2 * D + ch] * sigmoid_f(y[(size_t)t * 2 * D + D + ch]);
    memcpy(cache_t, dwin + (size_t)Tc * D, sizeof(float) * (size_t)LP * D);
    for (int t = 0; t < Tc; ++t)
        for (int ch = 0; ch < D; ++ch) {
            float acc = 0.f;
            for (int kk = 0; kk < K; ++kk) acc += L->dw_w[ch * K + kk] * dwin[(size_t)(t + kk) * D + ch];
            if (L->dw_b) acc += L->dw_b[ch];
            t2[(size_t)t * D + ch] = acc;
        }
    if (L->conv_ln) {
        orc_layer_norm(t2, Tc, D, L->bn_g, L->bn_b, 1e-5f, t2);
    } else {
        for (int t = 0; t < Tc; ++t)
            for (int ch = 0; ch < D; ++ch) {
                const float sc1 = L->bn_g[ch] / sqrtf(L->bn_var[ch] + 1e-5f);
                const float sh1 = L->bn_b[ch] - L->bn_mean[ch] * sc1;
                t2[(size_t)t * D + ch] = t2[(size_t)t * D + ch] * sc1 + sh1;
            }
    }
    for (size_t i = 0; i < MD; ++i) t2[i] = silu_f(t2[i]);
    orc_linear(t2, Tc, D, L->pw2_w, D, L->pw2_b, t1);
    for (size_t i = 0; i < MD; ++i) r[i] += t1[i];
    /* stage D (:332-337) */
    orc_layer_norm(r, Tc, D, L->ff2_ln_g, L->ff2_ln_b, 1e-5f, t1);
    ffn(t1, Tc, D, FF, L->ff2_w1, L->ff2_b1, L->ff2_w2, L->ff2_b2, t2);
    for (size_t i = 0; i < MD; ++i) r[i] += t2[i] * 0.5f;
    orc_layer_norm(r, Tc, D, L->out_ln_g, L->out_ln_b, 1e-5f, out);
    free(r); free(t1); free(t2); free(ain); free(kv); free(q); free(k); free(v); free(p); free(ctx);
    free(y); free(dwin);
}

int orc_stream_step(orc_stream* st, const float* mel, int n, int is_last, float* out) {
    const int D = st->D, CL = st->cache_len;
    const int drop = st->step != 0 ? st->drop_extra : 0;
    const int Tsub = orc_subsampled_len_c(n, 1);
    const int Tc = orc_stream_chunk_len(st, n);
    if (Tc == 0) { st->step += 1; return 0; }                 /* :367-371 */
    float* sx = fbuf((size_t)Tsub * D);
    int vo = 0;
    orc_subsampling(st->S, mel, 1, st->F, n, &n, 1, sx, &vo);   /* whole window is audio */
    float* x = fbuf((size_t)Tc * D);
    float* y = fbuf((size_t)Tc * D);
    memcpy(x, sx + (size_t)drop * D, sizeof(float) * (size_t)Tc * D);
    if (st->xscaling) {
        const float s = sqrtf((float)D);
        for (size_t i = 0; i < (size_t)Tc * D; ++i) x[i] *= s;
    }
    const int Pn = Tc + CL;                                    /* :376-381 */
    float* pe = fbuf((size_t)(2 * Pn - 1) * D);
    orc_rel_pos_encoding(Pn, D, pe);
    for (int l = 0; l < st->n_layers; ++l) {
        stream_layer(&st->layers[l], x, Tc, pe, CL, st->clc_len, st->cache_ch + (size_t)l * CL * D,
                     st->cache_t + (size_t)l * (st->K - 1) * D, y);
        float* tmp = x; x = y; y = tmp;
    }
    st->clc_len = st->clc_len + Tc < CL ? st->clc_len + Tc : CL;  /* :447-448 */
    st->step += 1;
    const int valid = is_last ? Tc : (st->valid_out_len < Tc ? st->valid_out_len : Tc);
    memcpy(out, x, sizeof(float) * (size_t)valid * D);
    free(sx); free(x); free(y); free(pe);
    return valid;
}

/* ------------------------------------------------------------------------ */
/* Output heads                                                              */
/* ------------------------------------------------------------------------ */

void orc_ctc_head(const float* enc, int T, int D, const float* W, const float* b,
                  int V, float* logprobs, int32_t* argmax) {
    orc_linear(enc, T, D, W, V, b, logprobs);                  /* ctc_decoder.cpp:98-102 */
    for (int t = 0; t < T; ++t) {
        float* r = logprobs + (size_t)t * V;
        float mx = r[0];
        for (int v = 1; v < V; ++v) if (r[v] > mx) mx = r[v];
        double den = 0.0;
        for (int v = 0; v < V; ++v) den += exp((double)r[v] - (double)mx);
        for (int v = 0; v < V; ++v)                            /* :107-108 log(softmax) */
            r[v] = (float)(((double)r[v] - (double)mx) - log(den));
        int best = 0;
        for (int v = 1; v < V; ++v) if (r[v] > r[best]) best = v;   /* search.cpp:57-61 */
        argmax[t] = best;
    }
}

int orc_ctc_greedy(const int32_t* argmax, int T, int blank_id, int32_t* out) {
    int n = 0;
    int32_t prev = blank_id;
    for (int t = 0; t < T; ++t) {                              /* search.cpp:63 */
        const int32_t p = argmax[t];
        if ((p != prev || prev == blank_id) && p != blank_id) out[n++] = p;
        prev = p;
    }
    return n;
}

void orc_tdt_joint_argmax(const float* enc, int T, int D, const float* Wenc,
                          const float* benc, int Hj, const float* g, int P,
                          const float* Wpred, const float* bpred,
                          const float* Wout, const float* bout, int n_tok,
                          int n_dur, float* logits, int32_t* tok, int32_t* dur) {
    const int V = n_tok + n_dur;
    float* ep = fbuf((size_t)T * Hj);
    float* pp = fbuf((size_t)Hj);
    float* f = fbuf((size_t)T * Hj);
    orc_linear(enc, T, D, Wenc, Hj, benc, ep);                 /* joint.cpp:37-63 */
    orc_linear(g, 1, P, Wpred, Hj, bpred, pp);                 /* joint.cpp:89-93 */
    for (int t = 0; t < T; ++t)
        for (int h = 0; h < Hj; ++h) {                         /* :94-95 */
            const float s = ep[(size_t)t * Hj + h] + pp[h];
            f[(size_t)t * Hj + h] = s > 0.f ? s : 0.f;
        }
    orc_linear(f, T, Hj, Wout, V, bout, logits);               /* :96-100 */
    for (int t = 0; t < T; ++t) {                              /* tdt.cpp:76-79 */
        const float* r = logits + (size_t)t * V;
        int bt = 0, bd = 0;
        for (int i = 1; i < n_tok; ++i) if (r[i] > r[bt]) bt = i;
        for (int i = 1; i < n_dur; ++i) if (r[n_tok + i] > r[n_tok + bd]) bd = i;
        tok[t] = bt;
        dur[t] = bd;
    }
    free(ep); free(pp); free(f);
}

/* ------------------------------------------------------------------------ */
/* Greedy transducer decode: prediction.cpp, joint.cpp, tdt.cpp,            */
/* transducer_batch.cpp, decode_common.hpp                                   */
/* ------------------------------------------------------------------------ */

static float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }   /* ggml_sigmoid */

void orc_lstm_step(const orc_transducer* m, int32_t token, int is_sos, const float* h_in, const float* c_in,
                   float* h_out, float* c_out, float* g_out) {
    const int H = m->H;
    float* x = fbuf((size_t)H);
    float* za = fbuf((size_t)4 * H);
    float* zb = fbuf((size_t)4 * H);
    for (int j = 0; j < H; ++j) x[j] = is_sos ? 0.0f : m->embed[(size_t)token * H + j];
    for (int l = 0; l < m->L; ++l) {
        orc_linear(x, 1, H, m->w_ih[l], 4 * H, m->b_ih[l], za);            /* W_ih x + b_ih */
        orc_linear(h_in + (size_t)l * H, 1, H, m->w_hh[l], 4 * H, m->b_hh[l], zb);   /* W_hh h + b_hh */
        for (int j = 0; j < H; ++j) {
            const float zi = za[j] + zb[j], zf = za[H + j] + zb[H + j];
            const float zg = za[2 * H + j] + zb[2 * H + j], zo = za[3 * H + j] + zb[3 * H + j];
            const float c = orc_sigmoid(zf) * c_in[(size_t)l * H + j] + orc_sigmoid(zi) * tanhf(zg);
            c_out[(size_t)l * H + j] = c;
            h_out[(size_t)l * H + j] = orc_sigmoid(zo) * tanhf(c);
        }
        for (int j = 0; j < H; ++j) x[j] = h_out[(size_t)l * H + j];
    }
    memcpy(g_out, h_out + (size_t)(m->L - 1) * H, sizeof(float) * (size_t)H);
    free(x); free(za); free(zb);
}

static int orc_argmax_first(const float* a, int n) {         /* decode_common.hpp:5-9 */
    int best = 0;
    float bv = a[0];
    for (int i = 1; i < n; ++i) if (a[i] > bv) { bv = a[i]; best = i; }
    return best;
}

static float orc_max_prob_conf(const float* a, int n, int k) {   /* decode_common.hpp:12-20 */
    float mx = a[0];
    for (int i = 1; i < n; ++i) if (a[i] > mx) mx = a[i];
    double den = 0.0;
    for (int i = 0; i < n; ++i) den += exp((double)a[i] - (double)mx);
    const double p = exp((double)a[k] - (double)mx) / den, N = (double)n;
    return (float)((N * p - 1.0) / (N - 1.0));
}

int orc_transducer_greedy(const orc_transducer* m, const float* enc, int T, const int32_t* durations, int n_dur,
                          int blank_id, int max_symbols, int32_t* ids, int32_t* frames, float* conf,
                          int32_t* span, int cap) {
    const int H = m->H, L = m->L, Hj = m->Hj, Vp = m->Vp;
    const int tc = n_dur > 0 ? Vp - n_dur : Vp;
    float* ep = fbuf((size_t)(T > 0 ? T : 1) * Hj);
    if (T > 0) orc_linear(enc, T, m->D, m->jenc_w, Hj, m->jenc_b, ep);       /* joint.cpp:37-63 */
    float *ch = fbuf((size_t)L * H), *cc = fbuf((size_t)L * H);              /* committed state */
    float *oh = fbuf((size_t)L * H), *oc = fbuf((size_t)L * H);              /* step output */
    float *g = fbuf((size_t)H), *pp = fbuf((size_t)Hj), *f = fbuf((size_t)Hj), *lg = fbuf((size_t)Vp);
    memset(ch, 0, sizeof(float) * (size_t)L * H);
    memset(cc, 0, sizeof(float) * (size_t)L * H);
    int n = 0, t = 0, emitted_any = 0, g_valid = 0, overflow = 0;
    int32_t last = blank_id;
#define ORC_JOINT()                                                            \
    do {                                                                       \
        orc_linear(g, 1, H, m->jpred_w, Hj, m->jpred_b, pp);                   \
        for (int h = 0; h < Hj; ++h) {                                         \
            const float s = ep[(size_t)t * Hj + h] + pp[h];                    \
            f[h] = s > 0.f ? s : 0.f;                                          \
        }                                                                      \
        orc_linear(f, 1, Hj, m->jout_w, Vp, m->jout_b, lg);                    \
    } while (0)
#define ORC_EMIT(K, SPAN)                                                      \
    do {                                                                       \
        if (n >= cap) { overflow = 1; break; }                                 \
        ids[n] = (K); frames[n] = t; conf[n] = orc_max_prob_conf(lg, tc, (K)); \
        span[n] = (SPAN); ++n;                                                 \
        last = (K); emitted_any = 1; g_valid = 0;                              \
        memcpy(ch, oh, sizeof(float) * (size_t)L * H);                         \
        memcpy(cc, oc, sizeof(float) * (size_t)L * H);                         \
    } while (0)
    while (t < T && !overflow) {
        if (n_dur > 0) {                                        /* tdt.cpp:40-112 */
            int symbols = 0, need_loop = 1;
            while (need_loop && symbols < max_symbols && !overflow) {
                if (!g_valid) {
                    orc_lstm_step(m, last, !emitted_any, ch, cc, oh, oc, g);
                    g_valid = 1;
                }
                ORC_JOINT();
                const int k = orc_argmax_first(lg, tc), dk = orc_argmax_first(lg + tc, n_dur);
                const int skip = durations[dk];
                if (k != blank_id) ORC_EMIT(k, skip);
                symbols += 1;
                t += skip;
                need_loop = skip == 0;
            }
            if (symbols == max_symbols) t += 1;
        } else {                                                /* RNNT: advance-by-1 */
            int symbols = 0;
            for (;;) {
                if (!g_valid) {
                    orc_lstm_step(m, last, !emitted_any, ch, cc, oh, oc, g);
                    g_valid = 1;
                }
                ORC_JOINT();
                const int k = orc_argmax_first(lg, Vp);
                if (k == blank_id) { t += 1; break; }
                ORC_EMIT(k, 1);
                if (overflow) break;
                if (++symbols >= max_symbols) { t += 1; break; }
            }
        }
    }
#undef ORC_JOINT
#undef ORC_EMIT
    free(ep); free(ch); free(cc); free(oh); free(oc); free(g); free(pp); free(f); free(lg);
    return overflow ? -1 : n;
}

/* ------------------------------------------------------------------------ */
/* Log-mel front end: mel.cpp, fft.cpp, model.cpp:114-146                   */
/* The reference's CPU build has no FMA contraction (baseline x86-64), so    */
/* these functions are compiled without it as well.                          */
/* ------------------------------------------------------------------------ */

void orc_mel_window(const float* win, int win_len, int n_fft, float* out) {
    /* mel.cpp:31-46: zero-pad (n_fft - win_len)/2 on the left */
    for (int i = 0; i < n_fft; ++i) out[i] = 0.f;
    if (win_len == n_fft) {
        memcpy(out, win, sizeof(float) * (size_t)n_fft);
        return;
    }
    const int left = (n_fft - win_len) / 2;
    for (int i = 0; i < win_len && left + i < n_fft; ++i)
        if (left + i >= 0) out[left + i] = win[i];
}

int orc_mel_frames(const orc_mel_cfg* c, int S) {
    if (S <= 0) return 0;
    const int padded = S + 2 * (c->n_fft / 2);
    return padded >= c->n_fft ? 1 + (padded - c->n_fft) / c->hop : 0;
}

/* fft.cpp:9-51: bit reversal, then butterfly stages with the twiddle advanced
 * by complex multiplication (w <- w * e^{-2 pi i / len}) inside each group. */
__attribute__((optimize("fp-contract=off")))
static void orc_fft_inplace(double* re, double* im, int n) {
    for (int i = 1, j = 0; i < n; ++i) {
        int bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j ^= bit;
        if (i < j) {
            double t = re[i]; re[i] = re[j]; re[j] = t;
            t = im[i]; im[i] = im[j]; im[j] = t;
        }
    }
    for (int len = 2; len <= n; len <<= 1) {
        const double ang = -2.0 * M_PI / len, wr = cos(ang), wi = sin(ang);
        for (int i = 0; i < n; i += len) {
            double cr = 1.0, ci = 0.0;
            for (int k = 0; k < len / 2; ++k) {
                const int u = i + k, v = i + k + len / 2;
                const double tr = cr * re[v] - ci * im[v];
                const double ti = cr * im[v] + ci * re[v];
                re[v] = re[u] - tr;
                im[v] = im[u] - ti;
                re[u] = re[u] + tr;
                im[u] = im[u] + ti;
                const double nr = cr * wr - ci * wi, ni = cr * wi + ci * wr;
                cr = nr;
                ci = ni;
            }
        }
    }
}

void orc_rfft(const float* in, int n, float* re, float* im) {
    /* fft.cpp:53-74 */
    double* br = (double*)malloc(sizeof(double) * (size_t)n);
    double* bi = (double*)malloc(sizeof(double) * (size_t)n);
    for (int i = 0; i < n; ++i) { br[i] = (double)in[i]; bi[i] = 0.0; }
    orc_fft_inplace(br, bi, n);
    for (int k = 0; k <= n / 2; ++k) { re[k] = (float)br[k]; im[k] = (float)bi[k]; }
    free(br);
    free(bi);
}

__attribute__((optimize("fp-contract=off")))
int orc_mel(const orc_mel_cfg* c, const float* window, const float* fb,
            const float* samples, int S, float* feats) {
    const int n_fft = c->n_fft, hop = c->hop, n_mels = c->n_mels, n_bins = n_fft / 2 + 1;
    const int T = orc_mel_frames(c, S);
    if (T == 0) return 0;
    /* preemphasis in f64 (mel.cpp:110-117), then the zero-padded signal
     * (pad_mode "constant", mel.cpp:137-142) */
    const int pad = n_fft / 2, plen = S + 2 * pad;
    double* padded = (double*)calloc((size_t)plen, sizeof(double));
    for (int t = 0; t < S; ++t) {
        double x = samples[t];
        if (c->preemph > 0.0f && t > 0) x = (double)samples[t] - (double)c->preemph * (double)samples[t - 1];
        padded[pad + t] = x;
    }
    float* frame = (float*)malloc(sizeof(float) * (size_t)n_fft);
    float* re = (float*)malloc(sizeof(float) * (size_t)n_bins);
    float* im = (float*)malloc(sizeof(float) * (size_t)n_bins);
    double* power = (double*)malloc(sizeof(double) * (size_t)n_bins);
    for (int t = 0; t < T; ++t) {
        /* MelKernel::frame_logmel (mel.cpp:63-95) */
        const double* fin = padded + (size_t)t * hop;
        for (int i = 0; i < n_fft; ++i) frame[i] = (float)(fin[i] * (double)window[i]);
        orc_rfft(frame, n_fft, re, im);
        for (int b = 0; b < n_bins; ++b) {
            const double mag = sqrt((double)re[b] * re[b] + (double)im[b] * im[b]);
            power[b] = c->mag_power == 1.0f ? mag : pow(mag, (double)c->mag_power);
        }
        for (int m = 0; m < n_mels; ++m) {
            const float* fbm = fb + (size_t)m * n_bins;
            double acc = 0.0;
            for (int b = 0; b < n_bins; ++b) acc += (double)fbm[b] * power[b];
            feats[(size_t)m * T + t] = (float)log(acc + (double)c->log_guard);
        }
    }
    /* per-feature normalisation (mel.cpp:153-183): mean and unbiased std over
     * the first S/hop frames, std += 1e-5, later frames zeroed */
    if (c->per_feature) {
        const int valid = S / hop < T ? S / hop : T;
        for (int m = 0; m < n_mels; ++m) {
            float* row = feats + (size_t)m * T;
            double mean = 0.0, var = 0.0;
            if (valid > 0) {
                for (int t = 0; t < valid; ++t) mean += row[t];
                mean /= (double)valid;
            }
            if (valid > 1) {
                for (int t = 0; t < valid; ++t) {
                    const double d = (double)row[t] - mean;
                    var += d * d;
                }
                var /= (double)(valid - 1);
            }
            const double sd = sqrt(var) + 1e-5;
            for (int t = 0; t < T; ++t) row[t] = t < valid ? (float)(((double)row[t] - mean) / sd) : 0.0f;
        }
    }
    free(padded);
    free(frame);
    free(re);
    free(im);
    free(power);
    return T;
}

void orc_mel_batch(const orc_mel_cfg* c, const float* window, const float* fb,
                   const float* pcm, int B, int S_stride, const int* n_samples,
                   int T_max, float* out, int* T_out) {
    memset(out, 0, sizeof(float) * (size_t)B * c->n_mels * T_max);
#pragma omp parallel for schedule(dynamic)
    for (int b = 0; b < B; ++b) {
        const int T = orc_mel_frames(c, n_samples[b]);
        T_out[b] = T;
        if (T == 0 || T > T_max) continue;
        float* f = (float*)malloc(sizeof(float) * (size_t)c->n_mels * T);
        orc_mel(c, window, fb, pcm + (size_t)b * S_stride, n_samples[b], f);
        for (int m = 0; m < c->n_mels; ++m)
            memcpy(out + ((size_t)b * c->n_mels + m) * T_max, f + (size_t)m * T, sizeof(float) * (size_t)T);
        free(f);
    }
}

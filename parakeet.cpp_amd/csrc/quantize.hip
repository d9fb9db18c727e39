// Weight quantisation on the device: ggml_quantize_chunk for q8_0 and q4_K
// (the quantisers parakeet-cli quantize runs, examples/cli/main.cpp:322-426;
// ggml v0.13.0 quantize_row_q8_0_ref / quantize_row_q4_K_ref).  Every value
// is computed with the same f32 operations in the same order as the scalar
// reference quantisers (no FMA contraction in this file; division and sqrt
// are correctly rounded), so the blocks are the reference quantisers' bytes.
//
// q8_0: one thread per 32-value block.  q4_K: one thread per 256-value
// super-block (the sub-block fits and the 6-bit code packing are sequential
// per super-block); an offline step, a 4096 x 1024 matrix is 16 k threads.
#pragma clang fp contract(off)

#include "common.hpp"
#include "gemm.hpp"

namespace pkx {
namespace {

__device__ __forceinline__ int nearest_int_dev(float fval) {
    const float val = fval + 12582912.f;   // 1.5 * 2^23: round to nearest, ties to even
    return (__builtin_bit_cast(int, val) & 0x007fffff) - 0x00400000;
}

__device__ __forceinline__ void put_u16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}

__device__ __forceinline__ uint16_t f16_bits(float v) { return __builtin_bit_cast(uint16_t, (f16)v); }
__device__ __forceinline__ float f16_val(uint16_t b) { return (float)__builtin_bit_cast(f16, b); }

__global__ void quantize_q8_0_kernel(const float* __restrict__ x, uint8_t* __restrict__ y, int64_t rows,
                                     int64_t per_row) {
    const int64_t nb = per_row / 32, blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= rows * nb) return;
    const float* v = x + blk * 32;
    uint8_t* o = y + blk * 34;
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / ((1 << 7) - 1);
    const float id = d != 0.f ? 1.0f / d : 0.0f;
    put_u16(o, f16_bits(d));
    for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)(int8_t)roundf(v[j] * id);
}

// make_qkx2_quants(32, 15, x, w, L, &min, Laux, -1, 0.1, 20, false)
__device__ float fit_q4_subblock(const float* x, const float* weights, uint8_t* L, float* the_min, uint8_t* Laux) {
    constexpr int n = 32, nmax = 15, nstep = 20;
    constexpr float rmin = -1.f, rdelta = 0.1f;
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
        const int l = nearest_int_dev(iscale * (x[i] - min));
        L[i] = (uint8_t)(l < 0 ? 0 : l > nmax ? nmax : l);
        float diff = scale * L[i] + min - x[i];
        diff = diff * diff;
        best_mad += weights[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int_dev(iscale * (x[i] - min));
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

__global__ __launch_bounds__(64) void quantize_q4_k_kernel(const float* __restrict__ xs, uint8_t* __restrict__ ys,
                                                           int64_t n_blocks) {
    const int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= n_blocks) return;
    const float* x = xs + blk * 256;
    uint8_t* y = ys + blk * 144;
    uint8_t L[256], Laux[32], sc[12];
    float weights[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = fit_q4_subblock(x + 32 * j, weights, L + 32 * j, &mins[j], Laux);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    for (int i = 0; i < 12; ++i) sc[i] = 0;
    for (int j = 0; j < 8; ++j) {
        uint8_t ls = (uint8_t)nearest_int_dev(inv_scale * scales[j]);
        uint8_t lm = (uint8_t)nearest_int_dev(inv_min * mins[j]);
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
    const uint16_t dh = f16_bits(max_scale / 63.f), mh = f16_bits(max_min / 63.f);
    for (int j = 0; j < 8; ++j) {
        uint8_t s, m;
        if (j < 4) {
            s = sc[j] & 63;
            m = sc[j + 4] & 63;
        } else {
            s = (uint8_t)((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4));
            m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j - 0] >> 6) << 4));
        }
        const float d = f16_val(dh) * s;
        if (!d) continue;
        const float dm = f16_val(mh) * m;
        for (int ii = 0; ii < 32; ++ii) {
            const int l = nearest_int_dev((x[32 * j + ii] + dm) / d);
            L[32 * j + ii] = (uint8_t)(l < 0 ? 0 : l > 15 ? 15 : l);
        }
    }
    put_u16(y, dh);
    put_u16(y + 2, mh);
    for (int i = 0; i < 12; ++i) y[4 + i] = sc[i];
    uint8_t* q = y + 16;
    for (int j = 0; j < 256; j += 64) {
        for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
        q += 32;
    }
}

}  // namespace

void quantize_rows(int gtype, const float* x, void* y, int64_t rows, int64_t per_row, hipStream_t s) {
    require(rows >= 0 && per_row > 0, "quantize: bad shape");
    if (rows == 0) return;
    if (gtype == GT_Q8_0) {
        require(per_row % 32 == 0, "quantize: q8_0 needs a row length divisible by 32");
        const int64_t n = rows * (per_row / 32);
        launch(quantize_q8_0_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, x, (uint8_t*)y, rows, per_row);
    } else if (gtype == GT_Q4_K) {
        require(per_row % 256 == 0, "quantize: q4_K needs a row length divisible by 256");
        const int64_t n = rows * (per_row / 256);
        launch(quantize_q4_k_kernel, dim3(cdiv(n, 64)), dim3(64), 0, s, x, (uint8_t*)y, n);
    } else {
        throw std::invalid_argument("quantize: type must be q8_0 (8) or q4_K (12)");
    }
    PKX_LAUNCH_CHECK();
}

}  // namespace pkx

// Subsampling tail on the matrix cores: conv.3 -> conv.5 -> conv.6 -> flatten
// in one persistent kernel (subsampling.cpp:168-231).
//
// The three steps run one after the other as separate launches move the
// conv.3 map (B x T2 x 32 x 256 f16) through HBM twice more than needed and
// re-read both 128 KB weights for every tile.  Here each block owns a run of
// output frames (b, t3) and keeps both pointwise weights in registers for the
// whole run: eight waves, wave w holding output channels 32 w .. 32 w + 31 of
// conv.3 (as B fragments of v_mfma_f32_32x32x16_f16, 64 VGPRs) and of conv.6
// (B fragments of v_mfma_f32_16x16x32_f16, 64 VGPRs), loaded from a copy in
// fragment order (sub_tail_prepare: each load instruction reads 1 KB
// contiguous, instead of 16 bytes from each of 32 weight rows; measured at
// 256 blocks: 31.6 us per launch against 35.8 us from the row-major weights,
// the start-up before the first frame 8.5k cycles against 20k).  Per frame the block
//   1. DMAs the two new input rows t2 = 2 t3, 2 t3 + 1 (2 x 16 KB) into LDS
//      (the frame after next is in flight while this one computes),
//   2. runs conv.3 on them (64 pixels x 256 x 256) and keeps bias + ReLU of
//      the result, rounded to f16, in registers; with the row 2 t3 - 1 kept
//      from the previous frame these are the three rows the depthwise conv
//      reads, so conv.3 runs once per input row,
//   3. runs conv.5 on its own channels from those registers (each lane holds
//      16 consecutive columns of one channel; the one column a lane's window
//      reaches past its range comes from its partner lane) and writes the
//      16 x 256 result to LDS as f16,
//   4. runs conv.6 on that (16 pixels x 256 x 256), adds bias, ReLU and the
//      frame mask and stores the channel-major row (8-byte stores, 512
//      contiguous bytes per wave and column block).
// HBM traffic is the input map once plus the flattened output; the product
// work is 2 x (2 T2 + T3) x 32 x 256 x 256 flops on the matrix cores.
#include "subsampling.hpp"

#include "elementwise.hpp"

#include <algorithm>
#include <type_traits>

namespace pkx {

namespace {
constexpr int TC = 256;                   // channels
constexpr int TF2 = 32;                   // conv.3 map columns
constexpr int TF3 = 16;                   // conv.5 output columns
constexpr int ROW_BYTES = TF2 * TC * 2;   // one input row t2: 16 KB
constexpr int A_BYTES = 2 * ROW_BYTES;    // one frame's input: two rows
constexpr int DW_BYTES = TF3 * TC * 2;    // conv.5 output of one frame: 8 KB
constexpr int TAIL_THREADS = 512;
}  // namespace

// Fragment order of the pointwise weights (TAIL_FRAG halves): conv.3 unit
// (w, s, lane) = W3[32 w + lane % 32][16 s + 8 (lane / 32) .. + 7] at
// ((w * 16 + s) * 64 + lane) * 8; conv.6 unit (w, j, s, lane) =
// W6[32 w + 16 j + lane % 16][32 s + 8 (lane / 16) .. + 7] at
// 65536 + ((w * 16 + 8 j + s) * 64 + lane) * 8.
constexpr int TAIL_FRAG = 2 * TC * TC;

struct SubTailParams {
    const f16* in;
    const f16* wf;   // fragment-ordered conv.3 and conv.6 weights
    const float* b3;
    const float* w5;
    const float* b5;
    const float* b6;
    const int* valid2;
    const int* valid3;
    f16* out;
    int B, T2, T3;
};

// ReLU and a wave-uniform row mask in one v_med3_f32: median(x, 0, +inf) is
// max(x, 0), median(x, 0, 0) is 0 (fmaxf costs two v_max_f32, the mask a
// v_cndmask more).
__device__ __forceinline__ float relu_mask_hi(bool keep) { return keep ? __builtin_huge_valf() : 0.f; }
__device__ __forceinline__ float relu_masked(float x, float hi) { return __builtin_amdgcn_fmed3f(x, 0.f, hi); }

__global__ __launch_bounds__(TAIL_THREADS, 1) void sub_tail_kernel(SubTailParams p) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * A_BYTES + DW_BYTES];
    uint8_t* const dwb = smem + 2 * A_BYTES;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int q = lane >> 5, r32 = lane & 31, l16 = lane & 15, g16 = lane >> 4;

    // frames [r0, r1) of the flattened (b, t3) range; a run that starts
    // inside an item first computes conv.3 row 2 t3 - 1 on its own ("prime")
    const int R = p.B * p.T3;
    const int r0 = (int)((int64_t)blockIdx.x * R / gridDim.x);
    const int r1 = (int)((int64_t)(blockIdx.x + 1) * R / gridDim.x);
    if (r0 >= r1) return;
    const int has_prime = (r0 % p.T3) != 0 ? 1 : 0;
    const int NJ = r1 - r0 + has_prime;

    // DMA: 16-byte unit u = (4 w + k) * 64 + lane of a job's buffer is tile
    // i = u / 1024 (waves 0-3: tile 0, waves 4-7: tile 1), MFMA row
    // m = (u / 32) % 32, physical chunk u % 32 = r32, which holds channel
    // chunk r32 ^ m (the XOR keeps the 32 rows of one MFMA read on distinct
    // banks); tile i is input row t2s + i.
    const int dtile = w >> 2;
    uint32_t dsub[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int m = ((4 * w + k) * 2 + q) & 31;
        dsub[k] = (uint32_t)(tail_col(m) * (TC * 2) + ((r32 ^ m) << 4));
    }
    // job jn: the prime of frame r0 (jn = 0 when has_prime), then frames r0, r0 + 1, ...
    auto job_frame = [&](int jn) { return r0 + (jn > 0 ? jn - has_prime : 0); };
    auto issue = [&](int jn) {
        const bool prime = has_prime && jn == 0;
        const int r = job_frame(jn);
        const int b = r / p.T3, t3 = r - b * p.T3;
        const int t2 = (prime ? 2 * t3 - 1 : 2 * t3) + dtile;   // >= 0: a prime has t3 >= 1
        const bool live = t2 >= 0 && t2 < p.T2 && !(prime && dtile == 1);
        const __amdgpu_buffer_rsrc_t rs =
            make_rsrc(p.in + (int64_t)b * p.T2 * TF2 * TC, (int64_t)p.T2 * ROW_BYTES);
        uint8_t* dst = smem + (jn & 1) * A_BYTES + 4 * w * 1024;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            lds_dma16(rs, dst + k * 1024, live ? (uint32_t)t2 * ROW_BYTES + dsub[k] : OOB, 0);
    };
    issue(0);

    // weights of this wave's channels, held for the whole run
    const int n3 = 32 * w + r32;
    half8v bw3[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) bw3[s] = *(const half8v*)(p.wf + ((w * 16 + s) * 64 + lane) * 8);
    half8v bw6[2][8];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int s = 0; s < 8; ++s) bw6[j][s] = *(const half8v*)(p.wf + TC * TC + ((w * 16 + 8 * j + s) * 64 + lane) * 8);
    const float b3 = p.b3[n3], b5 = p.b5[n3];
    float w5[9];
#pragma unroll
    for (int e = 0; e < 9; ++e) w5[e] = p.w5[n3 * 9 + e];
    const float b6[2] = {p.b6[32 * w + l16], p.b6[32 * w + 16 + l16]};

    half2v carry[8];          // conv.3 row 2 t3 - 1, columns 16 q .. 16 q + 15
    half4v pend[2];           // the previous frame's output, stored one frame later
    f16* pdst = nullptr;
#pragma unroll
    for (int k = 0; k < 8; ++k) carry[k] = (half2v){};

    auto relu_row = [&](const float16v& a, bool ok, half2v (&o)[8]) {
        const float hi = relu_mask_hi(ok);
#pragma unroll
        for (int k = 0; k < 8; ++k)
            o[k] = (half2v){(f16)relu_masked(a[2 * k] + b3, hi), (f16)relu_masked(a[2 * k + 1] + b3, hi)};
    };

    for (int jn = 0; jn < NJ; ++jn) {
        const bool prime = has_prime && jn == 0;
        const int r = job_frame(jn);
        const int b = r / p.T3, t3 = r - b * p.T3;
        const int v2 = p.valid2 ? p.valid2[b] : p.T2;
        // this job's rows have landed (every wave's share), the previous
        // frame's stores and the DMA issued a frame ago are complete
        wait_vmcnt<0>();
        __syncthreads();
        if (pdst) {
            *(half4v*)pdst = pend[0];
            *(half4v*)(pdst + 16 * 16) = pend[1];
            pdst = nullptr;
        }
        if (jn + 1 < NJ) issue(jn + 1);

        // conv.3: 32 (prime) or 64 pixels x this wave's 32 channels.  Step s
        // reads channel chunk 2 s + q of row 32 i + r32, stored at chunk
        // (2 s + q) ^ r32 = ((q ^ r32) ^ 2 s): the XOR with 32 s is formed per
        // read (xo is opaque per job, so the compiler does not keep 16 offset
        // registers live), and the reads run two steps ahead of the MFMAs.
        const uint8_t* A = smem + (jn & 1) * A_BYTES + r32 * 512;
        uint32_t xo = (uint32_t)((q ^ r32) << 4);
        asm volatile("" : "+v"(xo));
        auto lda = [&](int s, int i) { return *(const half8v*)(A + i * (32 * 512) + (xo ^ (uint32_t)(s << 5))); };
        float16v acc[2] = {(float16v){}, (float16v){}};
        auto conv3 = [&](auto nt) {
            constexpr int NT = decltype(nt)::value;
            half8v af[3][NT];
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int i = 0; i < NT; ++i) af[s][i] = lda(s, i);
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                if (s + 2 < 16) {
#pragma unroll
                    for (int i = 0; i < NT; ++i) af[(s + 2) % 3][i] = lda(s + 2, i);
                }
#pragma unroll
                for (int i = 0; i < NT; ++i)
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s % 3][i], bw3[s], acc[i], 0, 0, 0);
            }
            // issue order: the first two steps' reads, then per step the reads
            // two ahead and the step's MFMAs
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * NT, 0);
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                if (s + 2 < 16) __builtin_amdgcn_sched_group_barrier(0x100, NT, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, NT, 0);
            }
        };
        if (prime) {
            conv3(std::integral_constant<int, 1>{});
            relu_row(acc[0], 2 * t3 - 1 < v2, carry);
            continue;
        }
        conv3(std::integral_constant<int, 2>{});
        half2v rows[3][8];
        if (t3 == 0) {   // row -1: the zero padding
#pragma unroll
            for (int k = 0; k < 8; ++k) rows[0][k] = (half2v){};
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) rows[0][k] = carry[k];
        }
        relu_row(acc[0], 2 * t3 < v2, rows[1]);
        relu_row(acc[1], 2 * t3 + 1 < p.T2 && 2 * t3 + 1 < v2, rows[2]);
#pragma unroll
        for (int k = 0; k < 8; ++k) carry[k] = rows[2][k];

        // conv.5: outputs f3 = 8 q + o read local columns 2 o - 1 .. 2 o + 1;
        // local column -1 is column 15 of the partner lane (half 1) or the
        // zero padding (half 0)
        f16 xm[3];
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) {
            const int v = __builtin_bit_cast(int, rows[kh][7]);
            const int got = __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, v);
            xm[kh] = q ? __builtin_bit_cast(half2v, got)[1] : (f16)0.f;
        }
#pragma unroll
        for (int o = 0; o < 8; ++o) {
            float a = b5;
#pragma unroll
            for (int kh = 0; kh < 3; ++kh)
#pragma unroll
                for (int kw = 0; kw < 3; ++kw) {
                    const int c = 2 * o - 1 + kw;
                    const f16 x = c < 0 ? xm[kh] : rows[kh][c >> 1][c & 1];
                    a += w5[kh * 3 + kw] * (float)x;
                }
            const int f3 = 8 * q + o;
            *(f16*)(dwb + f3 * 512 + (((n3 >> 3) ^ f3) << 4) + ((n3 & 7) << 1)) = (f16)a;
        }
        __syncthreads();

        // conv.6: 16 pixels x this wave's 32 channels (two 16-column blocks)
        float4v acc6[2] = {(float4v){}, (float4v){}};
        {
            half8v a6[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) a6[s] = *(const half8v*)(dwb + l16 * 512 + (((4 * s + g16) ^ l16) << 4));
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc6[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a6[s], bw6[j][s], acc6[j], 0, 0, 0);
            // all eight reads first (the tile is 8 KB), then the MFMAs as they land
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
        }
        const float hi6 = relu_mask_hi(!(p.valid3 && t3 >= p.valid3[b]));
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) pend[j][e] = (f16)relu_masked(acc6[j][e] + b6[j], hi6);
        // channel 32 w + 16 j + l16, columns 4 g16 .. 4 g16 + 3
        pdst = p.out + (int64_t)r * (TC * TF3) + (32 * w + l16) * TF3 + 4 * g16;
    }
    if (pdst) {
        *(half4v*)pdst = pend[0];
        *(half4v*)(pdst + 16 * 16) = pend[1];
    }
}

// ---------------------------------------------------------------------------
// Stage 1 on the matrix cores: conv.0 (1 -> 256, 3x3, stride 2, pad 1) + bias
// + ReLU, the stage masks, and the depthwise conv.2 (3x3, stride 2) + bias
// (subsampling.cpp:143-184), for 128 mel bins (conv.0 map 64 columns wide,
// output 32).  conv.0 is a product over im2col rows: 9 f16 mel taps per
// pixel (padded to K = 16) against the f16 filter taps of each channel, the
// accumulator seeded with the bias (f32).  A block owns a run of output rows
// t2 of one item; per row it forms the two new conv.0 rows 2 t2, 2 t2 + 1
// (128 pixels: four 32-row MFMA tiles per wave, wave w taking channels
// 32 w .. 32 w + 31) and keeps row 2 t2 - 1 from the previous row.  With the
// column mapping of tail_col each lane then holds 16 consecutive columns of
// each conv.0 row of its channel, and runs the depthwise conv on them in f32
// (the one column left of its range comes from its partner lane).  Outputs
// go through LDS so each output row (32 x 256 f16, contiguous in memory) is
// written with 16-byte stores.  The mel values of the next row are fetched
// while the current one computes.
// ---------------------------------------------------------------------------
namespace {
constexpr int S1_F = 128, S1_F2 = 32;   // mel bins, conv.2 map columns
constexpr int S1_THREADS = 512;
}  // namespace

struct SubStage1Params {
    const float* mel;     // [B][128][T]
    const int* valid0;    // mel frames t >= valid0[b] read as zero (nullable)
    const int* valid1;    // conv.0 rows t1 >= valid1[b] zero (nullable)
    const float* w0;      // [256][9]
    const float* b0;
    const float* w2;      // [256][9]
    const float* b2;
    f16* out;             // [B][T2][32][256]
    int B, T, T1, T2, nch;
};

__global__ __launch_bounds__(S1_THREADS, 1) void sub_stage1_mfma_kernel(SubStage1Params p) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * 128 * 32 + 2 * S1_F2 * TC * 2];
    f16* const col = (f16*)smem;                   // [2][128 rows][16 taps]
    uint8_t* const stg = smem + 2 * 128 * 32;      // [2][32 f2][256 channels] f16
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 5, r32 = lane & 31;
    const int b = blockIdx.x / p.nch, ch = blockIdx.x - b * p.nch;
    const int t2a = (int)((int64_t)ch * p.T2 / p.nch), t2b = (int)((int64_t)(ch + 1) * p.T2 / p.nch);
    if (t2a >= t2b) return;
    const int v0 = p.valid0 ? p.valid0[b] : p.T;
    const int v1 = p.valid1 ? p.valid1[b] : p.T1;
    // job 0 of a run that starts past the item's first row forms conv.0 row
    // 2 t2a - 1 alone ("prime"); job jn >= prime makes output row t2a + jn - prime
    const int prime = t2a > 0 ? 1 : 0;
    const int NJ = t2b - t2a + prime;

    // im2col rows (MFMA row order): row P = tid / 4 of the 128 is tile
    // i = P / 32, MFMA row P % 32, i.e. conv.0 row 2 t2 + i / 2 and column
    // 32 (i % 2) + tail_col(P % 32); thread kh = tid % 4 < 3 fills taps
    // 3 kh .. 3 kh + 2 (taps 9 .. 15 stay zero)
    const int P = tid >> 2, kh = tid & 3, ti = P >> 5;
    const int f1 = 32 * (ti & 1) + tail_col(P & 31);
    const float* melb = p.mel + (int64_t)b * S1_F * p.T;
    auto fetch = [&](int jn, float (&v)[3]) {
        const bool pr = prime && jn == 0;
        const int t1 = pr ? 2 * t2a - 1 : 2 * (t2a + jn - prime) + (ti >> 1);
        const int t = 2 * t1 - 1 + kh;
        const bool rok = kh < 3 && t >= 0 && t < p.T && t < v0 && !(pr && ti >= 2);
#pragma unroll
        for (int kw = 0; kw < 3; ++kw) {
            const int f = 2 * f1 - 1 + kw;
            v[kw] = rok && f >= 0 && f < S1_F ? melb[(int64_t)f * p.T + t] : 0.f;
        }
    };
    for (int e = tid; e < 2 * 128; e += S1_THREADS) *(half8v*)(col + e * 16 + 8) = (half8v){};

    // per-lane constants: conv.0 taps of channel n (B fragment: taps 8 q .. 8 q + 7,
    // tap 8 alone in half 1), biases, depthwise taps
    const int n = 32 * w + r32;
    half8v bw0 = (half8v){};
    if (q == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) bw0[e] = (f16)p.w0[n * 9 + e];
    } else {
        bw0[0] = (f16)p.w0[n * 9 + 8];
    }
    const float b0 = p.b0[n], b2 = p.b2[n];
    float w2[9];
#pragma unroll
    for (int e = 0; e < 9; ++e) w2[e] = p.w2[n * 9 + e];

    float carry[2][16];   // conv.0 row 2 t2 - 1 (columns 16 q + 32 i + r, after ReLU and mask)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) carry[i][r] = 0.f;
    float v[3];
    fetch(0, v);
    __syncthreads();

    int out_prev = -1;   // output row held in the other staging buffer
    for (int jn = 0; jn < NJ; ++jn) {
        const bool pr = prime && jn == 0;
        const int t2 = t2a + jn - prime;
        f16* cb = col + (jn & 1) * 128 * 16;
        if (kh < 3) {
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) cb[P * 16 + 3 * kh + kw] = (f16)v[kw];
        }
        if (jn + 1 < NJ) fetch(jn + 1, v);
        __syncthreads();
        // the previous output row leaves LDS (16 KB contiguous in memory)
        if (out_prev >= 0) {
            const uint8_t* src = stg + ((jn - 1) & 1) * (S1_F2 * TC * 2) + tid * 32;
            uint8_t* dst = (uint8_t*)(p.out + ((int64_t)b * p.T2 + out_prev) * S1_F2 * TC) + tid * 32;
            *(int4v*)dst = *(const int4v*)src;
            *(int4v*)(dst + 16) = *(const int4v*)(src + 16);
        }
        // conv.0: tiles 0, 1 = row 2 t2 (prime: 2 t2a - 1), tiles 2, 3 = row 2 t2 + 1
        float16v acc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][r] = b0;
        }
        if (pr) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const half8v a = *(const half8v*)(cb + (32 * i + r32) * 16 + 8 * q);
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bw0, acc[i], 0, 0, 0);
            }
            const float hi = relu_mask_hi(2 * t2a - 1 < v1);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) carry[i][r] = relu_masked(acc[i][r], hi);
            out_prev = -1;
            continue;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const half8v a = *(const half8v*)(cb + (32 * i + r32) * 16 + 8 * q);
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bw0, acc[i], 0, 0, 0);
        }
        const float hi1 = relu_mask_hi(2 * t2 < v1 && 2 * t2 < p.T1);
        const float hi2 = relu_mask_hi(2 * t2 + 1 < v1 && 2 * t2 + 1 < p.T1);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[i][r] = relu_masked(acc[i][r], hi1);
                acc[2 + i][r] = relu_masked(acc[2 + i][r], hi2);
            }
        // conv.2: rows kh = 0 (carry), 1 (acc 0, 1), 2 (acc 2, 3); output
        // column 16 i + 8 q + o reads local columns 2 o - 1 .. 2 o + 1; local
        // column -1 is column 32 i + 16 q - 1: the partner's column 15 of
        // tile i (q = 1), of tile 0 (q = 0, i = 1), or the zero padding
        float xm[3][2];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const float c0 = k == 0 ? carry[0][15] : acc[2 * k - 2][15];
            const float c1 = k == 0 ? carry[1][15] : acc[2 * k - 1][15];
            const float g0 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, c0)));
            const float g1 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, c1)));
            xm[k][0] = q ? g0 : 0.f;
            xm[k][1] = q ? g1 : g0;
        }
        uint8_t* so = stg + (jn & 1) * (S1_F2 * TC * 2);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int o = 0; o < 8; ++o) {
                float a = b2;
#pragma unroll
                for (int k = 0; k < 3; ++k)
#pragma unroll
                    for (int kw = 0; kw < 3; ++kw) {
                        const int c = 2 * o - 1 + kw;
                        const float x = c < 0 ? xm[k][i] : k == 0 ? carry[i][c] : acc[2 * k - 2 + i][c];
                        a += w2[k * 3 + kw] * x;
                    }
                const int f2 = 16 * i + 8 * q + o;
                *(f16*)(so + f2 * (TC * 2) + n * 2) = (f16)a;
            }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) carry[i][r] = acc[2 + i][r];
        out_prev = t2;
    }
    if (out_prev >= 0) {
        __syncthreads();
        const uint8_t* src = stg + ((NJ - 1) & 1) * (S1_F2 * TC * 2) + tid * 32;
        uint8_t* dst = (uint8_t*)(p.out + ((int64_t)b * p.T2 + out_prev) * S1_F2 * TC) + tid * 32;
        *(int4v*)dst = *(const int4v*)src;
        *(int4v*)(dst + 16) = *(const int4v*)(src + 16);
    }
}

bool sub_stage1_mfma_supported(int C, int F, bool causal) { return C == TC && F == S1_F && !causal; }

void launch_sub_stage1_mfma(const float* mel, const int* valid0, const int* valid1, const float* w0, const float* b0,
                            const float* w2, const float* b2, void* out, int B, int T, hipStream_t s) {
    if (B == 0 || T == 0) return;
    const int T1 = sub_stage_len(T, false), T2 = sub_stage_len(T1, false);
    require((int64_t)B * S1_F * T <= ((int64_t)1 << 40), "subsampling stage 1: input too large");
    const int cus = device_cu_count();
    const int nch = std::max(1, std::min(T2, (cus + B - 1) / B));
    require((int64_t)B * nch <= 0x7fffffff, "subsampling stage 1: too many items");
    SubStage1Params p{mel, valid0, valid1, w0, b0, w2, b2, (f16*)out, B, T, T1, T2, nch};
    launch(sub_stage1_mfma_kernel, dim3(B * nch), dim3(S1_THREADS), 0, s, p);
    PKX_LAUNCH_CHECK();
}

// one thread per 16-byte unit of the fragment-ordered copy
__global__ __launch_bounds__(256) void sub_tail_prepare_kernel(const f16* w3, const f16* w6, f16* wf) {
    const int u = blockIdx.x * 256 + threadIdx.x;   // < TAIL_FRAG / 8
    const int lane = u & 63, ws = u >> 6;
    const f16* src;
    if (ws < 128) {   // conv.3: ws = w * 16 + s
        const int w = ws >> 4, s = ws & 15;
        src = w3 + (32 * w + (lane & 31)) * TC + 16 * s + 8 * (lane >> 5);
    } else {          // conv.6: ws - 128 = w * 16 + 8 j + s
        const int v = ws - 128, w = v >> 4, j = (v >> 3) & 1, s = v & 7;
        src = w6 + (32 * w + 16 * j + (lane & 15)) * TC + 32 * s + 8 * (lane >> 4);
    }
    *(half8v*)(wf + (size_t)u * 8) = *(const half8v*)src;
}

bool sub_tail_supported(int C, int F2, bool causal) { return C == TC && F2 == TF2 && !causal; }

size_t sub_tail_frag_bytes() { return (size_t)TAIL_FRAG * 2; }

void sub_tail_prepare(const void* w3, const void* w6, void* frag, hipStream_t s) {
    launch(sub_tail_prepare_kernel, dim3(TAIL_FRAG / 8 / 256), dim3(256), 0, s, (const f16*)w3, (const f16*)w6,
           (f16*)frag);
    PKX_LAUNCH_CHECK();
}

void launch_sub_tail(const void* in, const void* frag, const float* b3, const float* w5, const float* b5,
                     const float* b6, const int* valid2, const int* valid3, void* out, int B, int T2, int T3,
                     hipStream_t s) {
    if (B == 0 || T3 == 0) return;
    require(T2 >= 1 && T3 == sub_stage_len(T2, false), "subsampling tail: T3 must be (T2 - 1) / 2 + 1");
    require((int64_t)T2 * ROW_BYTES <= 0x7fffffff, "subsampling tail: input rows of one item exceed 2 GB");
    require((int64_t)B * T3 <= 0x7fffffff / 2, "subsampling tail: too many frames");
    SubTailParams p{(const f16*)in, (const f16*)frag, b3, w5, b5, b6, valid2, valid3, (f16*)out, B, T2, T3};
    const int grid = (int)std::min<int64_t>((int64_t)B * T3, device_cu_count());
    launch(sub_tail_kernel, dim3(grid), dim3(TAIL_THREADS), 0, s, p);
    PKX_LAUNCH_CHECK();
}

}  // namespace pkx

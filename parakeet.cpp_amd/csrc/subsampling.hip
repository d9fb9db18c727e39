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

// MFMA row m of a 32-row tile <-> map column.  The 32x32 accumulator gives
// lane half q the rows 8 g + 4 q + e (register 4 g + e, e < 4); feeding row m
// from column 16 q + 4 g + e leaves column 16 q + r in register r, so each
// lane holds 16 consecutive columns of its channel.
__device__ __forceinline__ int tail_col(int m) { return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3); }

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
#pragma unroll
        for (int k = 0; k < 8; ++k)
            o[k] = ok ? (half2v){(f16)fmaxf(a[2 * k] + b3, 0.f), (f16)fmaxf(a[2 * k + 1] + b3, 0.f)}
                      : (half2v){};
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

        // conv.3: 32 (prime) or 64 pixels x this wave's 32 channels
        const uint8_t* A = smem + (jn & 1) * A_BYTES;
        float16v acc[2] = {(float16v){}, (float16v){}};
        if (prime) {
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const half8v a = *(const half8v*)(A + r32 * 512 + (((2 * s + q) ^ r32) << 4));
                acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bw3[s], acc[0], 0, 0, 0);
            }
            relu_row(acc[0], 2 * t3 - 1 < v2, carry);
            continue;
        }
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const half8v a = *(const half8v*)(A + (32 * i + r32) * 512 + (((2 * s + q) ^ r32) << 4));
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bw3[s], acc[i], 0, 0, 0);
            }
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
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const half8v a = *(const half8v*)(dwb + l16 * 512 + (((4 * s + g16) ^ l16) << 4));
#pragma unroll
            for (int j = 0; j < 2; ++j) acc6[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bw6[j][s], acc6[j], 0, 0, 0);
        }
        const bool dead = p.valid3 && t3 >= p.valid3[b];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = acc6[j][e] + b6[j];
                pend[j][e] = dead ? (f16)0.f : (f16)(v > 0.f ? v : 0.f);
            }
        // channel 32 w + 16 j + l16, columns 4 g16 .. 4 g16 + 3
        pdst = p.out + (int64_t)r * (TC * TF3) + (32 * w + l16) * TF3 + 4 * g16;
    }
    if (pdst) {
        *(half4v*)pdst = pend[0];
        *(half4v*)(pdst + 16 * 16) = pend[1];
    }
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

// Subsampling kernels on the matrix cores (gfx950).
#pragma once
#include "common.hpp"

namespace pkx {

// Subsampling stage 1 on the matrix cores (f16 mode): conv.0 (1 -> 256,
// 3x3, stride 2, pad 1) + bias + ReLU over mel [B][128][T] f32 (frames
// t >= valid0[b] zero when valid0 is set), the stage mask on its rows
// (t1 >= valid1[b] zero when valid1 is set) and the depthwise conv.2 + bias;
// output channels-last [B][T2][32][256] f16 (subsampling.cpp:143-184).  The
// mel values and conv.0 taps are rounded to f16 (f32 accumulation), the
// conv.0 map is kept in f32, as in launch_sub_stage1's f16 mode.
bool sub_stage1_mfma_supported(int C, int F, bool causal);
void launch_sub_stage1_mfma(const float* mel, const int* valid0, const int* valid1, const float* w0, const float* b0,
                            const float* w2, const float* b2, void* out, int B, int T, hipStream_t s);

// Subsampling tail, fused: conv.3 (pointwise C -> C, 1x1) + bias + ReLU,
// the stage mask on its rows (t2 >= valid2[b] zero when valid2 is set),
// conv.5 (depthwise 3x3, stride 2, zero padding 1) + bias, conv.6
// (pointwise) + bias + ReLU, the flatten to channel-major rows and the
// output-frame mask (t3 >= valid3[b] zero when valid3 is set).
// subsampling.cpp:168-192 (second depthwise/pointwise stage pair and the
// first stage's pointwise), :195-204 (flatten), :206-231 (frame mask).
//   in   [B][T2][32][256] f16 (output of launch_sub_stage1, channels last)
//   w3, w6 [256][256] f16 (out, in), via the fragment-ordered copy;
//   b3, b5, b6 [256] f32; w5 [256][9] f32
//   out  [B][T3][256 * 16] f16, element c * 16 + f
// Shape: 256 channels, 32 map columns (128 mel bins), symmetric padding
// (non-causal); T3 = (T2 - 1) / 2 + 1.  The f16 values the unfused chain
// stores between its steps (conv.3 and conv.5 outputs) are rounded the same
// way here.
// The pointwise weights go in as one copy in MFMA fragment order, made once
// by sub_tail_prepare from the row-major [256][256] f16 weights into a
// buffer of sub_tail_frag_bytes().
bool sub_tail_supported(int C, int F2, bool causal);
size_t sub_tail_frag_bytes();
void sub_tail_prepare(const void* w3, const void* w6, void* frag, hipStream_t s);
void launch_sub_tail(const void* in, const void* frag, const float* b3, const float* w5, const float* b5,
                     const float* b6, const int* valid2, const int* valid3, void* out, int B, int T2, int T3,
                     hipStream_t s);

}  // namespace pkx

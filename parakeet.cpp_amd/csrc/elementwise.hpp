// Memory-bound kernels of the encoder path.
#pragma once
#include "common.hpp"

namespace pkx {

// LayerNorm over the last dim (conformer.cpp:300-307, eps 1e-5).
//   y = LN(x; g, b) written as the activation type of `prec`, or, with
//   y_f32 != nullptr, first y_f32 = LN(x; g, b) (may alias x) and then
//   y = LN(y_f32; g2, b2): the layer's norm_out fused with the next layer's
//   norm_feed_forward1 (one pass over the residual stream).
// With y == nullptr only y_f32 = LN(x) is written (f32 output in any mode).
struct LnParams {
    const float* x = nullptr;
    const float* g = nullptr;
    const float* b = nullptr;
    float* y_f32 = nullptr;
    const float* g2 = nullptr;
    const float* b2 = nullptr;
    void* y = nullptr;
    int64_t M = 0;
    int D = 0;
    float eps = 1e-5f;
    bool silu = false;   // y = silu(LN(x; g, b)): the conv module's LayerNorm conv norm (conformer.cpp:126-133, :157)
    // with g2 / b2 and y (no y_f32): y = LN2(LN(x)) and LN's {mean, rstd} per
    // row (float2 [M]); x is left as it is
    float* rows = nullptr;
};
void launch_layernorm(Precision prec, const LnParams& p, hipStream_t s);

// Conv module middle (conformer.cpp:81-157): depthwise conv (K taps,
// cross-correlation; zero padding (K-1)/2 both sides, or K-1 before only when
// causal, conformer.cpp:100-120) + bias, then with bn_scale/bn_shift the
// folded BatchNorm and SiLU into `out` in the activation type, or without them
// the raw conv + bias into `out` as f32 (for the LayerNorm conv norm).
// in [B][T][D] activation type; w [D][K].
void launch_dwconv(Precision prec, const void* in, void* out, const float* w, const float* dw_bias,
                   const float* bn_scale, const float* bn_shift, int B, int T, int D, int K, bool causal,
                   hipStream_t s);

// Output length of one k3 s2 subsampling stage: all_paddings 2, or 3 when
// causal (2 before, 1 after; subsampling.cpp:25-46).
inline int sub_stage_len(int t, bool causal) { return (t + (causal ? 3 : 2) - 3) / 2 + 1; }

// Subsampling conv.0 (subsampling.cpp:143-157: Conv2d(1->C, 3x3, s2, p1) + bias
// + ReLU over mel [B][F][T] f32, frames t >= valid0[b] zero when valid0 is set),
// the stage mask on its rows (t1 >= valid1[b] zero) and the first depthwise
// conv (subsampling.cpp:168-184), fused; output channels-last [B][T2][F2][C].
// causal: CausalConv2D padding (2 before, 1 after on both axes).
void launch_sub_stage1(Precision prec, const float* mel, const int* valid0, const int* valid1, const float* w0,
                       const float* b0, const float* w2, const float* b2, void* out, int B, int F, int T, int C,
                       hipStream_t s, bool causal = false);
// Subsampling depthwise 3x3 s2 p1 + bias (subsampling.cpp:168-184), channels-last,
// input time rows t >= vmask[b] read as zero when vmask != nullptr.
void launch_sub_dwconv(Precision prec, const void* in, const int* vmask, const float* w,
                       const float* bias, void* out, int B, int Ti, int Fi, int C, hipStream_t s,
                       bool causal = false);

// pos_enc.cpp:10-34 in f64, stored as the activation type: [2T-1][D].
void launch_rel_pos_encoding(Precision prec, void* out, int T, int D, hipStream_t s);

// Row-wise log_softmax + first-max argmax over V (ctc_decoder.cpp:107-108,
// search.cpp:57-61).  logits [M][V] f32 in, logprobs [M][V] f32 out (may alias).
void launch_log_softmax_argmax(const float* logits, float* logprobs, int32_t* argmax, int64_t M,
                               int V, hipStream_t s);

// Split argmax per row (tdt.cpp:76-79): tok = argmax[0,n_tok), dur = argmax[n_tok, n_tok+n_dur).
void elementwise_module_ready();
void launch_split_argmax(const float* logits, int64_t M, int n_tok, int n_dur, int32_t* tok,
                         int32_t* dur, hipStream_t s);

// f32 -> activation type copy (f16 mode inputs of the unit entry points).
void launch_cast_f32(Precision prec, const float* x, void* y, int64_t n, hipStream_t s);
// x[i] += y[i] (f32).
void launch_add_f32(float* x, const float* y, int64_t n, hipStream_t s);

// Time-major [B][T][D] f32 -> per-item channels-first [D][valid[b]] compacted,
// item b at out + offs[b] (encoder.cpp:158-166).
void launch_compact_channels_first(const float* x, int B, int T, int D, const int* valid,
                                   const int64_t* offs, float* out, hipStream_t s);

}  // namespace pkx

// GEMM family: Y = epilogue(X[M][K] . W[N][K]^T) on gfx950 MFMA.
//
// Replaces ggml_mul_mat(W, x) for every linear on the encoder path
// (conformer.cpp:309-324 FFN, relpos_attention.cpp:180-194,305 q/k/v/pos/out,
// conformer.cpp:48-53,158-162 pointwise convs, subsampling.cpp:189,233-236,
// ctc_decoder.cpp:98, joint.cpp:55-56) together with the element-wise ops that
// follow each of them in the reference graph (bias add, SiLU, GLU + pad mask,
// x0.5 residual, ReLU, flatten transpose), fused into the epilogue.
#pragma once
#include "common.hpp"

namespace pkx {

enum Epi : int {
    EPI_STORE = 0,      // Y(act) = alpha*(acc + bias)
    EPI_STORE_F32 = 1,  // Y(f32) = alpha*(acc + bias)
    EPI_SILU = 2,       // Y(act) = silu(acc + bias)                         conformer.cpp:321
    EPI_RESID = 3,      // R(f32) += alpha*(acc + bias)                       conformer.cpp:326-352
    EPI_GLU = 4,        // Y(act)[m][j] = a*sigmoid(b), 0 for t >= valid     conformer.cpp:55-80
    EPI_RELU = 5,       // Y(act) = relu(acc + bias)                          subsampling.cpp:189-191
    EPI_RELU_TR = 6,    // relu + flatten to [b][t][c][f], 0 for t >= valid   subsampling.cpp:194-230
    EPI_RELU2_F32 = 7,  // Y(f32) = relu((acc + bias) + bias2)                joint.cpp:89-95
    // GLU + pad mask, then depthwise conv over time (K = GLU_DW_K, zero padding
    // at each item's edges) + bias + folded BatchNorm + SiLU     conformer.cpp:55-157
    EPI_GLU_DW = 8,
    // EPI_RESID, then for the LayerNorm that follows: H(f16) = R * ln_g and the
    // statistics of R over each 32-column group (mean, sum of squared deviations)
    EPI_RESID_LN = 9,
    EPI_COUNT = 10
};

constexpr int GLU_DW_K = 9;   // depthwise kernel size of the fused conv-module epilogue

struct GemmParams {
    const void* A = nullptr;   // activations, row stride lda elements
    int64_t lda = 0;
    const void* Wq = nullptr;  // weight payload (device layout per type, see DevWeight)
    const void* Ws = nullptr;  // per-block scales (q8_0: f16 [K/64][ldw][2]; q4_K: float2 [K/64][ldw][2])
    int ldw = 0;               // q8_0 / q4_K: rows of each 64-wide K slab block of Wq / Ws (0: N)
    const float* bias = nullptr;
    const float* bias2 = nullptr;
    void* Y = nullptr;         // output (EPI_RESID: the f32 residual updated in place)
    int64_t ldy = 0;
    float alpha = 1.0f;
    const int* valid = nullptr;  // per-item valid rows; row m -> item m / T, time m % T
    int T = 1;
    int trF = 1;               // EPI_RELU_TR: rows are (b, t, f) with f fastest, F' = trF
    int M = 0, N = 0, K = 0;
    int xcd_gm = 1;            // tile grid split over the 8 XCDs: xcd_gm row bands x (8 / xcd_gm) column bands
    // EPI_GLU_DW: depthwise weights [N/2][GLU_DW_K], its bias, BatchNorm folded to
    // y = (conv + dw_b) * dw_scale + dw_shift (per channel)
    const float* dw_w = nullptr;
    const float* dw_b = nullptr;
    const float* dw_scale = nullptr;
    const float* dw_shift = nullptr;
    // EPI_GLU_DW with f16 weights: their copy in the item-tile kernel's
    // fragment order (glu_frag_prepare), or null (the kernel then reads Wq)
    const void* wfrag = nullptr;
    // EPI_RESID_LN outputs (N % 32 == 0)
    const float* ln_g = nullptr;   // [N] gamma of the next LayerNorm
    void* ln_h = nullptr;          // f16 [M][N]: R * gamma
    float* ln_stats = nullptr;     // float2 [M][N / 32]: {mean, sum of squared deviations}
    // EPI_RESID_LN: the residual read is LN(R) rather than R, with R's per-row
    // {mean, rstd} in res_rows (float2 [M]) and the LayerNorm's gamma / beta in
    // res_g / res_b [N]: R holds the stream before a LayerNorm whose output was
    // not stored, and the update writes the normalised stream plus the product
    const float* res_rows = nullptr;
    const float* res_g = nullptr;
    const float* res_b = nullptr;
    // A LayerNorm folded into this product (EPI_STORE / SILU / GLU / GLU_DW):
    // A = x * gamma (f16, from EPI_RESID_LN) and
    //   y = rstd_m * (acc - mean_m * fold_c1[n]) + bias[n],
    // fold_c1 = W . gamma, bias = W . beta + b (launch_ln_fold_consts).
    const float* fold_stats = nullptr;   // float2 [M][fold_groups]
    const float* fold_c1 = nullptr;
    int fold_groups = 0;
    float fold_eps = 1e-5f;
    // Split-K across workgroups: launch_gemm cuts the K range of small grids
    // (M <= 512 residual products) over ksplit workgroups per tile when the
    // caller supplies this workspace: sk_part holds the partial tiles
    // (sk_part_floats floats), sk_cnt one arrival counter per tile (sk_cnt_n
    // ints, zero when allocated; every launch leaves them zero again).  Calls
    // sharing one workspace must not overlap.
    float* sk_part = nullptr;
    int64_t sk_part_floats = 0;
    int* sk_cnt = nullptr;
    int sk_cnt_n = 0;
    int ksplit = 1;            // set by launch_gemm
};

// c1[n] = sum_k g[k] w[n][k], c2[n] = sum_k b[k] w[n][k] + bias[n] for a
// LayerNorm (g, b) folded into the product with device weight (Wq, Ws) of
// type wtype; w is the f16 value the GEMM's dequantisation produces.
void launch_ln_fold_consts(int wtype, const void* Wq, const void* Ws, int N, int K, const float* g,
                           const float* b, const float* bias, float* c1, float* c2, hipStream_t s);

// True when launch_gemm can run EPI_GLU_DW for this shape: the f16 MFMA path,
// N (= 2 x channels) a multiple of 64 and K a multiple of 64.
bool gemm_glu_dw_supported(Precision prec, int wtype, int N, int K);

// EPI_GLU_DW on items of T <= 128 frames runs one 128-row tile per item; with
// f16 weights it reads them from a copy in its fragment order (GemmParams::
// wfrag, glu_frag_bytes(N, K) bytes), made once by glu_frag_prepare from the
// row-major [N][K] weights.  Supported for f16, N % 128 == 0, K % 512 == 0.
bool glu_frag_supported(int wtype, int N, int K);
size_t glu_frag_bytes(int N, int K);
void glu_frag_prepare(const void* w, int N, int K, void* frag, hipStream_t s);

// Launch one GEMM.  prec selects the activation type (f16: MFMA 16x16x32 f16
// with weights dequantised to f16 in registers; f32: MFMA 16x16x4 f32 with
// weights dequantised to f32).  wtype is the ggml type of the device weight.
void launch_gemm(Precision prec, int wtype, int epi, const GemmParams& p, hipStream_t s);

// Loads the GEMM file's code object on the current device.
void gemm_module_ready();

// Bit-exact dequantisation of raw ggml blocks (GGUF layout) to f32.
void launch_dequantize(int wtype, const void* src, float* dst, int64_t n, hipStream_t s);

}  // namespace pkx

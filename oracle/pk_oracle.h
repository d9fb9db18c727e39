/*
 * pk_oracle.h -- CPU restatement of the parakeet.cpp FastConformer encoder path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * encoder and the "port" CPU baseline that bench.py times beside it.  Only the
 * tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product library never links or calls it.
 *
 * Every function names the reference file:line it restates.  The reference's
 * own arithmetic lives in ggml (an un-vendored submodule that is absent), so
 * the restatement computes the exact math of each graph op in f32 storage with
 * f32 (dot products) or f64 (norm/softmax statistics) accumulation.
 *
 * Layouts (all row-major, innermost last):
 *   activations  [B][T][D]            (ggml ne [D,T,B])
 *   weights      [N][K]               (ggml ne [K,N]; quant blocks along K)
 *   pos_emb      [2T-1][D]
 *   mel          [B][n_mels][T_max]   (MelBatch layout, src/encoder.hpp:17-23)
 */
#ifndef PK_ORACLE_H
#define PK_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids used by the GGUF weight layout. */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q4_K = 12 };

void     orc_set_threads(int n);
int      orc_get_threads(void);

/* IEEE binary16 <-> binary32, round-to-nearest-even (ggml FP32_TO_FP16). */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* Bytes of one row of ne0 elements in the given type (0 if ne0 is not a
 * multiple of the block size or the type is unknown). */
int64_t  orc_row_bytes(int type, int64_t ne0);

/* Dequantise n elements (n a multiple of the block size) to f32.
 * q8_0: 34-byte block {f16 d; i8 q[32]}, w = d*q.
 * q4_K: 144-byte super-block {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]},
 *       w = d*sc_j*q - dmin*m_j (ggml v0.13.0 block_q4_K). Returns 0 on success. */
int      orc_dequantize(int type, const void* src, float* dst, int64_t n);
/* Quantise n f32 values into the given type (f16, q8_0, q4_K): ggml's
 * quantize_row_q8_0_ref (d = f16(amax/127), q = roundf(x / (amax/127))) and
 * quantize_row_q4_K_ref (make_qkx2_quants per 32-value sub-block, 6-bit
 * scale/min codes against d = max_scale/63, dmin = max_min/63). */
int      orc_quantize(int type, const float* src, void* dst, int64_t n);

/* pos_enc.cpp:10-34 -- table [2T-1][d] for positions +(T-1) .. -(T-1). */
void orc_rel_pos_encoding(int T, int d, float* out);

/* conformer.cpp:300-307 -- y = (x-mean)/sqrt(var+eps)*g + b over the last dim. */
void orc_layer_norm(const float* x, int64_t M, int D, const float* g,
                    const float* b, float eps, float* y);

/* y[M][N] = x[M][K] . W[N][K]^T (+ bias[N]) -- ggml_mul_mat(W, x) (+ ggml_add). */
void orc_linear(const float* x, int64_t M, int K, const float* W, int N,
                const float* bias, float* y);

/* One conformer layer's weights, dequantised to f32.  Optional biases may be
 * NULL (bias=False checkpoints, relpos_attention.cpp:126-137). */
typedef struct {
    int D, H, FF, K;
    const float *ff1_ln_g, *ff1_ln_b, *ff1_w1, *ff1_b1, *ff1_w2, *ff1_b2;
    const float *att_ln_g, *att_ln_b;
    const float *wq, *bq, *wk, *bk, *wv, *bv, *wo, *bo, *wpos;
    const float *pos_bias_u, *pos_bias_v;              /* [H][dk] */
    const float *conv_ln_g, *conv_ln_b;
    const float *pw1_w, *pw1_b;                         /* [2D][D], [2D] */
    const float *dw_w, *dw_b;                           /* [D][K], [D] */
    const float *bn_g, *bn_b, *bn_mean, *bn_var;        /* [D] each */
    const float *pw2_w, *pw2_b;                         /* [D][D], [D] */
    const float *ff2_ln_g, *ff2_ln_b, *ff2_w1, *ff2_b1, *ff2_w2, *ff2_b2;
    const float *out_ln_g, *out_ln_b;
    /* streaming-model variants (model_loader.cpp:110-121); zero = offline model */
    int conv_causal;                /* depthwise conv left pad K-1, no right pad */
    int conv_ln;                    /* conv_norm_type "layer_norm" (bn_g/bn_b as gamma/beta) */
    int att_limited;                /* att_context_style "chunked_limited" */
    int att_left, att_right;        /* att_context_size [left, right] */
} orc_layer;

/* dw_striding subsampling weights (torch layouts == GGUF memory order). */
typedef struct {
    int C, D;                      /* conv channels, d_model */
    const float *w0, *b0;          /* conv.0  [C][1][3][3], [C] */
    const float *w2, *b2;          /* conv.2  depthwise [C][1][3][3] */
    const float *w3, *b3;          /* conv.3  pointwise [C][C] */
    const float *w5, *b5;          /* conv.5  depthwise */
    const float *w6, *b6;          /* conv.6  pointwise */
    const float *wout, *bout;      /* out     [D][C*F'], [D] */
    int causal;                    /* causal_downsampling: pad 2 before, 1 after on both axes */
} orc_subsampling_w;

/* relpos_attention.cpp:162-306 (batched) / :40-160 (B=1).  x is the already
 * normalised input [B][T][D]; pe [2T-1][D]; valid[B]; out [B][T][D]. */
void orc_relpos_attention(const orc_layer* L, const float* x, int B, int T,
                          const float* pe, const int* valid, float* out);

/* conformer.cpp:38-164 -- conv module after norm_conv. */
void orc_conv_module(const orc_layer* L, const float* c, int B, int T,
                     const int* valid, float* out);

/* conformer.cpp:285-353 -- full layer.  If conv_out != NULL it receives the
 * conv-module output (forward_with_conv, conformer.cpp:434). */
void orc_conformer_layer(const orc_layer* L, const float* x, int B, int T,
                         const float* pe, const int* valid, float* out,
                         float* conv_out);

/* subsampling.cpp:25-46 (all_paddings 2; _c: 3 when causal) */
int  orc_valid_out_len(int T, int in_valid);
int  orc_subsampled_len(int T);
int  orc_valid_out_len_c(int T, int in_valid, int causal);
int  orc_subsampled_len_c(int T, int causal);

/* subsampling.cpp:48-240 (stage_masks=1, batched semantics) and :242-386
 * (stage_masks=0, scalar semantics).  mel [B][F][T]; valid_in[b] is the entry
 * valid length (NULL -> T-1 per item).  out [B][T'][D]; valid_out[B]. */
int  orc_subsampling(const orc_subsampling_w* S, const float* mel, int B, int F,
                     int T, const int* valid_in, int stage_masks, float* out,
                     int* valid_out);

/* encoder.cpp:97-167.  out [B][T'][D] (time-major, uncompacted).
 * capture (optional) receives every layer output [L][B][T'][D]. */
int  orc_encoder_forward(const orc_subsampling_w* S, const orc_layer* layers,
                         int n_layers, int xscaling, const float* mel, int B,
                         int F, int T, const int* valid_in, int stage_masks,
                         float* out, int* valid_out, float* capture);

/* ---- cache-aware streaming encoder (streaming_encoder.cpp) ---------------- */
/* StreamingEncoder state (streaming_encoder.hpp:55-95): per layer the
 * attention cache of norm_self_att outputs [cache_len][D] and the depthwise
 * conv cache of GLU outputs [K-1][D], time-major, zero at reset. */
typedef struct orc_stream orc_stream;
orc_stream* orc_stream_new(const orc_subsampling_w* S, const orc_layer* layers, int n_layers,
                           int xscaling, int F, int cache_len, int drop_extra, int valid_out_len);
void orc_stream_free(orc_stream* st);
void orc_stream_reset(orc_stream* st);
/* StreamingEncoder::step (streaming_encoder.cpp:340-462): mel window [F][n]
 * (pre-encode overlap included); writes the kept frames [n_valid][D] to out
 * (capacity: the window's subsampled length) and returns n_valid. */
int  orc_stream_step(orc_stream* st, const float* mel, int n, int is_last, float* out);
/* The chunk output length before the valid slice (0 when the window is too short). */
int  orc_stream_chunk_len(const orc_stream* st, int n);

/* ctc_decoder.cpp:34-116 -- log_softmax(enc . W^T + b) over V, enc [T][D]
 * time-major; argmax with first-max tie-break (search.cpp:57-61). */
void orc_ctc_head(const float* enc, int T, int D, const float* W, const float* b,
                  int V, float* logprobs, int32_t* argmax);
/* search.cpp:21-90 -- collapse repeats and blanks; returns the token count. */
int  orc_ctc_greedy(const int32_t* argmax, int T, int blank_id, int32_t* out);

/* joint.cpp:37-63 enc_proj, :65-104 step logits, tdt.cpp:76-79 split argmax.
 * For every frame t: f = relu(enc_proj[t] + pred_proj), logits = Wout f + bout,
 * tok[t] = argmax logits[0, n_tok), dur[t] = argmax logits[n_tok, n_tok+n_dur). */
void orc_tdt_joint_argmax(const float* enc, int T, int D, const float* Wenc,
                          const float* benc, int Hj, const float* g, int P,
                          const float* Wpred, const float* bpred,
                          const float* Wout, const float* bout, int n_tok,
                          int n_dur, float* logits, int32_t* tok, int32_t* dur);

/* ---- greedy transducer decode (prediction.cpp, joint.cpp, tdt.cpp,
 *      transducer_batch.cpp, decode_common.hpp) ------------------------------ */
typedef struct {
    int H, L, V1;                     /* pred_hidden, LSTM layers (<= 4), embedding rows (vocab+1) */
    const float* embed;               /* [V1][H] */
    const float *w_ih[4], *w_hh[4];   /* [4H][H] per layer, gates (i, f, g, o) */
    const float *b_ih[4], *b_hh[4];   /* [4H] */
    int Hj, D, Vp;                    /* joint hidden, encoder width, vocab + 1 + n_durations */
    const float *jenc_w, *jenc_b;     /* [Hj][D], [Hj] */
    const float *jpred_w, *jpred_b;   /* [Hj][H], [Hj] */
    const float *jout_w, *jout_b;     /* [Vp][Hj], [Vp] */
} orc_transducer;

/* prediction.cpp:47-109 -- one stacked-LSTM step: x = embed[token] (zeros
 * for SOS), per layer z = (W_ih x + b_ih) + (W_hh h + b_hh),
 * c' = sigmoid(f) c + sigmoid(i) tanh(g), h' = sigmoid(o) tanh(c').
 * h_in/c_in/h_out/c_out [L][H]; g_out = top-layer h'. */
void orc_lstm_step(const orc_transducer* m, int32_t token, int is_sos, const float* h_in, const float* c_in,
                   float* h_out, float* c_out, float* g_out);
/* tdt.cpp:8-118 (n_dur > 0) / rnnt greedy (n_dur == 0) for one item, enc
 * [T][D]: emitted ids with NeMo's per-token frame, max_prob confidence and
 * span (decode_types.hpp).  Returns the count, -1 if cap is exceeded. */
int orc_transducer_greedy(const orc_transducer* m, const float* enc, int T, const int32_t* durations, int n_dur,
                          int blank_id, int max_symbols, int32_t* ids, int32_t* frames, float* conf,
                          int32_t* span, int cap);

/* ---- log-mel front end (mel.cpp, fft.cpp, model.cpp:114-146) ------------ */
typedef struct {
    int n_fft, hop, n_mels, per_feature;   /* per_feature: normalize == "per_feature" */
    float preemph, mag_power, log_guard;
} orc_mel_cfg;

/* mel.cpp:25-46 -- a win_length window centre-padded to n_fft. */
void orc_mel_window(const float* win, int win_len, int n_fft, float* out);
/* Frames of an S-sample clip: 1 + (S + 2 (n_fft/2) - n_fft) / hop (mel.cpp:132-135). */
int  orc_mel_frames(const orc_mel_cfg* c, int S);
/* fft.cpp:9-74 -- radix-2 rfft of n floats (n a power of two), bins 0..n/2 as f32. */
void orc_rfft(const float* in, int n, float* re, float* im);
/* mel.cpp:99-185 -- MelFrontend::compute for one clip: feats [n_mels][T]
 * (window: n_fft values, fb: [n_mels][n_fft/2+1]).  Returns T. */
int  orc_mel(const orc_mel_cfg* c, const float* window, const float* fb,
             const float* samples, int S, float* feats);
/* model.cpp:119-146 -- build_mel_batch: per-clip log-mel stacked to T_max,
 * out [B][n_mels][T_max] zero-padded, T_out[b] each clip's frame count. */
void orc_mel_batch(const orc_mel_cfg* c, const float* window, const float* fb,
                   const float* pcm, int B, int S_stride, const int* n_samples,
                   int T_max, float* out, int* T_out);

#ifdef __cplusplus
}
#endif
#endif

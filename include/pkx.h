/*
 * pkx.h -- C ABI of the MI355X (gfx950) FastConformer encoder for parakeet.cpp.
 *
 * Plain C: pointers, sizes and int status codes (0 = ok, nonzero = error with
 * a message in pkx_last_error()).  No C++ exception crosses this boundary.
 * "dev" pointers are device (HBM) addresses; "host" pointers are CPU memory.
 * Every compute call is asynchronous on the given stream (NULL = default
 * stream) unless stated otherwise.
 *
 * Layouts follow the reference (see the citations on each entry point):
 *   mel          [B][n_mels][T_max] f32      (MelBatch, src/encoder.hpp:17-23)
 *   activations  [B][T][d_model]    f32      (ggml ne [d,T,B])
 *   weights      GGUF v3 tensors, verbatim NeMo names, ggml ne order,
 *                types f32 / f16 / q8_0 / q4_K (docs/conversion.md:21-128,
 *                docs/quantization.md:74-99)
 *
 * One model handle owns its device weights and a grow-only workspace.  A
 * handle is not re-entrant: calls on one handle must not overlap (the
 * reference serialises all compute behind one mutex, src/ggml_graph.cpp:35,84);
 * distinct handles may run concurrently on distinct streams.
 */
#ifndef PKX_H
#define PKX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKX_ABI_VERSION 3

typedef struct pkx_model pkx_model;

/* ggml type ids accepted for weights (the GGUF layout's own numbering). */
enum { PKX_TYPE_F32 = 0, PKX_TYPE_F16 = 1, PKX_TYPE_Q8_0 = 8, PKX_TYPE_Q4_K = 12 };

/* Compute precision of a model handle.
 *   F32: f32 activations, weights dequantised to f32, f32 MFMA (16x16x4) GEMMs
 *        -- the exact-precision path (f32 GGUFs, parity at 1e-4).
 *   F16: f32 residual stream and statistics, f16 GEMM/attention operands with
 *        f32 accumulation, weights dequantised to f16 in registers
 *        (f16 / q8_0 / q4_K GGUFs; f32 pointwise-conv weights are converted
 *        to f16 at upload).
 *   AUTO: F16 if any allowlisted linear is f16/q8_0/q4_K, else F32. */
enum { PKX_PREC_AUTO = -1, PKX_PREC_F32 = 0, PKX_PREC_F16 = 1 };

/* Subsampling time-masking semantics.
 *   BATCHED: zero trailing frames before every conv stage
 *            (Subsampling::build_graph_batched, src/subsampling.cpp:95-147,
 *            used by Encoder::forward_batch).
 *   SCALAR:  mask only the flattened output (Subsampling::build_graph,
 *            src/subsampling.cpp:281-300, used by Encoder::forward). */
enum { PKX_MASK_BATCHED = 0, PKX_MASK_SCALAR = 1 };
/* Flag or-ed into pkx_subsampling_forward's mask_mode: valid_T holds entry valid
 * lengths as the streaming windows count them (every frame of the window is
 * audio, src/subsampling.hpp:53-61: in_valid_frames), 1 <= valid_T[b] <= T_max,
 * instead of true frame counts whose entry valid length is one less. */
enum { PKX_MASK_WHOLE_FRAMES = 4 };

/* Encoder hyper-parameters (the encoder fields of pk::ParakeetConfig,
 * src/model_loader.hpp:27-52; GGUF keys parakeet.encoder.*). */
typedef struct {
    int d_model, n_layers, n_heads, ff_dim, conv_kernel;
    int n_mels;          /* parakeet.encoder.feat_in */
    int sub_channels;    /* parakeet.encoder.subsampling_conv_channels */
    int xscaling;        /* parakeet.encoder.xscaling */
    int vocab_size;      /* parakeet.vocab_size (CTC/TDT heads: vocab_size + 1 tokens) */
    int n_durations;     /* len(parakeet.tdt.durations), 0 if no TDT head */
    /* cache-aware streaming models (src/model_loader.cpp:110-131); all zero
     * (att_left/att_right -1) for offline models */
    int conv_ln;         /* parakeet.encoder.conv_norm_type == "layer_norm" */
    int causal_sub;      /* parakeet.encoder.causal_downsampling */
    int conv_causal;     /* parakeet.encoder.conv_causal */
    int att_limited;     /* att_context_style == "chunked_limited" and att_right >= 0 */
    int att_left, att_right;
    int stream_chunk_first, stream_chunk, stream_pre_cache;   /* parakeet.streaming.*: mel frames */
    int stream_cache_len, stream_valid_out_len, stream_drop_extra;
} pkx_config;

/* ---- status ---------------------------------------------------------------- */
int         pkx_abi_version(void);
/* Message of the last failing call on this thread ("" if none). */
const char* pkx_last_error(void);

/* ---- device plumbing (HIP runtime, for callers without their own) ---------- */
int pkx_device_count(int* n);
int pkx_malloc(void** dev, size_t bytes);
int pkx_free(void* dev);
/* Free and total device memory of the current device (hipMemGetInfo). */
int pkx_mem_info(size_t* free_bytes, size_t* total_bytes);
int pkx_memcpy_h2d(void* dev_dst, const void* host_src, size_t bytes, void* stream);
int pkx_memcpy_d2h(void* host_dst, const void* dev_src, size_t bytes, void* stream);
int pkx_memcpy_d2d(void* dev_dst, const void* dev_src, size_t bytes, void* stream);
int pkx_stream_create(void** stream);
int pkx_stream_destroy(void* stream);
int pkx_stream_synchronize(void* stream);
int pkx_event_create(void** event);
int pkx_event_destroy(void* event);
int pkx_event_record(void* event, void* stream);
int pkx_event_elapsed_ms(float* ms, void* start, void* stop);   /* synchronises on stop */

/* ---- model handle ----------------------------------------------------------
 * Replaces pk::ModelLoader::load + realize_weights (src/model_loader.cpp:47-167)
 * for the encoder path: weights are uploaded once and never re-copied. */

/* Read a GGUF v3 file (parakeet.* KV + verbatim tensor names) and upload the
 * encoder, CTC-head and TDT-joint tensors.  precision: PKX_PREC_*. */
int pkx_model_load_gguf(const char* path, int precision, pkx_model** out);

/* Every key-value pair of a GGUF v3 header, in file order: the KV half of
 * gguf_init_from_file that pk::ModelLoader::load reads ParakeetConfig from
 * (src/model_loader.cpp:99-156).  visit(user, key, type, elem_type, n, data):
 * type is the GGUF value type (4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array,
 * ...); elem_type is the element type of an array and equals type for a
 * scalar; n is the element count (1 for a scalar); data points to n packed
 * little-endian values (bools as one byte), or to n pkx_gguf_str for strings.
 * Pointers are valid only during the call. */
typedef struct { const char* s; size_t n; } pkx_gguf_str;
typedef void (*pkx_gguf_kv_fn)(void* user, const char* key, int type, int elem_type, uint64_t n, const void* data);
int pkx_gguf_read_kv(const char* path, pkx_gguf_kv_fn visit, void* user);

/* Build a handle from tensors supplied one by one (same names, ggml ne order
 * and raw bytes as in a GGUF), then pkx_model_finalize(). */
int pkx_model_create(const pkx_config* cfg, int precision, pkx_model** out);
int pkx_model_set_tensor(pkx_model* m, const char* name, int ggml_type, int n_dims,
                         const int64_t* ne, const void* host_data, size_t nbytes);
int pkx_model_finalize(pkx_model* m);
int pkx_model_free(pkx_model* m);
/* precision: resolved PKX_PREC_F32/F16; has_ctc/has_joint: heads present. */
int pkx_model_info(pkx_model* m, pkx_config* cfg, int* precision, int* has_ctc, int* has_joint);

/* ---- length arithmetic (pk::Subsampling::valid_out_len, src/subsampling.cpp:25-46) */
int pkx_subsampled_len(int T_mel);
int pkx_valid_out_len(int T_mel, int in_valid);   /* in_valid < 0: offline T-1 */

/* ---- hot path ----------------------------------------------------------------
 * Replaces pk::Encoder::forward_batch (src/encoder.cpp:97-167) and
 * forward_capture (src/encoder.cpp:30-95): subsampling -> xscaling ->
 * rel-pos table -> n_layers conformer blocks, one stream-ordered launch
 * sequence.
 *   mel_dev     [B][n_mels][T_max] f32
 *   valid_T     host [B]: true mel frames per item (NULL = T_max); the entry
 *               valid length is valid_T[b]-1 (src/encoder.cpp:111-112)
 *   out_dev     [B][T'][d_model] f32, T' = pkx_subsampled_len(T_max); frames
 *               t >= valid_out[b] are padding (not zeroed, as in the reference)
 *   T_out       host: T'
 *   valid_out   host [B] (may be NULL)
 *   capture_dev NULL, or [n_layers][B][T'][d_model] f32 per-layer outputs */
int pkx_encoder_forward(pkx_model* m, const float* mel_dev, int B, int T_max,
                        const int* valid_T, int mask_mode, float* out_dev, int* T_out,
                        int* valid_out, float* capture_dev, void* stream);

/* Per-item channels-first compaction of an encoder output
 * (src/encoder.cpp:158-166): item b -> out_dev + offs[b], [d_model][valid[b]].
 * valid_dev [B] int32 and offs_dev [B] int64 are device arrays. */
int pkx_compact_channels_first(const float* x_dev, int B, int T, int d_model,
                               const int* valid_dev, const int64_t* offs_dev, float* out_dev,
                               void* stream);

/* pk::Subsampling::forward / build_graph_batched (src/subsampling.cpp:48-240,
 * :242-386, :388-419): out_dev [B][T'][d_model].  xscaling is not applied
 * here (it belongs to the encoder, src/encoder.cpp:122-124). */
int pkx_subsampling_forward(pkx_model* m, const float* mel_dev, int B, int T_max,
                            const int* valid_T, int mask_mode, float* out_dev, int* T_out,
                            int* valid_out, void* stream);

/* pk::ConformerLayer::forward / forward_with_conv (src/conformer.cpp:426-516)
 * and build_graph_batched (:285-353).  x_dev, out_dev [B][T][d_model] f32
 * (may alias); valid host [B] (NULL = T); conv_out_dev NULL or [B][T][d_model]
 * receives the conv-module output.  pos_emb_dev is the caller's relative
 * positional table [2T-1][d_model] f32 (the reference's pos_emb argument,
 * src/conformer.hpp:70-91), used as given; NULL computes
 * pk::rel_pos_encoding(T, d_model) on the device. */
int pkx_conformer_layer_forward(pkx_model* m, int layer, const float* x_dev, int B, int T,
                                const int* valid, const float* pos_emb_dev, float* out_dev,
                                float* conv_out_dev, void* stream);

/* pk::RelPosAttention::forward / build_graph_batched
 * (src/relpos_attention.cpp:162-306, :308-333): x_dev is the already
 * normalised input [B][T][d_model]; pos_emb_dev as for
 * pkx_conformer_layer_forward (src/relpos_attention.hpp:52-55). */
int pkx_relpos_attention_forward(pkx_model* m, int layer, const float* x_dev, int B, int T,
                                 const int* valid, const float* pos_emb_dev, float* out_dev,
                                 void* stream);

/* pk::ConformerLayer::conv_module_forward (src/conformer.cpp:518-543) and
 * build_conv_module (:38-164): c_dev = norm_conv(residual). */
int pkx_conv_module_forward(pkx_model* m, int layer, const float* c_dev, int B, int T,
                            const int* valid, float* out_dev, void* stream);

/* pk::CTCDecoder::forward (src/ctc_decoder.cpp:34-116) over M time-major frames
 * enc_dev [M][d_model]: logprobs_dev [M][vocab+1] f32 (log_softmax) and
 * argmax_dev [M] int32 (first max, src/search.cpp:57-61). */
int pkx_ctc_forward(pkx_model* m, const float* enc_dev, int64_t M, float* logprobs_dev,
                    int32_t* argmax_dev, void* stream);

/* TDT joint over every frame with one prediction-net output g:
 * Joint::precompute_enc_proj + step_logits (src/joint.cpp:37-104) and the
 * split argmax of tdt_greedy (src/tdt.cpp:76-79).  g_dev [pred_hidden];
 * logits_dev [M][vocab+1+n_durations]; tok_dev, dur_dev [M] int32. */
int pkx_tdt_joint_argmax(pkx_model* m, const float* enc_dev, int64_t M, const float* g_dev,
                         float* logits_dev, int32_t* tok_dev, int32_t* dur_dev, void* stream);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops or harnesses that forbid
 * hipMalloc).  pkx_tdt_joint_argmax with the same kernels and results, its
 * scratch (the prediction projection [joint_hidden] and the joint hidden
 * activations [M][joint_hidden], f32) held in a fixed per-GPU device array of
 * PKX_JOINT_NOALLOC_MAX_FLOATS floats (16 MiB, kept until the process ends)
 * instead of the model's grow-only workspace.  Calls no hipMalloc / hipFree.
 * Fails (nonzero, message in pkx_last_error) when
 * M > (PKX_JOINT_NOALLOC_MAX_FLOATS - joint_hidden rounded up to 64) /
 * joint_hidden, i.e. 6552 frames at joint_hidden 640.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (any stream, any
 * model handle) race. */
#define PKX_JOINT_NOALLOC_MAX_FLOATS (4u << 20)
int pkx_tdt_joint_argmax_noalloc(pkx_model* m, const float* enc_dev, int64_t M, const float* g_dev,
                                 float* logits_dev, int32_t* tok_dev, int32_t* dur_dev, void* stream);

/* ---- kernel-level entry points (ggml ops the encoder issues) ---------------- */

/* Dequantise n raw ggml-layout elements (q8_0 / q4_K / f16) to f32, bit-exact
 * with ggml's dequantize_row_* (the src0 side of ggml_mul_mat). */
int pkx_dequantize(int ggml_type, const void* src_dev, float* dst_dev, int64_t n, void* stream);

/* y = x . W^T (+ bias): ggml_mul_mat(W, x) + ggml_add with W given in raw GGUF
 * layout (host_w, N rows of K), uploaded for this call.  precision selects the
 * F32 or F16 path.  x_dev [M][K] f32, y_dev [M][N] f32. */
int pkx_linear(int precision, int ggml_type, int N, int K, const void* host_w, size_t nbytes,
               const float* bias_dev, const float* x_dev, int64_t M, float* y_dev, void* stream);

/* y += alpha * (x . W^T + bias): the residual products of the encoder
 * (ggml_add(r, ggml_scale(ggml_mul_mat(W, x), 0.5)), src/conformer.cpp:326-330,
 * with alpha 0.5; alpha 1 for linear_out / pointwise_conv2) on the kernels the
 * encoder runs them with, including the split-K path for products of at most
 * 512 rows and K >= 1024.  y_dev [M][N] f32, read and written. */
int pkx_linear_residual(int precision, int ggml_type, int N, int K, const void* host_w, size_t nbytes,
                        const float* bias_dev, const float* x_dev, int64_t M, float alpha, float* y_dev,
                        void* stream);

/* LayerNorm over the last dim, f32 in/out (ggml_norm + mul + add,
 * src/conformer.cpp:300-307). */
int pkx_layernorm(const float* x_dev, const float* g_dev, const float* b_dev, float* y_dev,
                  int64_t M, int D, float eps, void* stream);

/* pk::rel_pos_encoding (src/pos_enc.cpp:10-34): out_dev [2T-1][D] f32. */
int pkx_rel_pos_encoding(int T, int D, float* out_dev, void* stream);

/* ---- greedy transducer decode ---------------------------------------------------
 * transducer_greedy_batch (src/transducer_batch.cpp:24-213): the batched greedy
 * TDT (n_durations > 0, frame advance = durations[argmax of the duration
 * logits]) or RNNT (n_durations = 0) decode over the model's prediction
 * network (src/prediction.cpp) and joint (src/joint.cpp), on the device.
 * enc_dev [B][T_max][d_model] f32 (the encoder output, time-major), T_valid
 * (host) frames per item.  Outputs (host, [B][cap] each, NULL to skip): token
 * ids, NeMo frame / max_prob confidence / span per token (src/decode_types.hpp);
 * counts (host) [B] tokens per item.  A decode needing more than cap tokens
 * for an item is an error. */
int pkx_transducer_greedy(pkx_model* m, const float* enc_dev, int B, int T_max, const int* T_valid,
                          const int32_t* durations, int n_durations, int blank_id, int max_symbols, int cap,
                          int32_t* ids, int32_t* frames, float* conf, int32_t* span, int* counts, void* stream);

/* ---- cache-aware streaming encoder --------------------------------------------
 * pk::StreamingEncoder (src/streaming_encoder.hpp:33-95, .cpp:340-462) for
 * models with a streaming configuration (pkx_config.att_limited and the causal
 * flags; the GGUF's parakeet.streaming.* keys), for n_streams streams advanced
 * together (each its own caches; all take windows of the same length).  The
 * model must outlive the handle; one handle is not re-entrant. */
typedef struct pkx_streaming pkx_streaming;
/* StreamingEncoder::StreamingEncoder + reset(): windows of at most max_window
 * mel frames (pre-encode overlap included; at most 255). */
int pkx_streaming_create(pkx_model* m, int n_streams, int max_window, void* stream, pkx_streaming** out);
int pkx_streaming_free(pkx_streaming* st);
/* StreamingEncoder::reset (:72-79): zero caches, step 0. */
int pkx_streaming_reset(pkx_streaming* st, void* stream);
/* chunk_size_first / chunk_size / pre_encode_cache_size / valid_out_len /
 * step_num (streaming_encoder.hpp:62-67); NULL outputs are skipped. */
int pkx_streaming_info(const pkx_streaming* st, int* chunk_first, int* chunk, int* pre_cache, int* valid_out_len,
                       int* step);
/* Encoder frames the next step yields for a window of n mel frames (before the
 * valid slice): the subsampled length minus the drop of every step after the
 * first (:350-366); -1 for a null handle. */
int pkx_streaming_chunk_len(const pkx_streaming* st, int n_mel_frames);
/* StreamingEncoder::step for every stream: mel_dev [n_streams][n_mels][n]
 * f32; out_dev [n_streams][chunk_len][d_model] f32 receives every chunk frame,
 * of which the first *n_valid are the step's output (valid_out_len mid-stream,
 * all on the last chunk: keep_all_outputs). */
int pkx_streaming_step(pkx_streaming* st, const float* mel_dev, int n_mel_frames, int is_last, float* out_dev,
                       int* n_valid, void* stream);

/* ---- log-mel front end --------------------------------------------------------
 * pk::MelFrontend::compute (src/mel.hpp:33-41, src/mel.cpp:99-185) for a batch
 * of 16 kHz mono clips, stacked to T_max as build_mel_batch does
 * (src/model.cpp:114-146), on the device.  f64 preemphasis, radix-2 FFT,
 * power, filterbank sum and log with the reference's f32 roundings; per-feature
 * normalisation over each clip's first n_samples/hop frames. */
typedef struct pkx_mel pkx_mel;
typedef struct {
    int n_fft, win_length, hop_length, n_mels;
    int per_feature;      /* parakeet.preprocessor.normalize == "per_feature" */
    float preemph, mag_power, log_zero_guard;
} pkx_mel_config;

/* MelKernel::MelKernel (src/mel.cpp:16-61): window of window_len values
 * (centre-padded to n_fft), filterbank fb [n_mels][n_fft/2+1].  n_fft is a
 * power of two in [64, 512]. */
int pkx_mel_create(const pkx_mel_config* cfg, const float* window, int window_len, const float* fb,
                   pkx_mel** out);
/* The same from a GGUF: parakeet.preprocessor.* (src/model_loader.cpp:133-141)
 * and the preprocessor.featurizer.window / .fb tensors. */
int pkx_mel_load_gguf(const char* path, pkx_mel** out);
int pkx_mel_free(pkx_mel* m);
int pkx_mel_info(const pkx_mel* m, pkx_mel_config* cfg);
/* Frames of an n-sample clip (src/mel.cpp:132-135): 1 + n/hop for an even n_fft,
 * 0 for n = 0; -1 for a null handle. */
int pkx_mel_frames(const pkx_mel* m, int n_samples);
/* pcm_dev [B][S_stride] f32, n_samples (host) [B] <= S_stride ->
 * mel_dev [B][n_mels][T_max] (T_max >= every clip's frames, zero-padded),
 * T_out (host) [B] frames per clip.  Returns once the batch is computed; one
 * handle is not re-entrant. */
int pkx_mel_forward(pkx_mel* m, const float* pcm_dev, int B, int64_t S_stride, const int* n_samples,
                    float* mel_dev, int T_max, int* T_out, void* stream);

/* ---- weight quantisation ------------------------------------------------------
 * ggml_quantize_chunk for q8_0 (gtype 8) and q4_K (gtype 12) on the device,
 * the quantisers parakeet-cli quantize runs (examples/cli/main.cpp:322-426;
 * ggml v0.13.0 quantize_row_q8_0_ref / quantize_row_q4_K_ref, same f32
 * operations): src_dev [n_rows][n_per_row] f32 -> dst_dev n_rows rows of
 * blocks (n_per_row % 32 for q8_0, % 256 for q4_K). */
int pkx_quantize(int gtype, const float* src_dev, void* dst_dev, int64_t n_rows, int64_t n_per_row, void* stream);
/* parakeet-cli quantize <in> <out> <type> (examples/cli/main.cpp:322-426):
 * every KV pair copied verbatim; the allowlisted f32 2-D linears (main.cpp:
 * 279-303) with ne0 divisible by the block quantised on the device, the other
 * allowlisted 2-D f32 tensors kept (n_skipped), everything else copied.
 * gtype: 8 (q8_0) or 12 (q4_K), the types this encoder runs.  Counts may be
 * NULL. */
int pkx_quantize_gguf(const char* in_path, const char* out_path, int gtype, int* n_quantized, int* n_kept,
                      int* n_skipped);

/* ---- profiling ----------------------------------------------------------------
 * No counterpart in the reference (its benchmarks time whole calls).
 * family_mask selects kernel families by bit (bit i = family i in the order
 * subsampling, layernorm, gemm_ffn, gemm_qkv, gemm_pos, attention, gemm_out,
 * gemm_pw1_glu, dwconv, gemm_pw2, pos_enc); 0 turns profiling off and every
 * call resets the totals.  Kernels of a selected family are launched with
 * start/stop events on their own dispatch (no extra packets, no host syncs), so
 * the times are kernel execution times.  stride >= 1 samples every stride-th
 * launch of the selected families (counted across calls), which keeps the
 * per-launch event cost off most launches of a timed run.  pkx_model_profile_read waits for the
 * pending launches and returns accumulated milliseconds and kernel launch
 * counts per family (arrays of PKX_PROF_FAMILIES entries).  Profiling state is
 * per model and per calling thread. */
#define PKX_PROF_FAMILIES 11
#define PKX_PROF_ALL ((1u << PKX_PROF_FAMILIES) - 1u)
int pkx_model_set_profiling(pkx_model* m, unsigned family_mask, int stride);
int pkx_model_profile_read(pkx_model* m, double* ms, int64_t* launches);

#ifdef __cplusplus
}
#endif
#endif /* PKX_H */

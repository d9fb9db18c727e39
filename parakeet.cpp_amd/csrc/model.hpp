// Device-resident encoder model and its forward orchestration.
//
// Replaces the reference's L2 graph runtime for the encoder path
// (backend.cpp:140-285, ggml_graph.cpp:81-98, model_loader.cpp:47-98): weights
// are uploaded once, repacked into MFMA-friendly layouts (q8_0 -> int8 + f16
// scale planes, q4_K -> nibble plane + {d*sc, dmin*m} pairs, pointwise_conv1
// rows interleaved for the fused GLU epilogue, q/k/v concatenated), BatchNorm
// is folded once at upload instead of per call (conformer.cpp:134-154), and a
// grow-only workspace holds every activation of a forward.
#pragma once
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "attention.hpp"
#include "common.hpp"
#include "elementwise.hpp"
#include "gemm.hpp"
#include "subsampling.hpp"

namespace pkx {

struct ModelConfig {
    int d_model = 0, n_layers = 0, n_heads = 0, ff_dim = 0, conv_kernel = 0;
    int n_mels = 0, sub_channels = 0;
    int xscaling = 0;
    int vocab_size = 0, n_durations = 0;
    // cache-aware streaming models (model_loader.cpp:110-131); zeros = offline
    int conv_ln = 0;              // conv_norm_type "layer_norm"
    int causal_sub = 0;           // causal_downsampling
    int conv_causal = 0;          // causal depthwise conv
    int att_limited = 0;          // att_context_style "chunked_limited" (att_right >= 0)
    int att_left = -1, att_right = -1;
    int stream_chunk_first = 0, stream_chunk = 0, stream_pre_cache = 0;   // mel frames
    int stream_cache_len = 0, stream_valid_out_len = 0, stream_drop_extra = 0;
};

struct HostTensor {
    int gtype = GT_F32;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};   // ggml order (ne[0] fastest)
    std::vector<uint8_t> bytes;
    int64_t nelem() const { return ne[0] * ne[1] * ne[2] * ne[3]; }
};

// Device weight layouts: f32 / f16 [N][K]; q8_0 slab-major, int8 [K/64][ldn][64]
// with f16 scales [K/64][ldn][2] (one 64-wide K slab of ldn rows is contiguous,
// so a GEMM tile's slab of weights and of scales each stream as whole cache
// lines); q4_K slab-major too, nibbles [K/64][ldn][32] with float2
// {scale, min} [K/64][ldn][2].
struct DevWeight {
    int gtype = -1;   // device storage type (GT_F32/GT_F16/GT_Q8_0/GT_Q4_K)
    int N = 0, K = 0;
    int ldn = 0;      // q8_0 / q4_K: rows per slab block (N of the allocation a view points into)
    void* q = nullptr;
    void* s = nullptr;
    bool ok() const { return gtype >= 0; }
};

struct LayerDev {
    float *ff1_ln_g = nullptr, *ff1_ln_b = nullptr, *att_ln_g = nullptr, *att_ln_b = nullptr;
    float *conv_ln_g = nullptr, *conv_ln_b = nullptr, *ff2_ln_g = nullptr, *ff2_ln_b = nullptr;
    float *out_ln_g = nullptr, *out_ln_b = nullptr;
    DevWeight ff1_w1, ff1_w2, ff2_w1, ff2_w2;
    float *ff1_b1 = nullptr, *ff1_b2 = nullptr, *ff2_b1 = nullptr, *ff2_b2 = nullptr;
    DevWeight wqkv, wo, wpos;
    float *bqkv = nullptr, *bo = nullptr, *pos_u = nullptr, *pos_v = nullptr;
    DevWeight pw1, pw2;
    float *pw1_b = nullptr, *pw2_b = nullptr, *dw_w = nullptr, *dw_b = nullptr;
    float *bn_scale = nullptr, *bn_shift = nullptr;
    float *cn_g = nullptr, *cn_b = nullptr;   // conv_norm_type "layer_norm": gamma, beta
    // LayerNorms folded into the product that follows them (f16 path):
    // c1 = W . gamma, c2 = W . beta + b for norm_self_att -> q/k/v,
    // norm_conv -> pointwise_conv1, norm_feed_forward2 -> feed_forward2.linear1
    float *qkv_c1 = nullptr, *qkv_c2 = nullptr, *pw1_c1 = nullptr, *pw1_c2 = nullptr;
    float *ff2_c1 = nullptr, *ff2_c2 = nullptr;
    // f16 pointwise_conv1 in the conv-module item-tile kernel's fragment order
    // (glu_frag_prepare), or null
    void* pw1_frag = nullptr;
};

struct SubDev {
    float *w0 = nullptr, *b0 = nullptr, *w2 = nullptr, *b2 = nullptr, *w5 = nullptr, *b5 = nullptr;
    DevWeight w3, w6, out;
    float *b3 = nullptr, *b6 = nullptr, *bout = nullptr;
    void* tail_w = nullptr;   // conv.3 / conv.6 in MFMA fragment order (fused tail only)
};

struct HeadsDev {
    DevWeight ctc;
    float* ctc_b = nullptr;
    DevWeight jenc, jpred, jout;
    float *jenc_b = nullptr, *jpred_b = nullptr, *jout_b = nullptr;
    int n_tok = 0, n_dur = 0;
};

// RNNT/TDT prediction network on the device (prediction.hpp:27-50): the
// stacked LSTM with each layer's [W_ih | W_hh] concatenated along K, so one
// f32 product gives z = W_ih x + W_hh h; biases summed.
struct PredDev {
    int H = 0, L = 0, V1 = 0;
    float* embed = nullptr;            // [V1][H]
    float* wcat[4] = {};               // [4H][2H] f32 row-major
    float* bsum[4] = {};               // b_ih + b_hh, [4H]
    float* jpred = nullptr;            // joint.pred.weight as f32 [Hj][H]
    float* jout = nullptr;             // joint.joint_net.2.weight as f32 [Vp][Hj]
    bool ok() const { return L > 0; }
};

// State of a group of cache-aware streams advanced in lockstep
// (StreamingEncoder, streaming_encoder.hpp:33-95).  The attention cache holds
// the projected keys and values of the last cache_len frames (the reference
// keeps norm_self_att outputs and projects them again every chunk; the
// projection is linear, so caching its result gives the same keys and values
// without recomputing cache_len rows per layer and chunk) in a ring per layer
// and stream; the conv cache holds the last K-1 GLU outputs.  Device buffers
// are owned here and sized at creation.
struct StreamState {
    int B = 0, max_window = 0, tc_max = 0, tsub_max = 0;
    int CL = 0, LP = 0, np = 0;
    int step = 0, clc = 0, head = 0;   // chunks taken, valid cache frames, ring start
    void* kc = nullptr;                // [L][B][CL][D] keys, activation type
    void* vc = nullptr;                // [L][B][CL][D] values, activation type
    float* cc = nullptr;               // [L][B][LP][D] GLU history, oldest first
    void* ppos = nullptr;              // [L][np][D] act: linear_pos of the table rows for
                                       // distances CL+tc_max-1 .. -(tc_max-1)
    float* sub = nullptr;              // [B][tsub_max][D] subsampled window
    float* x = nullptr;                // [B][tc_max][D] residual stream
    void *h = nullptr, *u = nullptr, *qkv = nullptr, *g = nullptr;   // activations
    std::vector<void*> allocs;
    ~StreamState();
};

// Per-kernel-family timing collected when profiling is enabled.
enum KFam : int {
    KF_SUBSAMPLING = 0, KF_LAYERNORM, KF_GEMM_FFN, KF_GEMM_QKV, KF_GEMM_POS, KF_ATTENTION,
    KF_GEMM_OUT, KF_GEMM_PW1_GLU, KF_DWCONV, KF_GEMM_PW2, KF_POS_ENC, KF_COUNT
};

class Model {
public:
    Model(const ModelConfig& cfg, int precision);
    ~Model();
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    void set_tensor(const std::string& name, int gtype, int n_dims, const int64_t* ne,
                    const void* data, size_t nbytes);
    void finalize();

    const ModelConfig& config() const { return cfg_; }
    Precision precision() const { return prec_; }
    bool has_ctc() const { return heads_.ctc.ok(); }
    bool has_joint() const { return heads_.jout.ok(); }

    // Encoder (encoder.cpp:97-167).  mel [B][n_mels][T_max] f32 device,
    // valid_T host (true mel frames per item, nullptr = T_max).  out [B][T'][D]
    // f32 device; valid_out host [B].  stage_masks selects the batched
    // subsampling masking (subsampling.cpp:109-147) or the scalar one.
    int encoder_forward(const float* mel, int B, int T_max, const int* valid_T, bool stage_masks,
                        float* out, int* valid_out, float* capture, hipStream_t s);
    // whole_frames: every one of valid_T[b] mel frames is audio (a streaming
    // window), instead of the offline T-1 convention
    int subsampling_forward(const float* mel, int B, int T_max, const int* valid_T,
                            bool stage_masks, float* out, int* valid_out, hipStream_t s,
                            bool apply_xscaling = false, bool whole_frames = false);
    // pos: the caller's positional table [2T-1][D] f32 (device), or null for
    // rel_pos_encoding(T, D) computed here
    void conformer_layer_forward(int layer, const float* x, int B, int T, const int* valid, const float* pos,
                                 float* out, float* conv_out, hipStream_t s);
    void relpos_attention_forward(int layer, const float* x, int B, int T, const int* valid, const float* pos,
                                  float* out, hipStream_t s);
    void conv_module_forward(int layer, const float* c, int B, int T, const int* valid, float* out,
                             hipStream_t s);
    void ctc_forward(const float* enc, int64_t M, float* logprobs, int32_t* argmax, hipStream_t s);
    void tdt_joint_argmax(const float* enc, int64_t M, const float* g, float* logits, int32_t* tok,
                          int32_t* dur, hipStream_t s);
    // The same products on caller-provided device scratch (allocates nothing):
    // pp [joint_hidden] and hid [M][joint_hidden] f32, both fully written before
    // they are read.
    void tdt_joint_argmax_in(const float* enc, int64_t M, const float* g, float* logits, int32_t* tok,
                             int32_t* dur, float* pp, float* hid, hipStream_t s);
    int joint_hidden() const { return heads_.jout.ok() ? heads_.jenc.N : 0; }
    bool has_decoder() const { return pred_.ok() && heads_.jout.ok(); }
    // transducer_greedy_batch (transducer_batch.cpp:24-213): greedy TDT
    // (n_dur > 0, skip = durations[argmax]) or RNNT decode of B utterances in
    // lockstep rounds; enc [B][T_max][d_model] f32 device, T_valid host.
    // Outputs (host) per item b: counts[b] tokens in ids/frames/conf/span[b*cap ...].
    void transducer_greedy(const float* enc, int B, int T_max, const int* T_valid, const int32_t* durations,
                           int n_dur, int blank_id, int max_symbols, int cap, int32_t* ids, int32_t* frames,
                           float* conf, int32_t* span, int* counts, hipStream_t s);
    // Cache-aware streaming encoder (streaming_encoder.cpp) for models with a
    // streaming configuration: n_streams streams advanced together, windows of
    // at most max_window mel frames.
    std::unique_ptr<StreamState> stream_create(int n_streams, int max_window, hipStream_t s);
    void stream_reset(StreamState& st, hipStream_t s);
    // Frames a window of n mel frames yields before the valid slice (0: none).
    int stream_chunk_len(const StreamState& st, int n) const;
    // StreamingEncoder::step (streaming_encoder.cpp:340-462) for every stream:
    // mel [B][n_mels][n] f32 device (pre-encode overlap included); out
    // [B][stream_chunk_len][D] f32 device receives all chunk frames; returns
    // the number kept (valid_out_len mid-stream, all when is_last).
    int stream_step(StreamState& st, const float* mel, int n, bool is_last, float* out, hipStream_t s);
    void set_profiling(unsigned family_mask, int stride);
    void profile_read(double* ms_per_family, int64_t* launches_per_family);

private:
    struct Ws;
    void* dalloc(size_t bytes);
    float* upload_f32(const HostTensor& t);
    float* upload_f32(const std::vector<float>& v);
    DevWeight make_weight(const HostTensor& t, int N, int K, bool f16_gemm);
    DevWeight make_weight_rows(const std::vector<const HostTensor*>& parts, int K, bool f16_gemm,
                               bool glu_interleave);
    const HostTensor* find(const std::string& n) const;
    const HostTensor& need(const std::string& n) const;
    void ensure_ws(int B, int T_max);
    // pointwise_conv1 + GLU + pad mask + depthwise conv + bias + folded BN + SiLU
    // of the conv module, from the normed input A [M][D] to Y [M][D]
    // (fold: A = x * gamma with the row statistics of gemm_resid_ln)
    void conv_front(const LayerDev& L, const void* A, int64_t M, const int* valid, int B, int T, void* Y,
                    hipStream_t s, bool fold = false);
    void gemm(const DevWeight& w, int epi, const void* A, int64_t lda, int64_t M,
              const float* bias, void* Y, int64_t ldy, float alpha, const int* valid, int T,
              hipStream_t s, Precision prec, int fam, const float* bias2 = nullptr, int trF = 1);
    // residual product x += alpha * (A W^T + b) that also leaves, for the
    // LayerNorm (g) that follows, x * g in f16 (h) and the row statistics
    // (res_rows: x holds the stream before a LayerNorm (res_g, res_b) whose
    // output was not stored; the product adds to that LayerNorm's output)
    void gemm_resid_ln(const DevWeight& w, const void* A, int64_t M, const float* bias, float* x, float alpha,
                       const float* g, void* h, hipStream_t s, int fam, const float* res_rows = nullptr,
                       const float* res_g = nullptr, const float* res_b = nullptr);
    // split-K workspace for residual products of few rows (M <= 512), made on
    // first use; launch_gemm decides whether to split
    void splitk_ws(GemmParams& p, hipStream_t s);
    // product of a LayerNorm folded in (A = x * gamma from gemm_resid_ln)
    GemmParams fold_params(const DevWeight& w, const void* A, int64_t M, const float* c1, const float* c2,
                           void* Y, int64_t ldy);
    int stage_lengths(int B, int T_max, const int* valid_T, int* valid_out, hipStream_t s, bool whole_frames);
    void subsampling_kernels(const float* mel, int B, int T_max, bool stage_masks, float* out, hipStream_t s,
                             bool apply_xscaling);
    // conv.3 -> conv.5 -> conv.6 -> flatten as one kernel (launch_sub_tail):
    // f16 mode, 256 channels, 128 mel bins, symmetric padding, f16 pointwise weights
    bool sub_tail_fused() const;
    void encoder_kernels(const float* mel, int B, int T_max, int T3, bool stage_masks, float* out, float* capture,
                         hipStream_t s);
    void layer_body(int l, float* x, int B, int T, const int* d_valid, bool first_ln_done,
                    bool fuse_next_ln, bool pos_all, hipStream_t s);
    // positional table of T' frames in ws_->pe (act dtype): computed, or the
    // caller's f32 table cast
    void ensure_pe(int T, hipStream_t s, const float* given = nullptr);
    void att_window(AttnParams& a) const;
    void stage_valid(const std::vector<int>* v[4], hipStream_t s);
    void mark(int fam, bool begin);
    void* cast_to_act(const float* x, int64_t n, hipStream_t s);

    ModelConfig cfg_;
    Precision prec_;
    bool finalized_ = false;
    bool ln_fold_ = false;   // f16 path: norm_self_att / norm_conv / norm_feed_forward2 folded into GEMMs
    // layer_body left x before its norm_out, with that LayerNorm's per-row
    // {mean, rstd} in the workspace (the next block's FFN1 linear2 applies it)
    bool out_ln_pending_ = false;
    std::map<std::string, HostTensor> host_;
    std::vector<void*> allocs_;
    std::vector<LayerDev> layers_;
    SubDev sub_;
    DevWeight wpos_all_;   // linear_pos of all layers, [L*D][D]; layers_[l].wpos are row views
    HeadsDev heads_;
    PredDev pred_;
    std::unique_ptr<Ws> ws_;
    float* conv_capture_ = nullptr;   // conformer_layer_forward's conv-module output
    struct ProfHook;
    unsigned prof_mask_ = 0;
    int prof_stride_ = 1;        // time every stride-th launch of the selected families
    int64_t prof_seen_ = 0;
    int cur_fam_ = -1;
    std::unique_ptr<ProfHook> prof_hook_;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> prof_ev_;   // event pool, reused
    std::vector<int> prof_pending_;                             // family of pool entry i
    double prof_ms_[KF_COUNT] = {};
    int64_t prof_n_[KF_COUNT] = {};
};

// Upload one raw-layout weight (repacked for the f16 or f32 GEMM path); the
// device buffers are appended to `allocs`.
DevWeight build_weight(const HostTensor& t, int N, int K, bool f16_gemm, std::vector<void*>& allocs);

// Rows [row0, row0 + nrows) of a device weight, sharing its storage.
DevWeight weight_rows_view(const DevWeight& w, int row0, int nrows);

// y[M][N] = x[M][K] . W^T (+ bias) for one raw weight, f32 in/out; the weight
// is uploaded for this call and freed after the stream drains.  residual:
// y += alpha (x . W^T + bias) instead (the encoder's residual product, with
// its split-K path for few rows).
void linear_raw(Precision prec, const HostTensor& t, int N, int K, const float* bias, const float* x,
                int64_t M, float* y, hipStream_t s, bool residual = false, float alpha = 1.0f);

// GGUF v3 reader: fills a Model with the encoder (+ head) tensors and config.
std::unique_ptr<Model> load_gguf(const std::string& path, int precision);

// Every KV pair of a GGUF header in file order: type (GGUF numbering), element
// type (arrays; = type for scalars), element count, and either the packed raw
// values (numbers, bools) or the strings.
typedef std::function<void(const std::string& key, int type, int elem_type, uint64_t n, const void* raw,
                           const std::vector<std::string>* strs)>
    KvVisitor;
void read_gguf_kv(const std::string& path, const KvVisitor& visit);

// subsampling.cpp:25-46 arithmetic (all_paddings 2; 3 when causal)
int subsampled_len(int T, bool causal = false);
int valid_out_len(int T, int in_valid, bool causal = false);

}  // namespace pkx

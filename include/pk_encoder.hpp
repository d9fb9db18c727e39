// pk_encoder.hpp -- C++ host classes of parakeet.cpp's encoder path, backed by
// the gfx950 kernels behind the pkx C ABI (pkx.h).
//
// Same class names, method names, argument meaning and layouts as the
// reference's host API for this path, so the encoder calls of code written
// against it (the transcribe paths in src/model.cpp, the CLI bench, the layer
// tests) compile against this header.  Deviations, each because nothing here
// uses ggml:
//   * ModelLoader has no tensor(), ggml_ctx(), realize_weights() or
//     weights_realized() (the weights live on the device, not in a ggml
//     context); it adds load(path, precision), last_error(), handle(),
//     precision(), mel_handle() and device().
//   * The ggml graph builders (build_graph, build_graph_batched) have no
//     counterpart; their batched semantics are forward_batch() overloads.
//   * PredictionNet and Joint keep only their constructors: the reference's
//     per-step host methods (forward, step, step_logits) do not exist, since
//     transducer_greedy_batch runs every step on the device.
//   * A failing forward throws std::runtime_error (the reference asserts).
//   * Subsampling::forward takes in_valid_frames up to T (the whole window);
//     a larger count is refused (the reference would report a valid length
//     past Tout for frames the window does not have).
// Classes and their reference declarations:
//   pk::ModelLoader       src/model_loader.hpp:53-83
//   pk::ParakeetConfig    src/model_loader.hpp:27-52 (same fields and types)
//   pk::MelBatch          src/encoder.hpp:17-23
//   pk::Encoder           src/encoder.hpp:25-62
//   pk::Subsampling       src/subsampling.hpp:11-76
//   pk::ConformerLayer    src/conformer.hpp:48-110
//   pk::RelPosAttention   src/relpos_attention.hpp:31-66
//   pk::rel_pos_encoding  src/pos_enc.hpp:20
//   pk::PredictionNet, pk::Joint, pk::transducer_greedy_batch
//                         src/prediction.hpp:51-53, src/joint.hpp:29-31,
//                         src/transducer_batch.hpp:12-20
//   pk::StreamingEncoder  src/streaming_encoder.hpp:33-95
//   pk::MelFrontend       src/mel.hpp:31 (whole-clip front end)
//
// Errors: ModelLoader::load returns false (message in last_error() and on
// stderr), like the reference.  A failing forward throws std::runtime_error
// carrying pkx_last_error(); the reference asserts instead (src/encoder.cpp:90).
//
// Threading: one ModelLoader owns one device model and one HIP stream; the
// forward calls of every object built on it are serialised by a mutex inside
// it (the reference serialises all compute behind one global mutex,
// src/ggml_graph.cpp:35,84).  Distinct loaders run independently.
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "pkx.h"

namespace pk {

// Cache-aware streaming schedule (src/model_loader.hpp:15-26), filled for
// models whose att_context_style is not "regular".
struct StreamingCfg {
    std::vector<int32_t> chunk_size;
    std::vector<int32_t> shift_size;
    std::vector<int32_t> pre_encode_cache_size;
    int32_t cache_drop_size = 0;
    int32_t last_channel_cache_size = 0;
    int32_t valid_out_len = 0;
    int32_t drop_extra_pre_encoded = 0;
    bool present = false;
};

// The reference's ParakeetConfig, field for field (src/model_loader.hpp:27-52),
// read from the same GGUF keys with the same defaults
// (src/model_loader.cpp:99-156).
struct ParakeetConfig {
    std::string arch;
    // encoder
    uint32_t feat_in = 0, d_model = 0, n_layers = 0, n_heads = 0, ff_dim = 0, conv_kernel = 0;
    std::string conv_norm_type;
    uint32_t subsampling_factor = 0, subsampling_conv_channels = 0, pos_emb_max_len = 5000;
    bool xscaling = true;
    // cache-aware streaming / causal configuration
    int32_t att_context_left = -1, att_context_right = -1;
    std::string att_context_style = "regular";
    bool causal_downsampling = false;
    bool conv_causal = false;
    StreamingCfg streaming;
    // preprocessor
    uint32_t sample_rate = 16000, n_mels = 0, n_fft = 0, win_length = 0, hop_length = 0;
    float preemph = 0.0f, mag_power = 2.0f, log_zero_guard = 0.0f;
    std::string normalize;
    // transducer (optional)
    uint32_t pred_hidden = 0, pred_rnn_layers = 0, joint_hidden = 0;
    std::string joint_activation;
    std::vector<int32_t> tdt_durations;
    uint32_t max_symbols = 10;
    // vocab
    uint32_t vocab_size = 0, blank_id = 0;
    std::vector<std::string> tokenizer_pieces;
};

class ModelLoader {
public:
    ModelLoader();
    ~ModelLoader();
    ModelLoader(const ModelLoader&) = delete;
    ModelLoader& operator=(const ModelLoader&) = delete;

    // Read a GGUF (parakeet.* KV, verbatim NeMo tensor names) and upload the
    // encoder weights once.  precision: PKX_PREC_AUTO / _F32 / _F16.
    bool load(const std::string& path) { return load(path, PKX_PREC_AUTO); }
    bool load(const std::string& path, int precision);
    const ParakeetConfig& config() const { return cfg_; }
    const std::vector<std::string>& tokenizer_pieces() const { return cfg_.tokenizer_pieces; }
    const std::string& last_error() const { return err_; }

    pkx_model* handle() const { return model_; }
    int precision() const { return precision_; }
    // log-mel front end from the same GGUF (parakeet.preprocessor.* and
    // preprocessor.featurizer.*); null if the file has none
    pkx_mel* mel_handle() const { return mel_; }
    const std::string& mel_error() const { return mel_err_; }

    struct Device;                        // stream, staging buffers, lock
    Device& device() const { return *dev_; }

private:
    pkx_model* model_ = nullptr;
    pkx_mel* mel_ = nullptr;
    std::string mel_err_;
    ParakeetConfig cfg_;
    int precision_ = PKX_PREC_AUTO;
    std::string err_;
    std::unique_ptr<Device> dev_;
};

// A batch of clips' mel features, pre-stacked to T_max.
struct MelBatch {
    std::vector<float> data;     // [B][n_mels][T_max]: data[(b*n_mels + m)*T_max + t]
    int n_mels = 0;
    int T_max = 0;
    int B = 0;
    std::vector<int> valid_T;    // true mel frames per item, size B (<= T_max)
};

class Encoder {
public:
    explicit Encoder(const ModelLoader& ml);

    // mel [n_mels][T] -> enc_out [d_model][Tout] (channels-first).
    void forward(const std::vector<float>& mel, int n_mels, int T,
                 std::vector<float>& enc_out, int& d_model, int& Tout) const;

    // All B clips in one launch sequence; enc_outs[b] is [d_model][valid_Tout[b]].
    void forward_batch(const MelBatch& mels, std::vector<std::vector<float>>& enc_outs,
                       int& d_model, int& Tout, std::vector<int>& valid_Tout) const;

    // forward() plus the outputs of the layers listed in capture_layers, each
    // [T'][d_model], in layer_outs (parallel to capture_layers).
    void forward_capture(const std::vector<float>& mel, int n_mels, int T,
                         std::vector<float>& enc_out, int& d_model, int& Tout,
                         const std::vector<int>& capture_layers,
                         std::vector<std::vector<float>>& layer_outs) const;

private:
    const ModelLoader& ml_;
    int d_model_;
    int n_layers_;
    bool xscaling_;
};

class Subsampling {
public:
    explicit Subsampling(const ModelLoader& ml);

    // mel [n_mels][T] -> out [Tout][d_model] (scalar-path masking).
    void forward(const std::vector<float>& mel, int n_mels, int T,
                 std::vector<float>& out, int& Tout, int& d_model) const;
    void forward(const std::vector<float>& mel, int n_mels, int T,
                 std::vector<float>& out, int& Tout, int& d_model, int& valid_len) const;
    // in_valid_frames >= 0 replaces the offline T-1 entry valid length;
    // in_valid_frames == T is the whole window (the streaming chunks'
    // convention, subsampling.hpp:53-61); a count above T is refused.
    void forward(const std::vector<float>& mel, int n_mels, int T,
                 std::vector<float>& out, int& Tout, int& d_model, int& valid_len,
                 int in_valid_frames) const;

    // build_graph_batched semantics (per-stage time masks): mel [B][n_mels][T],
    // valid_in[b] is the entry valid length (< 0: T-1); out [B][Tp][d_model].
    void forward_batch(const float* mel, int n_mels, int T, int B, const std::vector<int>& valid_in,
                       std::vector<float>& out, int& Tp, std::vector<int>& valid_out) const;

    int valid_out_len(int T, int in_valid_frames = -1) const;

private:
    const ModelLoader& ml_;
    int d_model_;
};

class ConformerLayer {
public:
    ConformerLayer(const ModelLoader& ml, int layer_idx);

    // x [T][d_model]; pos_emb [pos_len = 2T-1][d_model], used as given (e.g.
    // rel_pos_encoding(T, d_model), or a table computed elsewhere in f32);
    // out [T][d_model].
    void forward(const std::vector<float>& x, int T, const std::vector<float>& pos_emb,
                 int pos_len, int valid_len, std::vector<float>& out) const;
    void forward_with_conv(const std::vector<float>& x, int T, const std::vector<float>& pos_emb,
                           int pos_len, int valid_len, std::vector<float>& out,
                           std::vector<float>& conv_out) const;
    // The conv module alone on conv_in = norm_conv(residual), [T][d_model].
    void conv_module_forward(const std::vector<float>& conv_in, int T, int valid_len,
                             std::vector<float>& out) const;
    // build_graph_batched semantics: x, out [B][T][d_model], valid_len size B.
    void forward_batch(const std::vector<float>& x, int T, int B, const std::vector<float>& pos_emb,
                       int pos_len, const std::vector<int>& valid_len, std::vector<float>& out) const;

private:
    const ModelLoader& ml_;
    int layer_idx_;
    int d_model_;
};

class RelPosAttention {
public:
    RelPosAttention(const ModelLoader& ml, int layer_idx);

    // x [T][d_model] (already normalised); pos_emb as for ConformerLayer.
    void forward(const std::vector<float>& x, int T, const std::vector<float>& pos_emb,
                 int pos_len, int valid_len, std::vector<float>& out) const;
    void forward_batch(const std::vector<float>& x, int T, int B, const std::vector<float>& pos_emb,
                       int pos_len, const std::vector<int>& valid_len, std::vector<float>& out) const;

private:
    const ModelLoader& ml_;
    int layer_idx_;
    int d_model_;
};

// pos_emb [2T-1][d_model] f32 (computed on the device in double, then f32).
void rel_pos_encoding(int T, int d_model, std::vector<float>& out);

// Per-emitted-token metadata (src/decode_types.hpp:25-30).
struct TokenInfo {
    int32_t id;
    int32_t frame;
    float conf;
    int32_t span;
};

// The prediction network (src/prediction.hpp:52-105) and joint
// (src/joint.hpp:27-80) of a loaded model.  Their weights are uploaded by the
// ModelLoader (prediction LSTM, joint enc / pred / output projections); these
// objects name them for transducer_greedy_batch, which runs every step on the
// device.  The reference's per-step host methods (forward, step, step_logits)
// have no counterpart here.
class PredictionNet {
public:
    explicit PredictionNet(const ModelLoader& ml);
    const ModelLoader& loader() const { return ml_; }

private:
    const ModelLoader& ml_;
};

class Joint {
public:
    explicit Joint(const ModelLoader& ml);
    const ModelLoader& loader() const { return ml_; }

private:
    const ModelLoader& ml_;
};

// Batched greedy transducer decode (src/transducer_batch.hpp:12-20) over the
// model's prediction network and joint, on the device.  encs[n]: row-major
// [T[n]][enc_hidden]; durations empty -> RNNT, else TDT.  Outputs per item:
// ids[n] and, if toks != nullptr, TokenInfo[n].  pred and joint must come from
// the same loader.
void transducer_greedy_batch(const PredictionNet& pred, const Joint& joint,
                             const std::vector<std::vector<float>>& encs, const std::vector<int>& T,
                             int enc_hidden, const std::vector<int32_t>& durations, int blank_id, int max_symbols,
                             std::vector<std::vector<int32_t>>& ids, std::vector<std::vector<TokenInfo>>* toks);
// The same with the loader named directly.
void transducer_greedy_batch(const ModelLoader& ml, const std::vector<std::vector<float>>& encs,
                             const std::vector<int>& T, int enc_hidden, const std::vector<int32_t>& durations,
                             int blank_id, int max_symbols, std::vector<std::vector<int32_t>>& ids,
                             std::vector<std::vector<TokenInfo>>* toks);

// Cache-aware streaming FastConformer encoder (src/streaming_encoder.hpp:33-95)
// on the device: per-layer attention and conv caches carried across chunks,
// so the concatenated chunk outputs are the offline limited-context encoder's
// frames.  One stream per object (the C ABI advances several together).
class StreamingEncoder {
public:
    explicit StreamingEncoder(const ModelLoader& ml);
    ~StreamingEncoder();
    StreamingEncoder(const StreamingEncoder&) = delete;
    StreamingEncoder& operator=(const StreamingEncoder&) = delete;

    // Zero the caches and the step counter (a fresh stream).
    void reset();
    // One mel window row-major [n_mels][n_mel_frames] (pre-encode overlap
    // included) -> the chunk's valid frames row-major [valid][d_model];
    // is_last keeps every produced frame (keep_all_outputs).
    std::vector<float> step(const std::vector<float>& mel_chunk_frames, int n_mel_frames, bool is_last,
                            int& n_valid_out);
    std::vector<float> step(const std::vector<float>& mel_chunk_frames, int n_mel_frames) {
        int v = 0;
        return step(mel_chunk_frames, n_mel_frames, false, v);
    }

    int chunk_size_first() const { return chunk_first_; }   // mel frames, step 0
    int chunk_size() const { return chunk_main_; }          // mel frames, later steps
    int pre_encode_cache_size() const { return pre_cache_; }
    int valid_out_len() const { return valid_out_len_; }
    int step_num() const;

private:
    const ModelLoader& ml_;
    pkx_streaming* st_ = nullptr;
    void* mel_dev_ = nullptr;
    void* out_dev_ = nullptr;
    int d_model_ = 0, n_mels_ = 0, max_window_ = 0;
    int chunk_first_ = 0, chunk_main_ = 0, pre_cache_ = 0, valid_out_len_ = 0;
};

// Log-mel front end (src/mel.hpp:33-41), on the device.
class MelFrontend {
public:
    explicit MelFrontend(const ModelLoader& ml);
    // samples: 16 kHz mono.  Out: feats row-major [n_mels][T] (frame-major inner = T).
    void compute(const std::vector<float>& samples, std::vector<float>& feats, int& n_mels, int& T) const;

private:
    const ModelLoader& ml_;
};

// Per-clip log-mel of a batch of 16 kHz mono clips, zero-padded and stacked to
// the longest clip (src/model.cpp:114-146): data [B][n_mels][T_max], valid_T
// each clip's frame count.  All clips in one device pass.
MelBatch build_mel_batch(const ModelLoader& ml, const std::vector<std::vector<float>>& pcms16k);

}  // namespace pk

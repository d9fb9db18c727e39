// ModelLoader / ParakeetConfig (src/model_loader.hpp:27-83): every field the
// reference's loader reads (src/model_loader.cpp:99-156) is filled from the
// GGUF with the reference's defaults.  Expected integer fields come from the
// baseline (cfg_expect, in the order listed below); the strings are the ones
// the synthetic model GGUF carries.
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE");
    if (!gguf || !base) { std::fprintf(stderr, "env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) return 1;
    std::vector<int32_t> want;
    if (!pktest::load_baseline_i32(base, "cfg_expect", want) || want.size() != 18) return 1;
    const pk::ParakeetConfig& c = ml.config();
    const uint32_t got[18] = {c.feat_in, c.d_model, c.n_layers, c.n_heads, c.ff_dim, c.conv_kernel,
                              c.subsampling_conv_channels, c.vocab_size, c.blank_id, c.pred_hidden,
                              c.pred_rnn_layers, c.joint_hidden, c.n_mels, c.n_fft, c.win_length, c.hop_length,
                              c.sample_rate, (uint32_t)c.tdt_durations.size()};
    const char* names[18] = {"feat_in", "d_model", "n_layers", "n_heads", "ff_dim", "conv_kernel",
                             "subsampling_conv_channels", "vocab_size", "blank_id", "pred_hidden",
                             "pred_rnn_layers", "joint_hidden", "n_mels", "n_fft", "win_length", "hop_length",
                             "sample_rate", "tdt_durations.size()"};
    bool ok = true;
    for (int i = 0; i < 18; ++i)
        if ((int64_t)got[i] != want[i]) {
            std::fprintf(stderr, "[loader] %s = %u, expected %d\n", names[i], got[i], want[i]);
            ok = false;
        }
    auto expect = [&](bool cond, const char* what) {
        if (!cond) std::fprintf(stderr, "[loader] %s\n", what);
        ok = ok && cond;
    };
    expect(c.arch == "hybrid_tdt_ctc", "arch");
    expect(c.conv_norm_type == "batch_norm", "conv_norm_type");
    expect(c.subsampling_factor == 8, "subsampling_factor");
    expect(c.pos_emb_max_len == 5000, "pos_emb_max_len");
    expect(c.att_context_style == "regular" && c.att_context_left == -1 && c.att_context_right == -1,
           "att_context defaults");
    expect(!c.causal_downsampling && !c.conv_causal && !c.streaming.present, "offline model: no streaming fields");
    expect(c.normalize == "per_feature", "normalize");
    expect(std::fabs(c.preemph - 0.97f) < 1e-7f && c.mag_power == 2.0f, "preemph / mag_power");
    expect(c.joint_activation == "relu" && c.max_symbols == 10, "joint activation / max_symbols");
    expect(c.tdt_durations == std::vector<int32_t>({0, 1, 2, 3, 4}), "tdt_durations");
    expect(ml.tokenizer_pieces().size() == c.vocab_size && !ml.tokenizer_pieces().empty() &&
               ml.tokenizer_pieces()[0] == "<unk>" && ml.tokenizer_pieces()[1] == "\xe2\x96\x81t1",
           "tokenizer pieces");
    std::fprintf(stderr, "[loader] d_model %u, %u layers, vocab %u, %zu pieces -> %s\n", c.d_model, c.n_layers,
                 c.vocab_size, ml.tokenizer_pieces().size(), ok ? "OK" : "FAIL");
    return ok ? 0 : 1;
}

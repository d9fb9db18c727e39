// Offline encoder parity for a cache-aware streaming model (the shape of
// tests/test_encoder_eou.cpp): causal subsampling, the LayerNorm conv norm
// with causal depthwise padding and the chunked-limited attention window, all
// in one whole-sequence Encoder::forward_capture.  Layers {0, mid, last} are
// captured and compared with enc_layer_* (per-layer rel-L2 fails the test
// here; the reference only prints them), then encoder_out [d_model][T'].
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF_EOU");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE_EOU");
    if (!gguf || !base) { std::fprintf(stderr, "eou env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) return 1;
    const pk::ParakeetConfig& c = ml.config();
    if (c.att_context_style != "chunked_limited" || !c.causal_downsampling || !c.conv_causal ||
        c.conv_norm_type != "layer_norm") {
        std::fprintf(stderr, "[encoder_eou] not a cache-aware streaming model\n");
        return 1;
    }
    const double bar = pktest::bar_for(ml.precision());

    std::vector<float> mel; std::vector<int64_t> ms;
    if (!pktest::load_baseline(base, "mel", mel, ms) || ms.size() != 2) return 1;
    const int n_mels = (int)ms[0], T = (int)ms[1];
    const int n_layers = (int)c.n_layers;
    std::vector<int> capture = {0, n_layers / 2, n_layers - 1};

    pk::Encoder enc(ml);
    std::vector<float> enc_out; int dm = 0, Tout = 0;
    std::vector<std::vector<float>> layer_outs;
    enc.forward_capture(mel, n_mels, T, enc_out, dm, Tout, capture, layer_outs);
    bool ok = true;
    const char* names[3] = {"enc_layer_0", "enc_layer_mid", "enc_layer_last"};
    for (int i = 0; i < 3; ++i) {
        std::vector<float> lref; std::vector<int64_t> ls;
        if (!pktest::load_baseline(base, names[i], lref, ls)) return 1;
        ok = pktest::compare_rel_l2(layer_outs[i], lref, names[i], bar) && ok;
    }
    std::vector<float> ref; std::vector<int64_t> rs;
    if (!pktest::load_baseline(base, "encoder_out", ref, rs)) return 1;
    if (rs.size() != 2 || (int)rs[0] != dm || (int)rs[1] != Tout) {
        std::fprintf(stderr, "[encoder_eou] encoder_out shape mismatch [%d,%d]\n", dm, Tout);
        return 1;
    }
    ok = pktest::compare(enc_out, ref, "encoder_eou", 5e-2f, 5e-2f) && ok;
    ok = pktest::compare_rel_l2(enc_out, ref, "encoder_eou", bar) && ok;
    return ok ? 0 : 1;
}

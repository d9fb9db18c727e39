// Whole-encoder parity (the shape of tests/test_encoder.cpp): the positional
// table against the baseline pos_emb, then Encoder::forward_capture on the
// baseline mel with layers {0, mid, last} captured, against enc_layer_* and
// encoder_out [d_model][T'].
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE");
    if (!gguf || !base) { std::fprintf(stderr, "env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) return 1;
    const double bar = pktest::bar_for(ml.precision());

    std::vector<float> posref; std::vector<int64_t> ps;
    if (!pktest::load_baseline(base, "pos_emb", posref, ps) || ps.size() != 2) return 1;
    const int pos_len = (int)ps[0], d_model = (int)ps[1], Tp_ref = (pos_len + 1) / 2;
    std::vector<float> poscomp;
    pk::rel_pos_encoding(Tp_ref, d_model, poscomp);
    // the reference's bar against NeMo's f32 table (tests/test_encoder.cpp:40),
    // then ours against the f64-evaluated table
    bool ok_pos = pktest::compare(poscomp, posref, "pos_emb", 1e-3f, 1e-3f);
    std::vector<float> pos64; std::vector<int64_t> p64s;
    if (!pktest::load_baseline(base, "pos_emb_f64", pos64, p64s)) return 1;
    ok_pos = pktest::compare(poscomp, pos64, "pos_emb_f64", 1e-6f, 1e-6f) && ok_pos;

    std::vector<float> mel; std::vector<int64_t> ms;
    if (!pktest::load_baseline(base, "mel", mel, ms) || ms.size() != 2) return 1;
    const int n_mels = (int)ms[0], T = (int)ms[1];
    const int n_layers = ml.config().n_layers;
    std::vector<int> capture = {0, n_layers / 2, n_layers - 1};

    pk::Encoder enc(ml);
    std::vector<float> enc_out; int dm = 0, Tout = 0;
    std::vector<std::vector<float>> layer_outs;
    enc.forward_capture(mel, n_mels, T, enc_out, dm, Tout, capture, layer_outs);
    bool ok = ok_pos;
    const char* names[3] = {"enc_layer_0", "enc_layer_mid", "enc_layer_last"};
    for (int c = 0; c < 3; ++c) {
        std::vector<float> lref; std::vector<int64_t> ls;
        if (!pktest::load_baseline(base, names[c], lref, ls)) return 1;
        ok = pktest::compare_rel_l2(layer_outs[c], lref, names[c], bar) && ok;
    }
    std::vector<float> ref; std::vector<int64_t> rs;
    if (!pktest::load_baseline(base, "encoder_out", ref, rs)) return 1;
    if (rs.size() != 2 || (int)rs[0] != dm || (int)rs[1] != Tout) {
        std::fprintf(stderr, "encoder_out shape mismatch [%d,%d]\n", dm, Tout);
        return 1;
    }
    ok = pktest::compare(enc_out, ref, "encoder", 5e-2f, 5e-2f) && ok;
    ok = pktest::compare_rel_l2(enc_out, ref, "encoder", bar) && ok;
    return ok ? 0 : 1;
}

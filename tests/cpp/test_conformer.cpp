// Conformer block parity (the shape of tests/test_conformer.cpp): baseline
// enc_pre_layers [T][d] + pos_emb, valid_len = T-1 -> ConformerLayer(0)
// forward_with_conv -> compare with enc_layer_0, and the conv-module output
// with l0_conv_out; then conv_module_forward alone on l0_conv_in.
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE");
    if (!gguf || !base) { std::fprintf(stderr, "env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) return 1;
    std::vector<float> xin, pos; std::vector<int64_t> xs, ps;
    if (!pktest::load_baseline(base, "enc_pre_layers", xin, xs) || xs.size() != 2) return 1;
    const int T = (int)xs[0], D = (int)xs[1];
    if (!pktest::load_baseline(base, "pos_emb", pos, ps) || ps.size() != 2) return 1;
    const int pos_len = (int)ps[0];
    if (pos_len != 2 * T - 1 || (int)ps[1] != D) { std::fprintf(stderr, "pos_emb shape\n"); return 1; }
    const int valid_len = T - 1;
    const double bar = pktest::bar_for(ml.precision());

    pk::ConformerLayer layer(ml, 0);
    std::vector<float> out, conv_out;
    layer.forward_with_conv(xin, T, pos, pos_len, valid_len, out, conv_out);
    bool ok = true;
    std::vector<float> cref, ref, cin, cout_ref, cm; std::vector<int64_t> s;
    if (!pktest::load_baseline(base, "l0_conv_out", cref, s)) return 1;
    ok = pktest::compare(conv_out, cref, "conformer.conv", 3e-2f, 3e-2f) && ok;
    ok = pktest::compare_rel_l2(conv_out, cref, "conformer.conv", bar) && ok;
    if (!pktest::load_baseline(base, "enc_layer_0", ref, s)) return 1;
    ok = pktest::compare(out, ref, "conformer", 3e-2f, 3e-2f) && ok;
    ok = pktest::compare_rel_l2(out, ref, "conformer", bar) && ok;

    if (!pktest::load_baseline(base, "l0_conv_in", cin, s) || !pktest::load_baseline(base, "l0_conv_module_out", cout_ref, s))
        return 1;
    layer.conv_module_forward(cin, T, valid_len, cm);
    ok = pktest::compare_rel_l2(cm, cout_ref, "conv_module", bar) && ok;
    return ok ? 0 : 1;
}

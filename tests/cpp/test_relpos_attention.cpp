// Relative-position attention parity (the shape of tests/test_relpos_attention.cpp):
// baseline l0_attn_in [T][d] + pos_emb [2T-1][d], valid_len = T-1 ->
// compare with l0_attn_out.
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE");
    if (!gguf || !base) { std::fprintf(stderr, "env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) return 1;
    std::vector<float> x, pos, ref; std::vector<int64_t> xs, ps, rs;
    if (!pktest::load_baseline(base, "l0_attn_in", x, xs) || xs.size() != 2) return 1;
    const int T = (int)xs[0], D = (int)xs[1];
    if (!pktest::load_baseline(base, "pos_emb", pos, ps) || ps.size() != 2) return 1;
    const int pos_len = (int)ps[0];
    if (pos_len != 2 * T - 1 || (int)ps[1] != D) { std::fprintf(stderr, "pos_emb shape\n"); return 1; }
    const int valid_len = T - 1;   // last frame is padding

    pk::RelPosAttention attn(ml, 0);
    std::vector<float> out;
    attn.forward(x, T, pos, pos_len, valid_len, out);
    if (!pktest::load_baseline(base, "l0_attn_out", ref, rs)) return 1;
    bool ok = pktest::compare(out, ref, "relpos_attention", 2e-2f, 2e-2f);
    ok = pktest::compare_rel_l2(out, ref, "relpos_attention", pktest::bar_for(ml.precision())) && ok;

    // a table other than rel_pos_encoding(T, d) is refused, not silently replaced
    std::vector<float> bad = pos;
    bad[1] += 0.5f;
    bool refused = false;
    try { attn.forward(x, T, bad, pos_len, valid_len, out); } catch (const std::invalid_argument&) { refused = true; }
    if (!refused) { std::fprintf(stderr, "non-standard pos_emb accepted\n"); ok = false; }
    return ok ? 0 : 1;
}

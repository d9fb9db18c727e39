// Batched conformer-block invariants (the shape of tests/test_conformer_batch.cpp):
// case A: B=2 copies at full length == the single-item forward;
// case B: valid lengths {T, T/2} == the per-item forwards.
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE");
    if (!gguf || !base) { std::fprintf(stderr, "env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) return 1;
    std::vector<float> x, pe; std::vector<int64_t> xs, ps;
    if (!pktest::load_baseline(base, "l0_attn_in", x, xs) || xs.size() != 2) return 1;
    const int T = (int)xs[0], D = (int)xs[1];
    if (!pktest::load_baseline(base, "pos_emb", pe, ps)) return 1;
    const int pos_len = (int)ps[0];
    pk::ConformerLayer layer(ml, 0);
    std::vector<float> xb((size_t)2 * T * D);
    for (int b = 0; b < 2; ++b) std::copy(x.begin(), x.end(), xb.begin() + (size_t)b * T * D);
    auto item = [&](const std::vector<float>& out, int b) {
        return std::vector<float>(out.begin() + (size_t)b * T * D, out.begin() + (size_t)(b + 1) * T * D);
    };
    bool ok = true;
    {
        std::vector<float> ref, out;
        layer.forward(x, T, pe, pos_len, T, ref);
        layer.forward_batch(xb, T, 2, pe, pos_len, {T, T}, out);
        ok = pktest::compare(item(out, 0), ref, "caseA_item0", 1e-3f, 1e-3f) && ok;
        ok = pktest::compare(item(out, 1), ref, "caseA_item1", 1e-3f, 1e-3f) && ok;
    }
    {
        const int v0 = T, v1 = T / 2;
        std::vector<float> ref0, ref1, out;
        layer.forward(x, T, pe, pos_len, v0, ref0);
        layer.forward(x, T, pe, pos_len, v1, ref1);
        layer.forward_batch(xb, T, 2, pe, pos_len, {v0, v1}, out);
        ok = pktest::compare(item(out, 0), ref0, "caseB_item0", 1e-3f, 1e-3f) && ok;
        ok = pktest::compare(item(out, 1), ref1, "caseB_item1", 1e-3f, 1e-3f) && ok;
    }
    return ok ? 0 : 1;
}

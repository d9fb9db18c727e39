// Subsampling parity (the shape of the reference's tests/test_subsampling.cpp):
// baseline mel [n_mels][T] -> pk::Subsampling::forward (scalar path) ->
// compare with baseline subsampling_out [T'][d_model].
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE");
    if (!gguf || !base) { std::fprintf(stderr, "env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) return 1;

    std::vector<float> mel; std::vector<int64_t> ms;
    if (!pktest::load_baseline(base, "mel", mel, ms) || ms.size() != 2) return 1;
    const int n_mels = (int)ms[0], T = (int)ms[1];

    pk::Subsampling sub(ml);
    std::vector<float> out; int Tout = 0, dm = 0, valid = 0;
    sub.forward(mel, n_mels, T, out, Tout, dm, valid);
    if (valid != sub.valid_out_len(T)) { std::fprintf(stderr, "valid %d != %d\n", valid, sub.valid_out_len(T)); return 1; }

    std::vector<float> ref; std::vector<int64_t> rs;
    if (!pktest::load_baseline(base, "subsampling_out", ref, rs)) return 1;
    if (rs.size() != 2 || (int)rs[0] != Tout || (int)rs[1] != dm) {
        std::fprintf(stderr, "shape mismatch got=[%d,%d]\n", Tout, dm);
        return 1;
    }
    bool ok = pktest::compare(out, ref, "subsampling", 1e-2f, 1e-2f);
    ok = pktest::compare_rel_l2(out, ref, "subsampling", pktest::bar_for(ml.precision())) && ok;
    return ok ? 0 : 1;
}

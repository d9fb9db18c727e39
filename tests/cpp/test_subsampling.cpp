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

    // Streaming convention: the whole window is audio (in_valid_frames = T),
    // so every output frame is valid (src/subsampling.hpp:53-61).
    std::vector<float> refw; std::vector<int64_t> rws;
    std::vector<int32_t> vw;
    if (!pktest::load_baseline(base, "subsampling_out_whole", refw, rws)) return 1;
    if (!pktest::load_baseline_i32(base, "subsampling_valid_whole", vw) || vw.size() != 1) return 1;
    std::vector<float> outw; int Toutw = 0, dmw = 0, validw = 0;
    sub.forward(mel, n_mels, T, outw, Toutw, dmw, validw, T);
    if (validw != (int)vw[0] || validw != sub.valid_out_len(T, T) || Toutw != Tout) {
        std::fprintf(stderr, "whole window: valid %d (baseline %d, valid_out_len %d), Tout %d\n", validw, (int)vw[0],
                     sub.valid_out_len(T, T), Toutw);
        return 1;
    }
    ok = pktest::compare_rel_l2(outw, refw, "subsampling (whole window)", pktest::bar_for(ml.precision())) && ok;
    // a count past the window is refused
    bool threw = false;
    try {
        sub.forward(mel, n_mels, T, outw, Toutw, dmw, validw, T + 1);
    } catch (const std::exception&) {
        threw = true;
    }
    if (!threw) { std::fprintf(stderr, "in_valid_frames = T + 1 was accepted\n"); return 1; }
    return ok ? 0 : 1;
}

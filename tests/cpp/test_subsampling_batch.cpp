// Batched subsampling (the shape of tests/test_subsampling_batch.cpp): a B=2
// batch {full clip, its first half zero-padded} through the per-stage-masked
// batched path must reproduce each clip's standalone result on its valid
// frames (the half clip's last frame excluded: the stage masks differ from the
// scalar path there).
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
    const int n_mels = (int)ms[0], T0 = (int)ms[1], T1 = T0 / 2;

    pk::Subsampling sub(ml);
    std::vector<float> r0, r1; int Tout0 = 0, Tout1 = 0, dm = 0, vl0 = 0, vl1 = 0;
    sub.forward(mel, n_mels, T0, r0, Tout0, dm, vl0);
    std::vector<float> mel1((size_t)n_mels * T1);
    for (int m = 0; m < n_mels; ++m)
        for (int t = 0; t < T1; ++t) mel1[(size_t)m * T1 + t] = mel[(size_t)m * T0 + t];
    sub.forward(mel1, n_mels, T1, r1, Tout1, dm, vl1);

    const int B = 2, Tmax = T0;
    std::vector<float> stacked((size_t)B * n_mels * Tmax, 0.0f);
    for (int m = 0; m < n_mels; ++m) {
        for (int t = 0; t < T0; ++t) stacked[(size_t)m * Tmax + t] = mel[(size_t)m * T0 + t];
        for (int t = 0; t < T1; ++t) stacked[((size_t)n_mels + m) * Tmax + t] = mel1[(size_t)m * T1 + t];
    }
    std::vector<float> outflat; int Tp = 0; std::vector<int> vout;
    sub.forward_batch(stacked.data(), n_mels, Tmax, B, {T0 - 1, T1 - 1}, outflat, Tp, vout);
    std::fprintf(stderr, "[subbatch] Tp=%d dm=%d Tout0=%d Tout1=%d valid_out={%d,%d}\n", Tp, dm, Tout0, Tout1,
                 vout[0], vout[1]);
    if (vout[0] != vl0 || vout[1] != vl1) { std::fprintf(stderr, "valid_out mismatch\n"); return 1; }
    auto slice = [&](int b, int Tv) {
        std::vector<float> s((size_t)Tv * dm);
        for (int t = 0; t < Tv; ++t)
            for (int c = 0; c < dm; ++c) s[(size_t)t * dm + c] = outflat[((size_t)b * Tp + t) * dm + c];
        return s;
    };
    bool a = pktest::compare(slice(0, Tout0), r0, "subbatch.item0", 1e-3f, 1e-3f);
    const int Tcmp = Tout1 > 1 ? Tout1 - 1 : Tout1;
    std::vector<float> r1i(r1.begin(), r1.begin() + (size_t)Tcmp * dm);
    bool b = pktest::compare(slice(1, Tcmp), r1i, "subbatch.item1", 5e-3f, 5e-3f);
    return (a && b) ? 0 : 1;
}

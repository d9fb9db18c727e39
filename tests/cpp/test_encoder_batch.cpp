// Batched encoder equivalence and padding invariance (the shape of
// tests/test_encoder_batch.cpp): a ragged B=2 batch {full mel, its first 3/4
// zero-padded} through forward_batch must match each clip's standalone
// forward on the item's valid frames; outputs are compacted per item to
// [d_model][valid_Tout[b]].
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE");
    if (!gguf || !base) { std::fprintf(stderr, "env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) { std::fprintf(stderr, "model load failed\n"); return 1; }
    std::vector<float> mel; std::vector<int64_t> ms;
    if (!pktest::load_baseline(base, "mel", mel, ms) || ms.size() != 2) return 1;
    const int n_mels = (int)ms[0], T0 = (int)ms[1], T1 = (T0 * 3) / 4;

    pk::Encoder enc(ml);
    std::vector<float> e0, e1; int dm = 0, to0 = 0, to1 = 0;
    enc.forward(mel, n_mels, T0, e0, dm, to0);
    std::vector<float> mel1((size_t)n_mels * T1);
    for (int m = 0; m < n_mels; ++m)
        for (int t = 0; t < T1; ++t) mel1[(size_t)m * T1 + t] = mel[(size_t)m * T0 + t];
    enc.forward(mel1, n_mels, T1, e1, dm, to1);

    pk::MelBatch mb;
    mb.B = 2; mb.n_mels = n_mels; mb.T_max = T0; mb.valid_T = {T0, T1};
    mb.data.assign((size_t)2 * n_mels * T0, 0.0f);
    for (int m = 0; m < n_mels; ++m) {
        for (int t = 0; t < T0; ++t) mb.data[(size_t)m * T0 + t] = mel[(size_t)m * T0 + t];
        for (int t = 0; t < T1; ++t) mb.data[((size_t)n_mels + m) * T0 + t] = mel1[(size_t)m * T1 + t];
    }
    std::vector<std::vector<float>> eo; int dmb = 0, tob = 0; std::vector<int> vt;
    enc.forward_batch(mb, eo, dmb, tob, vt);
    std::fprintf(stderr, "[encbatch] dm=%d to0=%d to1=%d | dmb=%d tob=%d vt={%d,%d}\n", dm, to0, to1, dmb, tob,
                 vt[0], vt[1]);
    if (dmb != dm || tob != to0 || eo.size() != 2 || vt[0] < 1 || vt[0] > tob || vt[1] < 1 || vt[1] > to1) return 1;
    auto cols = [&](const std::vector<float>& full, int Tfull, int Tv) {
        std::vector<float> s((size_t)dm * Tv);
        for (int c = 0; c < dm; ++c)
            for (int t = 0; t < Tv; ++t) s[(size_t)c * Tv + t] = full[(size_t)c * Tfull + t];
        return s;
    };
    bool a = pktest::compare(cols(eo[0], vt[0], vt[0]), cols(e0, to0, vt[0]), "encbatch.item0", 5e-2f, 5e-2f);
    bool b = pktest::compare(cols(eo[1], vt[1], vt[1]), cols(e1, to1, vt[1]), "encbatch.item1", 5e-2f, 5e-2f);
    return (a && b) ? 0 : 1;
}

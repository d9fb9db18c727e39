// Log-mel front end through the host classes (the shape of the reference's
// tests/test_mel.cpp): pk::MelFrontend::compute on the baseline's "pcm" (a
// speech fixture) against the baseline "mel" [n_mels][T], then
// build_mel_batch of {pcm, its first 60 %} against each clip alone.
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE");
    if (!gguf || !base) { std::fprintf(stderr, "env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) return 1;
    std::vector<float> pcm, ref; std::vector<int64_t> ps, rs;
    if (!pktest::load_baseline(base, "pcm", pcm, ps) || !pktest::load_baseline(base, "mel_pcm", ref, rs)) return 1;
    pk::MelFrontend mel(ml);
    std::vector<float> feats; int n_mels = 0, T = 0;
    mel.compute(pcm, feats, n_mels, T);
    std::fprintf(stderr, "[mel] samples=%zu n_mels=%d T=%d (baseline %lld x %lld)\n", pcm.size(), n_mels, T,
                 (long long)rs[0], (long long)rs[1]);
    if (rs.size() != 2 || n_mels != rs[0] || T != rs[1]) return 1;
    bool ok = pktest::compare(feats, ref, "mel", 1e-4f, 1e-4f);

    std::vector<float> part(pcm.begin(), pcm.begin() + (long)(pcm.size() * 6 / 10));
    std::vector<float> fp; int np_ = 0, Tp = 0;
    mel.compute(part, fp, np_, Tp);
    pk::MelBatch mb = pk::build_mel_batch(ml, {pcm, part});
    std::fprintf(stderr, "[mel] batch B=%d T_max=%d valid={%d,%d}\n", mb.B, mb.T_max, mb.valid_T[0], mb.valid_T[1]);
    if (mb.B != 2 || mb.T_max != T || mb.valid_T[0] != T || mb.valid_T[1] != Tp || mb.n_mels != n_mels) return 1;
    std::vector<float> b0((size_t)n_mels * T), b1((size_t)n_mels * Tp);
    bool pad_zero = true;
    for (int m = 0; m < n_mels; ++m) {
        for (int t = 0; t < T; ++t) b0[(size_t)m * T + t] = mb.data[(size_t)m * T + t];
        for (int t = 0; t < T; ++t) {
            const float v = mb.data[((size_t)n_mels + m) * T + t];
            if (t < Tp) b1[(size_t)m * Tp + t] = v;
            else pad_zero = pad_zero && v == 0.0f;
        }
    }
    ok = pktest::compare(b0, feats, "mel_batch.item0", 0.0f, 0.0f) && ok;
    ok = pktest::compare(b1, fp, "mel_batch.item1", 0.0f, 0.0f) && ok;
    if (!pad_zero) std::fprintf(stderr, "[mel] padding not zero\n");
    return (ok && pad_zero) ? 0 : 1;
}

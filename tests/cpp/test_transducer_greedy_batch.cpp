// Batched greedy TDT decode through the host classes (the shape of the
// reference's tests/test_transducer_greedy_batch.cpp): a ragged batch of
// encoder outputs decoded together must give each item's tokens as decoded
// alone, and both must equal the baseline ids / frames / spans.
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE");
    if (!gguf || !base) { std::fprintf(stderr, "env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) return 1;
    std::vector<float> enc; std::vector<int64_t> es;
    std::vector<int32_t> Tb, durs;
    if (!pktest::load_baseline(base, "dec_enc", enc, es) || !pktest::load_baseline_i32(base, "dec_T", Tb) ||
        !pktest::load_baseline_i32(base, "dec_durations", durs) || es.size() != 3) return 1;
    const int N = (int)es[0], T_max = (int)es[1], D = (int)es[2];
    std::vector<std::vector<float>> encs(N);
    std::vector<int> T(N);
    for (int n = 0; n < N; ++n) {
        T[n] = Tb[n];
        encs[n].assign(enc.begin() + (size_t)n * T_max * D, enc.begin() + (size_t)n * T_max * D + (size_t)T[n] * D);
    }
    const int blank = (int)ml.config().blank_id;
    // the reference's call shape: prediction net and joint of the loaded model
    pk::PredictionNet pred(ml);
    pk::Joint joint(ml);
    std::vector<std::vector<int32_t>> ids;
    std::vector<std::vector<pk::TokenInfo>> toks;
    pk::transducer_greedy_batch(pred, joint, encs, T, D, durs, blank, (int)ml.config().max_symbols, ids, &toks);
    bool ok = true;
    for (int n = 0; n < N; ++n) {
        std::vector<int32_t> ref_ids, ref_fr, ref_sp;
        const std::string s = std::to_string(n);
        if (!pktest::load_baseline_i32(base, "dec_ids_" + s, ref_ids) ||
            !pktest::load_baseline_i32(base, "dec_frames_" + s, ref_fr) ||
            !pktest::load_baseline_i32(base, "dec_spans_" + s, ref_sp)) return 1;
        std::vector<std::vector<int32_t>> one;
        std::vector<std::vector<pk::TokenInfo>> one_t;
        pk::transducer_greedy_batch(ml, {encs[n]}, {T[n]}, D, durs, blank, 10, one, &one_t);
        bool same = ids[n] == ref_ids && one[0] == ids[n] && toks[n].size() == ref_ids.size();
        for (size_t i = 0; same && i < toks[n].size(); ++i)
            same = toks[n][i].frame == ref_fr[i] && toks[n][i].span == ref_sp[i] && toks[n][i].id == ref_ids[i] &&
                   one_t[0][i].frame == ref_fr[i];
        std::fprintf(stderr, "[decbatch] item %d T=%d tokens=%zu (baseline %zu, alone %zu) -> %s\n", n, T[n],
                     ids[n].size(), ref_ids.size(), one[0].size(), same ? "OK" : "FAIL");
        ok = ok && same;
    }
    return ok ? 0 : 1;
}

// Cache-aware streaming encoder parity (the shape of tests/test_streaming_encoder.cpp):
// pk::StreamingEncoder driven through the model's own chunk schedule (first
// window chunk_size_first frames, later ones pre_encode_cache_size frames of
// overlap + chunk_size), the concatenated valid frames against the baseline
// stream_encoder_out [d_model][T'] and, over the leading frames (the final
// chunk's tail excluded), against the offline encoder_out [d_model][T'].
#include "parity.hpp"
#include "pk_encoder.hpp"

#include <algorithm>
#include <cstdlib>

int main() {
    const char* gguf = std::getenv("PARAKEET_TEST_GGUF_EOU");
    const char* base = std::getenv("PARAKEET_TEST_BASELINE_EOU");
    const char* bstream = std::getenv("PARAKEET_TEST_BASELINE_EOU_STREAM");
    if (!gguf || !base || !bstream) { std::fprintf(stderr, "eou stream env not set; skip\n"); return 77; }
    pk::ModelLoader ml;
    if (!ml.load(gguf)) { std::fprintf(stderr, "[stream] load failed: %s\n", ml.last_error().c_str()); return 1; }
    if (!ml.config().streaming.present) { std::fprintf(stderr, "[stream] not a streaming model\n"); return 1; }
    const double bar = pktest::bar_for(ml.precision());

    std::vector<float> mel; std::vector<int64_t> ms;
    if (!pktest::load_baseline(base, "mel", mel, ms) || ms.size() != 2) return 1;
    const int n_mels = (int)ms[0], T = (int)ms[1], D = ml.config().d_model;

    pk::StreamingEncoder enc(ml);
    auto window = [&](int lo, int hi) {
        std::vector<float> w((size_t)n_mels * (hi - lo));
        for (int m = 0; m < n_mels; ++m)
            for (int t = lo; t < hi; ++t) w[(size_t)m * (hi - lo) + (t - lo)] = mel[(size_t)m * T + t];
        return w;
    };
    std::vector<float> stream_out;
    int idx = 0, n_chunks = 0;
    bool first = true;
    while (idx < T) {
        const int size = first ? enc.chunk_size_first() : enc.chunk_size();
        const int hi = std::min(idx + size, T);
        const int lo = first ? idx : std::max(0, idx - enc.pre_encode_cache_size());
        const bool last = hi >= T;
        int valid = 0;
        std::vector<float> e = enc.step(window(lo, hi), hi - lo, last, valid);
        stream_out.insert(stream_out.end(), e.begin(), e.end());
        ++n_chunks;
        idx += size;
        first = false;
    }
    const int Tout = (int)(stream_out.size() / D);
    std::fprintf(stderr, "[stream] chunks=%d T'=%d step_num=%d\n", n_chunks, Tout, enc.step_num());
    bool ok = enc.step_num() == n_chunks;

    auto transpose = [&](const std::vector<float>& cf, int Tn) {   // [D][Tn] -> [Tn][D]
        std::vector<float> r((size_t)Tn * D);
        for (int c = 0; c < D; ++c)
            for (int t = 0; t < Tn; ++t) r[(size_t)t * D + c] = cf[(size_t)c * Tn + t];
        return r;
    };
    std::vector<float> sref; std::vector<int64_t> ss;
    if (!pktest::load_baseline(bstream, "stream_encoder_out", sref, ss) || ss.size() != 2 || ss[0] != D) return 1;
    if ((int)ss[1] != Tout) { std::fprintf(stderr, "[stream] T' %d vs %d\n", Tout, (int)ss[1]); return 1; }
    ok = pktest::compare_rel_l2(stream_out, transpose(sref, Tout), "streaming_encoder.vsStream", bar) && ok;

    std::vector<float> oref; std::vector<int64_t> os;
    if (!pktest::load_baseline(base, "encoder_out", oref, os) || os.size() != 2 || os[0] != D) return 1;
    const int lead = std::min(Tout, (int)os[1]) - enc.valid_out_len();
    std::vector<float> off = transpose(oref, (int)os[1]);
    std::vector<float> got(stream_out.begin(), stream_out.begin() + (size_t)lead * D);
    off.resize((size_t)lead * D);
    ok = pktest::compare_rel_l2(got, off, "streaming_encoder.vsOffline", bar) && ok;

    // reset() starts the same stream again
    enc.reset();
    int v0 = 0;
    std::vector<float> again = enc.step(window(0, std::min(enc.chunk_size_first(), T)),
                                        std::min(enc.chunk_size_first(), T), false, v0);
    ok = ok && v0 > 0 && std::equal(again.begin(), again.end(), stream_out.begin());
    std::fprintf(stderr, "[stream] reset replay -> %s\n", ok ? "OK" : "FAIL");
    return ok ? 0 : 1;
}

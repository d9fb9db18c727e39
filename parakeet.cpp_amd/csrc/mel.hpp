// Log-mel front end on the device: pk::MelFrontend::compute for a batch of
// clips (src/mel.cpp:99-185, src/fft.cpp) stacked like build_mel_batch
// (src/model.cpp:114-146).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

namespace pkx {

// parakeet.preprocessor.* (src/model_loader.cpp:133-141)
struct MelConfig {
    int n_fft = 512, win_length = 400, hop = 160, n_mels = 128;
    int per_feature = 1;               // normalize == "per_feature"
    float preemph = 0.97f, mag_power = 2.0f, log_guard = 5.9604644775390625e-8f;
};

constexpr int MEL_MAX_NFFT = 512;       // LDS sizing of the FFT kernel
constexpr int MEL_FRAMES_PER_BLOCK = 8;
constexpr int MEL_FB_LDS = 2048;        // filterbank nonzeros staged in LDS (more: read from L2)

class MelFront {
public:
    // window: win_len values centre-padded to n_fft (src/mel.cpp:25-46);
    // fb: [n_mels][n_fft/2+1] row-major (preprocessor.featurizer.fb).
    MelFront(const MelConfig& c, const float* window, int win_len, const float* fb);
    ~MelFront();
    MelFront(const MelFront&) = delete;
    MelFront& operator=(const MelFront&) = delete;

    const MelConfig& config() const { return cfg_; }
    // frames of an S-sample clip (src/mel.cpp:132-135)
    int frames(int S) const;
    // pcm [B][S_stride] f32 (device), n_samples host [B] -> out [B][n_mels][T_max]
    // (device, zero-padded), T_out host [B].  Not re-entrant per handle.
    void forward(const float* pcm, int B, int64_t S_stride, const int* n_samples, float* out, int T_max,
                 int* T_out, hipStream_t s);

private:
    MelConfig cfg_;
    int n_bins_ = 0, log2n_ = 0;
    float* d_window_ = nullptr;
    float* d_fb_ = nullptr;
    double* d_tw_ = nullptr;            // twiddles, [n_fft - 1][2]
    int* d_meta_ = nullptr;             // per clip {samples, frames}
    void* d_span_ = nullptr;            // int4 [n_mels]: nonzero bins of each filter, packed offset
    float* d_fbp_ = nullptr;            // packed nonzero filter values
    int fb_nnz_ = 0;
    int meta_cap_ = 0;
    std::vector<int> meta_;
};

// Reads parakeet.preprocessor.* and preprocessor.featurizer.{window,fb}.
void load_mel_gguf(const std::string& path, MelConfig& c, std::vector<float>& window, std::vector<float>& fb);

}  // namespace pkx

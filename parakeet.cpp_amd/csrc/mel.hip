// Log-mel front end: pk::MelFrontend::compute (src/mel.cpp:99-185) on a batch
// of clips, stacked to T_max like build_mel_batch (src/model.cpp:114-146).
//
// The reference computes in f64 on the CPU: preemphasis, a radix-2 FFT whose
// twiddles advance by complex multiplication (src/fft.cpp:9-51), the power
// spectrum, the filterbank sum and the log; f32 only where it rounds (the
// windowed frame, the FFT output).  The kernels keep every one of those
// roundings and the f64 operation order (no FMA contraction in this file;
// the twiddle table is the reference's own recurrence, built on the host), so
// per-frame results match the reference's up to the libm ulp of sqrt/pow/log.
//
// mel_spec_kernel: one workgroup per (16 frames, clip); each wave runs the
// FFT of one frame at a time in LDS (complex f64), keeps the frame's power
// spectrum in LDS, then the workgroup computes the 16 x n_mels filterbank sums
// (one f64 chain per output, summed in bin order) and writes log-mel.
// mel_norm_kernel: one workgroup per (mel bin, clip): per-feature mean and
// unbiased std over the clip's first S/hop frames, normalisation, zeroing of
// the rest of the row up to T_max.
#pragma clang fp contract(off)

#include <algorithm>
#include <cmath>
#include <cstring>

#include "common.hpp"
#include "mel.hpp"

namespace pkx {

struct MelParams {
    const float* pcm;
    int64_t S_stride;
    const int* meta;           // [B][2]: samples, frames
    const float* window;       // [n_fft]
    const float* fb;           // [n_mels][n_bins]
    const double* tw;          // [n_fft - 1][2]: stage of half-length h uses rows h-1 .. 2h-2
    const int4* span;          // [n_mels]: the filter's nonzero bins [x, y), packed offset z
    const float* fb_packed;    // the filters' values over their spans, back to back
    int fb_nnz;
    float* out;                // [B][n_mels][T_max]
    int T_max, n_fft, log2n, hop, n_mels, n_bins, per_feature;
    float preemph, mag_power, log_guard;
};

__global__ __launch_bounds__(256) void mel_spec_kernel(MelParams p) {
    constexpr int FB = MEL_FRAMES_PER_BLOCK, RPL = MEL_MAX_NFFT / 64;
    __shared__ double2 buf[4][MEL_MAX_NFFT];
    __shared__ double pw[FB][MEL_MAX_NFFT / 2 + 1];
    __shared__ double2 tws[MEL_MAX_NFFT];
    __shared__ float fbs[MEL_FB_LDS];
    const int b = blockIdx.y, t0 = blockIdx.x * FB;
    const int S = p.meta[2 * b], T = p.meta[2 * b + 1];
    if (t0 >= T) return;                               // uniform over the workgroup
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int N = p.n_fft, pad = N / 2;
    const float* x = p.pcm + (int64_t)b * p.S_stride;
    const double pre = (double)p.preemph;

    // every frame's windowed samples (src/mel.cpp:67-69) are loaded up front,
    // one global-memory round trip for the workgroup; twiddles and the
    // filterbank's nonzero values go to LDS
    float fr[FB / 4][RPL];
#pragma unroll
    for (int r = 0; r < FB / 4; ++r) {
        const int t = t0 + 4 * r + w;
#pragma unroll
        for (int ii = 0; ii < RPL; ++ii) {
            const int i = lane + 64 * ii;
            const int q = t * p.hop + i - pad;         // sample index of padded[t*hop + i]
            double v = 0.0;
            if (i < N && t < T && q >= 0 && q < S) {
                v = (double)x[q];
                if (p.preemph > 0.0f && q > 0) v = (double)x[q] - pre * (double)x[q - 1];
            }
            fr[r][ii] = i < N ? (float)(v * (double)p.window[i]) : 0.0f;
        }
    }
    for (int i = tid; i < N - 1; i += 256) tws[i] = make_double2(p.tw[2 * i], p.tw[2 * i + 1]);
    const bool fb_lds = p.fb_nnz <= MEL_FB_LDS;
    if (fb_lds)
        for (int i = tid; i < p.fb_nnz; i += 256) fbs[i] = p.fb_packed[i];

    for (int r = 0; r < FB / 4; ++r) {
        const int f = 4 * r + w;
        double2* B2 = buf[w];
        // the frame in bit-reversed order (src/fft.cpp:14-22)
#pragma unroll
        for (int ii = 0; ii < RPL; ++ii) {
            const int i = lane + 64 * ii;
            if (i < N) B2[(int)(__brev((unsigned)i) >> (32 - p.log2n))] = make_double2((double)fr[r][ii], 0.0);
        }
        __syncthreads();
        // butterfly stages (src/fft.cpp:25-50)
        for (int s = 0, h = 1; s < p.log2n; ++s, h <<= 1) {
            for (int bi = lane; bi < N / 2; bi += 64) {
                const int k = bi & (h - 1), u = ((bi >> s) << (s + 1)) + k, v = u + h;
                const double2 tw = tws[h - 1 + k];
                const double2 a = B2[u], c = B2[v];
                const double tr = tw.x * c.x - tw.y * c.y;
                const double ti = tw.x * c.y + tw.y * c.x;
                B2[v] = make_double2(a.x - tr, a.y - ti);
                B2[u] = make_double2(a.x + tr, a.y + ti);
            }
            __syncthreads();
        }
        // power spectrum (src/mel.cpp:73-79): bins rounded to f32 first (fft.cpp:70-71)
        for (int k = lane; k < p.n_bins; k += 64) {
            const float re = (float)B2[k].x, im = (float)B2[k].y;
            const double mag = sqrt((double)re * re + (double)im * im);
            pw[f][k] = p.mag_power == 1.0f ? mag : pow(mag, (double)p.mag_power);
        }
        __syncthreads();
    }
    // filterbank + log (src/mel.cpp:82-89), one f64 chain per output summed
    // in bin order over the filter's nonzero span only: every other bin would
    // add fb * power = +-0, which leaves the sum unchanged, so the result is
    // the reference's dense sum bit for bit.  Output (m, f) with f fastest.
    const int f = tid & (FB - 1), t = t0 + f;
    for (int m = tid / FB; m < p.n_mels; m += 256 / FB) {
        const int4 sp = p.span[m];                     // {first bin, end bin, packed offset, -}
        double acc = 0.0;
        if (fb_lds) {
            for (int k = sp.x; k < sp.y; ++k) acc += (double)fbs[sp.z + k - sp.x] * pw[f][k];
        } else {
            for (int k = sp.x; k < sp.y; ++k) acc += (double)p.fb_packed[sp.z + k - sp.x] * pw[f][k];
        }
        if (t < T) p.out[((int64_t)b * p.n_mels + m) * p.T_max + t] = (float)log(acc + (double)p.log_guard);
    }
}

__device__ __forceinline__ double block_sum_f64(double v, double* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(256) void mel_norm_kernel(MelParams p) {
    __shared__ double red[4];
    const int m = blockIdx.x, b = blockIdx.y;
    const int S = p.meta[2 * b], T = p.meta[2 * b + 1];
    float* row = p.out + ((int64_t)b * p.n_mels + m) * p.T_max;
    int keep = T;
    if (p.per_feature && T > 0) {
        // src/mel.cpp:157-182: mean and unbiased std over the first S/hop frames
        const int valid = min(S / p.hop, T);
        double s = 0.0;
        for (int t = threadIdx.x; t < valid; t += 256) s += (double)row[t];
        const double mean = valid > 0 ? block_sum_f64(s, red) / (double)valid : 0.0;
        double q = 0.0;
        for (int t = threadIdx.x; t < valid; t += 256) {
            const double d = (double)row[t] - mean;
            q += d * d;
        }
        const double ss = block_sum_f64(q, red);
        const double var = valid > 1 ? ss / (double)(valid - 1) : 0.0;
        const double sd = sqrt(var) + 1e-5;
        for (int t = threadIdx.x; t < valid; t += 256) row[t] = (float)(((double)row[t] - mean) / sd);
        keep = valid;
    }
    for (int t = keep + threadIdx.x; t < p.T_max; t += 256) row[t] = 0.0f;
}

MelFront::MelFront(const MelConfig& c, const float* window, int win_len, const float* fb) : cfg_(c) {
    require(c.n_fft >= 64 && c.n_fft <= MEL_MAX_NFFT && (c.n_fft & (c.n_fft - 1)) == 0,
            "mel: n_fft must be a power of two in [64, 512]");
    require(c.hop > 0 && c.n_mels > 0 && c.mag_power > 0.0f, "mel: hop, n_mels and mag_power must be positive");
    require(window && win_len > 0 && win_len <= c.n_fft, "mel: window of 1..n_fft values required");
    require(fb != nullptr, "mel: filterbank required");
    n_bins_ = c.n_fft / 2 + 1;
    log2n_ = 0;
    while ((1 << log2n_) < c.n_fft) ++log2n_;
    // window centre-padded to n_fft (src/mel.cpp:31-46)
    std::vector<float> wpad((size_t)c.n_fft, 0.0f);
    if (win_len == c.n_fft) {
        std::memcpy(wpad.data(), window, sizeof(float) * (size_t)c.n_fft);
    } else {
        const int left = (c.n_fft - win_len) / 2;
        for (int i = 0; i < win_len && left + i < c.n_fft; ++i)
            if (left + i >= 0) wpad[(size_t)(left + i)] = window[i];
    }
    // the twiddles each butterfly of src/fft.cpp:28-48 uses: w_0 = 1,
    // w_{k+1} = w_k * (cos a, sin a), a = -2 pi / len, same f64 operations
    std::vector<double> tw((size_t)(c.n_fft - 1) * 2);
    for (int len = 2; len <= c.n_fft; len <<= 1) {
        const double ang = -2.0 * M_PI / len, wr = std::cos(ang), wi = std::sin(ang);
        double cr = 1.0, ci = 0.0;
        for (int k = 0; k < len / 2; ++k) {
            tw[2 * (size_t)(len / 2 - 1 + k)] = cr;
            tw[2 * (size_t)(len / 2 - 1 + k) + 1] = ci;
            const double nr = cr * wr - ci * wi, ni = cr * wi + ci * wr;
            cr = nr;
            ci = ni;
        }
    }
    // each filter's nonzero span and its values packed back to back (the
    // kernel skips the exact zeros outside the span)
    std::vector<int4> span((size_t)c.n_mels);
    std::vector<float> packed;
    for (int m = 0; m < c.n_mels; ++m) {
        int lo = n_bins_, hi = 0;
        for (int k = 0; k < n_bins_; ++k)
            if (fb[(size_t)m * n_bins_ + k] != 0.0f) {
                lo = std::min(lo, k);
                hi = k + 1;
            }
        if (lo >= hi) lo = hi = 0;
        span[(size_t)m] = make_int4(lo, hi, (int)packed.size(), 0);
        for (int k = lo; k < hi; ++k) packed.push_back(fb[(size_t)m * n_bins_ + k]);
    }
    fb_nnz_ = (int)packed.size();
    PKX_HIP(hipMalloc(&d_span_, sizeof(int4) * span.size()));
    PKX_HIP(hipMemcpy(d_span_, span.data(), sizeof(int4) * span.size(), hipMemcpyHostToDevice));
    PKX_HIP(hipMalloc(&d_fbp_, sizeof(float) * std::max<size_t>(packed.size(), 1)));
    if (!packed.empty())
        PKX_HIP(hipMemcpy(d_fbp_, packed.data(), sizeof(float) * packed.size(), hipMemcpyHostToDevice));
    PKX_HIP(hipMalloc(&d_window_, sizeof(float) * (size_t)c.n_fft));
    PKX_HIP(hipMalloc(&d_fb_, sizeof(float) * (size_t)c.n_mels * n_bins_));
    PKX_HIP(hipMalloc(&d_tw_, sizeof(double) * tw.size()));
    PKX_HIP(hipMemcpy(d_window_, wpad.data(), sizeof(float) * wpad.size(), hipMemcpyHostToDevice));
    PKX_HIP(hipMemcpy(d_fb_, fb, sizeof(float) * (size_t)c.n_mels * n_bins_, hipMemcpyHostToDevice));
    PKX_HIP(hipMemcpy(d_tw_, tw.data(), sizeof(double) * tw.size(), hipMemcpyHostToDevice));
}

MelFront::~MelFront() {
    for (void* q : {(void*)d_window_, (void*)d_fb_, (void*)d_tw_, (void*)d_meta_, d_span_, (void*)d_fbp_})
        if (q) (void)hipFree(q);
}

int MelFront::frames(int S) const {
    if (S <= 0) return 0;
    const int padded = S + 2 * (cfg_.n_fft / 2);
    return padded >= cfg_.n_fft ? 1 + (padded - cfg_.n_fft) / cfg_.hop : 0;
}

void MelFront::forward(const float* pcm, int B, int64_t S_stride, const int* n_samples, float* out, int T_max,
                       int* T_out, hipStream_t s) {
    require(B > 0 && T_max >= 0 && n_samples && T_out && out, "mel: bad batch arguments");
    require(B <= 65535, "mel: at most 65535 clips per call");
    meta_.assign((size_t)2 * B, 0);
    for (int b = 0; b < B; ++b) {
        require(n_samples[b] >= 0 && n_samples[b] <= S_stride, "mel: clip length outside [0, S_stride]");
        const int T = frames(n_samples[b]);
        require(T <= T_max, "mel: T_max smaller than a clip's frame count");
        meta_[2 * (size_t)b] = n_samples[b];
        meta_[2 * (size_t)b + 1] = T;
        T_out[b] = T;
    }
    require(pcm != nullptr || S_stride == 0 || *std::max_element(n_samples, n_samples + B) == 0,
            "mel: null pcm");
    if (T_max == 0) return;
    if (meta_cap_ < 2 * B) {
        if (d_meta_) PKX_HIP(hipFree(d_meta_));
        d_meta_ = nullptr;
        PKX_HIP(hipMalloc(&d_meta_, sizeof(int) * (size_t)2 * B));
        meta_cap_ = 2 * B;
    }
    PKX_HIP(hipMemcpyAsync(d_meta_, meta_.data(), sizeof(int) * (size_t)2 * B, hipMemcpyHostToDevice, s));
    MelParams p{};
    p.pcm = pcm;
    p.S_stride = S_stride;
    p.meta = d_meta_;
    p.window = d_window_;
    p.fb = d_fb_;
    p.tw = d_tw_;
    p.span = (const int4*)d_span_;
    p.fb_packed = d_fbp_;
    p.fb_nnz = fb_nnz_;
    p.out = out;
    p.T_max = T_max;
    p.n_fft = cfg_.n_fft;
    p.log2n = log2n_;
    p.hop = cfg_.hop;
    p.n_mels = cfg_.n_mels;
    p.n_bins = n_bins_;
    p.per_feature = cfg_.per_feature;
    p.preemph = cfg_.preemph;
    p.mag_power = cfg_.mag_power;
    p.log_guard = cfg_.log_guard;
    launch(mel_spec_kernel, dim3(cdiv(T_max, MEL_FRAMES_PER_BLOCK), B), dim3(256), 0, s, p);
    PKX_LAUNCH_CHECK();
    launch(mel_norm_kernel, dim3(cfg_.n_mels, B), dim3(256), 0, s, p);
    PKX_LAUNCH_CHECK();
    // the host copy of meta_ is reused by the next call: finish the upload first
    PKX_HIP(hipStreamSynchronize(s));
}

}  // namespace pkx

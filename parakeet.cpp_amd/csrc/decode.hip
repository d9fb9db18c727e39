// Greedy transducer decode on the device: transducer_greedy_batch
// (src/transducer_batch.cpp:24-213) with the prediction net of
// src/prediction.cpp:118-178 and the joint of src/joint.cpp:37-63,106-143.
//
// All B items advance in lockstep rounds.  One round:
//   per LSTM layer l: z = [x_l | h_l] . [W_ih | W_hh]^T + (b_ih + b_hh)   (f32 GEMM)
//                     lstm_cell_kernel: c' = s(f) c + s(i) tanh(g), h' = s(o) tanh(c')
//   pp = W_pred g + b_pred                                                (f32 GEMM)
//   joint_relu_kernel: f = ReLU(enc_proj[t_b] + pp)
//   logits = W_out f + b_out                                              (f32 GEMM)
//   greedy_rule_kernel: argmaxes, the TDT / RNNT rule of the per-item loops,
//                       token records, state commit on emit.
// Every round recomputes the LSTM for all items: from an unchanged committed
// state it reproduces the same g bit for bit (the reference's g_valid cache
// skips that recomputation, with the same result).  The host launches rounds
// in chunks and reads the active flags between chunks; rounds after the last
// item finished change nothing (the rule kernel returns for inactive items).
//
// Device state (ws): X_l [B][2H] holds [x_l | committed h_l] for layer l
// (x_0 = embedding of the last token, zeros before the first emission; x_l =
// this round's h'_{l-1}), so a commit writes straight into the next round's
// GEMM operand.
#include <cmath>
#include <vector>

#include "common.hpp"
#include "gemm.hpp"
#include "model.hpp"

namespace pkx {

struct DecState {
    int* t;          // current frame
    int* active;     // 1 while t < T
    int* sym;        // symbols emitted at the current frame
    int* count;      // tokens emitted
    int* overflow;   // a token did not fit in cap
    const int* T;    // frames per item
};

__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + expf(-x)); }   // ggml_sigmoid

// z [B][4H] -> out_h/out_c [B][H]; h' also into the next layer's x (or g)
__global__ void lstm_cell_kernel(const float* z, const float* c_in, float* out_h, float* out_c, float* x_next,
                                 int ld_next, int B, int H) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)B * H) return;
    const int b = (int)(i / H), j = (int)(i - (int64_t)b * H);
    const float* zr = z + (int64_t)b * 4 * H;
    const float zi = zr[j], zf = zr[H + j], zg = zr[2 * H + j], zo = zr[3 * H + j];
    const float c = sigmoid_ref(zf) * c_in[i] + sigmoid_ref(zi) * tanhf(zg);
    const float h = sigmoid_ref(zo) * tanhf(c);
    out_c[i] = c;
    out_h[i] = h;
    x_next[(int64_t)b * ld_next + j] = h;
}

// f[b][:] = ReLU(enc_proj[b][clamp(t_b)][:] + pp[b][:])
__global__ void joint_relu_kernel(const float* ep, int T_max, const float* pp, float* f, DecState st, int B, int Hj) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)B * Hj) return;
    const int b = (int)(i / Hj), h = (int)(i - (int64_t)b * Hj);
    int t = st.t[b];
    const int T = st.T[b];
    t = t > T - 1 ? T - 1 : t;   // inactive / boundary items (their logits are not used)
    t = t < 0 ? 0 : t;
    const float s = ep[((int64_t)b * T_max + t) * Hj + h] + pp[i];
    f[i] = s > 0.f ? s : 0.f;
}

__device__ __forceinline__ void argmax_first(float& v, int& k) {
    // wave-wide max with the lowest index among equal values (decode_common.hpp:5-9)
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int ok = __shfl_xor(k, o, 64);
        if (ov > v || (ov == v && ok < k)) {
            v = ov;
            k = ok;
        }
    }
}

struct RuleArgs {
    const float* logits;   // [B][Vp]
    int Vp, n_tok, n_dur, blank, max_symbols, cap, B, H, L;
    const int32_t* durations;
    const float* embed;    // [V1][H]
    float* X[4];           // [B][2H] per layer
    float* cc[4];          // committed c, [B][H]
    const float* oh[4];    // this round's h', [B][H]
    const float* oc[4];    // this round's c', [B][H]
    int32_t *ids, *frames, *spans;
    float* confs;
};

// one wave per item: the per-item rule of transducer_batch.cpp:128-205
__global__ __launch_bounds__(256) void greedy_rule_kernel(RuleArgs a, DecState st) {
    const int lane = threadIdx.x & 63, b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= a.B || !st.active[b]) return;
    const float* lz = a.logits + (int64_t)b * a.Vp;
    float v = -INFINITY;
    int k = 0x7fffffff;
    for (int i = lane; i < a.n_tok; i += 64)
        if (lz[i] > v || (lz[i] == v && i < k)) {
            v = lz[i];
            k = i;
        }
    argmax_first(v, k);
    int dk = 0;
    if (a.n_dur > 0) {
        float dv = -INFINITY;
        int di = 0x7fffffff;
        for (int i = lane; i < a.n_dur; i += 64)
            if (lz[a.n_tok + i] > dv || (lz[a.n_tok + i] == dv && i < di)) {
                dv = lz[a.n_tok + i];
                di = i;
            }
        argmax_first(dv, di);
        dk = di < a.n_dur ? di : 0;   // no value above -inf (NaN logits): index 0, as the scalar loop
    }
    if (k >= a.n_tok) k = 0;
    const bool emit = k != a.blank;
    // max_prob confidence of the emitted token (decode_common.hpp:12-20), f64
    double den = 0.0;
    if (emit) {
        for (int i = lane; i < a.n_tok; i += 64) den += exp((double)lz[i] - (double)v);
        for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
    }
    const int t0 = st.t[b];
    if (emit) {
        // commit: the step's (h', c') become the item's state; the token's
        // embedding is the next step's layer-0 input
        for (int l = 0; l < a.L; ++l)
            for (int j = lane; j < a.H; j += 64) {
                a.X[l][(int64_t)b * 2 * a.H + a.H + j] = a.oh[l][(int64_t)b * a.H + j];
                a.cc[l][(int64_t)b * a.H + j] = a.oc[l][(int64_t)b * a.H + j];
            }
        for (int j = lane; j < a.H; j += 64) a.X[0][(int64_t)b * 2 * a.H + j] = a.embed[(int64_t)k * a.H + j];
    }
    if (lane != 0) return;
    int t = t0, sym = st.sym[b];
    if (a.n_dur > 0) {
        const int skip = a.durations[dk];
        if (emit) {
            const int n = st.count[b];
            if (n < a.cap) {
                const double p = 1.0 / den, N = (double)a.n_tok;   // exp(v - v) / den
                a.ids[(int64_t)b * a.cap + n] = k;
                a.frames[(int64_t)b * a.cap + n] = t;
                a.confs[(int64_t)b * a.cap + n] = (float)((N * p - 1.0) / (N - 1.0));
                a.spans[(int64_t)b * a.cap + n] = skip;
                st.count[b] = n + 1;
            } else {
                *st.overflow = 1;
            }
        }
        sym += 1;
        t += skip;
        if (!(skip == 0 && sym < a.max_symbols)) {
            if (sym == a.max_symbols) t += 1;
            sym = 0;
        }
    } else if (!emit) {
        t += 1;
        sym = 0;
    } else {
        const int n = st.count[b];
        if (n < a.cap) {
            const double p = 1.0 / den, N = (double)a.n_tok;
            a.ids[(int64_t)b * a.cap + n] = k;
            a.frames[(int64_t)b * a.cap + n] = t;
            a.confs[(int64_t)b * a.cap + n] = (float)((N * p - 1.0) / (N - 1.0));
            a.spans[(int64_t)b * a.cap + n] = 1;
            st.count[b] = n + 1;
        } else {
            *st.overflow = 1;
        }
        sym += 1;
        if (sym >= a.max_symbols) {
            t += 1;
            sym = 0;
        }
    }
    st.t[b] = t;
    st.sym[b] = sym;
    st.active[b] = t < st.T[b] ? 1 : 0;
}

namespace {
struct DecBufs {
    std::vector<void*> p;
    ~DecBufs() {
        for (void* q : p) (void)hipFree(q);
    }
    template <typename T> T* get(size_t n) {
        void* q = nullptr;
        PKX_HIP(hipMalloc(&q, n * sizeof(T) + 16));
        p.push_back(q);
        return (T*)q;
    }
};
}  // namespace

void Model::transducer_greedy(const float* enc, int B, int T_max, const int* T_valid, const int32_t* durations,
                              int n_dur, int blank_id, int max_symbols, int cap, int32_t* ids, int32_t* frames,
                              float* conf, int32_t* span, int* counts, hipStream_t s) {
    require(finalized_ && has_decoder(), "model has no prediction network + joint");
    require(B >= 1 && T_max >= 1 && T_valid && counts && cap >= 1 && max_symbols >= 1, "decode: bad arguments");
    const int H = pred_.H, L = pred_.L, Hj = heads_.jenc.N, D = cfg_.d_model;
    const int Vp = heads_.jout.N;
    require(n_dur == heads_.n_dur, "decode: durations do not match the joint's duration outputs");
    const int n_tok = Vp - n_dur;
    require(blank_id >= 0 && blank_id < n_tok && blank_id < pred_.V1, "decode: blank_id outside the token range");
    require(n_tok <= pred_.V1, "decode: joint tokens exceed the embedding rows");
    for (int b = 0; b < B; ++b) require(T_valid[b] >= 0 && T_valid[b] <= T_max, "decode: T_valid outside [0, T_max]");
    for (int i = 0; i < n_dur; ++i) require(durations && durations[i] >= 0, "decode: durations must be >= 0");

    DecBufs m;
    float* ep = m.get<float>((size_t)B * T_max * Hj);
    float* X[4] = {};
    float *cc[4] = {}, *oh[4] = {}, *oc[4] = {};
    for (int l = 0; l < L; ++l) {
        X[l] = m.get<float>((size_t)B * 2 * H);
        cc[l] = m.get<float>((size_t)B * H);
        oh[l] = m.get<float>((size_t)B * H);
        oc[l] = m.get<float>((size_t)B * H);
        PKX_HIP(hipMemsetAsync(X[l], 0, sizeof(float) * B * 2 * H, s));   // SOS input, zero state
        PKX_HIP(hipMemsetAsync(cc[l], 0, sizeof(float) * B * H, s));
    }
    float* z = m.get<float>((size_t)B * 4 * H);
    float* g = m.get<float>((size_t)B * H);
    float* pp = m.get<float>((size_t)B * Hj);
    float* f = m.get<float>((size_t)B * Hj);
    float* lg = m.get<float>((size_t)B * Vp);
    int* ints = m.get<int>((size_t)6 * B + 1);
    int32_t* d_dur = m.get<int32_t>((size_t)(n_dur > 0 ? n_dur : 1));
    int32_t* d_ids = m.get<int32_t>((size_t)B * cap);
    int32_t* d_fr = m.get<int32_t>((size_t)B * cap);
    int32_t* d_sp = m.get<int32_t>((size_t)B * cap);
    float* d_cf = m.get<float>((size_t)B * cap);

    std::vector<int> h((size_t)6 * B + 1, 0);
    for (int b = 0; b < B; ++b) {
        h[(size_t)B + b] = T_valid[b] > 0 ? 1 : 0;   // active
        h[(size_t)5 * B + b] = T_valid[b];           // T
    }
    PKX_HIP(hipMemcpyAsync(ints, h.data(), sizeof(int) * h.size(), hipMemcpyHostToDevice, s));
    if (n_dur > 0) PKX_HIP(hipMemcpyAsync(d_dur, durations, sizeof(int32_t) * n_dur, hipMemcpyHostToDevice, s));
    // ints: t [0, B), active [B, 2B), sym [2B, 3B), count [3B, 4B), T [5B, 6B), overflow 6B
    DecState st{ints, ints + B, ints + 2 * B, ints + 3 * B, ints + 6 * B, ints + 5 * B};

    // enc_proj over every frame of every item (joint.cpp:37-63)
    gemm(heads_.jenc, EPI_STORE_F32, enc, D, (int64_t)B * T_max, heads_.jenc_b, ep, Hj, 1.f, nullptr, 1, s,
         PREC_F32, -1);

    RuleArgs ra{};
    ra.logits = lg;
    ra.Vp = Vp;
    ra.n_tok = n_tok;
    ra.n_dur = n_dur;
    ra.blank = blank_id;
    ra.max_symbols = max_symbols;
    ra.cap = cap;
    ra.B = B;
    ra.H = H;
    ra.L = L;
    ra.durations = d_dur;
    ra.embed = pred_.embed;
    for (int l = 0; l < L; ++l) {
        ra.X[l] = X[l];
        ra.cc[l] = cc[l];
        ra.oh[l] = oh[l];
        ra.oc[l] = oc[l];
    }
    ra.ids = d_ids;
    ra.frames = d_fr;
    ra.spans = d_sp;
    ra.confs = d_cf;

    auto round = [&]() {
        for (int l = 0; l < L; ++l) {
            gemm(pred_.wcat[l], EPI_STORE_F32, X[l], 2 * H, B, pred_.bsum[l], z, 4 * H, 1.f, nullptr, 1, s,
                 PREC_F32, -1);
            float* xn = l + 1 < L ? X[l + 1] : g;
            launch(lstm_cell_kernel, dim3(cdiv((int64_t)B * H, 256)), dim3(256), 0, s, (const float*)z,
                   (const float*)cc[l], oh[l], oc[l], xn, l + 1 < L ? 2 * H : H, B, H);
            PKX_LAUNCH_CHECK();
        }
        gemm(heads_.jpred, EPI_STORE_F32, g, H, B, heads_.jpred_b, pp, Hj, 1.f, nullptr, 1, s, PREC_F32, -1);
        launch(joint_relu_kernel, dim3(cdiv((int64_t)B * Hj, 256)), dim3(256), 0, s, (const float*)ep, T_max,
               (const float*)pp, f, st, B, Hj);
        PKX_LAUNCH_CHECK();
        gemm(heads_.jout, EPI_STORE_F32, f, Hj, B, heads_.jout_b, lg, Vp, 1.f, nullptr, 1, s, PREC_F32, -1);
        launch(greedy_rule_kernel, dim3(cdiv(B, 4)), dim3(256), 0, s, ra, st);
        PKX_LAUNCH_CHECK();
    };

    // every round emits a token or advances a frame; at most max_symbols
    // tokens per frame: (max_symbols + 1) rounds per frame bound the loop
    const int64_t max_rounds = (int64_t)T_max * (max_symbols + 1) + 1;
    constexpr int CHUNK = 8;
    std::vector<int> act((size_t)B);
    int64_t rounds = 0;
    for (;;) {
        for (int r = 0; r < CHUNK; ++r) round();
        rounds += CHUNK;
        PKX_HIP(hipMemcpyAsync(act.data(), ints + B, sizeof(int) * B, hipMemcpyDeviceToHost, s));
        PKX_HIP(hipStreamSynchronize(s));
        bool any = false;
        for (int b = 0; b < B; ++b) any = any || act[b];
        if (!any) break;
        require(rounds <= max_rounds, "decode: round bound exceeded");
    }
    int ovf = 0;
    PKX_HIP(hipMemcpyAsync(counts, ints + 3 * B, sizeof(int) * B, hipMemcpyDeviceToHost, s));
    PKX_HIP(hipMemcpyAsync(&ovf, st.overflow, sizeof(int), hipMemcpyDeviceToHost, s));
    if (ids) PKX_HIP(hipMemcpyAsync(ids, d_ids, sizeof(int32_t) * B * cap, hipMemcpyDeviceToHost, s));
    if (frames) PKX_HIP(hipMemcpyAsync(frames, d_fr, sizeof(int32_t) * B * cap, hipMemcpyDeviceToHost, s));
    if (conf) PKX_HIP(hipMemcpyAsync(conf, d_cf, sizeof(float) * B * cap, hipMemcpyDeviceToHost, s));
    if (span) PKX_HIP(hipMemcpyAsync(span, d_sp, sizeof(int32_t) * B * cap, hipMemcpyDeviceToHost, s));
    PKX_HIP(hipStreamSynchronize(s));
    require(!ovf, "decode: more tokens than cap");
}

}  // namespace pkx

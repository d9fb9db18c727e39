// Greedy transducer decode on the device: transducer_greedy_batch
// (src/transducer_batch.cpp:24-213) with the prediction net of
// src/prediction.cpp:118-178 and the joint of src/joint.cpp:37-63,106-143.
//
// All B items advance in lockstep rounds; one round is L + 3 launches:
//   lstm layer l (dec_mv_kernel<MV_LSTM>): z = [x_l | h_l] . [W_ih | W_hh]^T
//       + (b_ih + b_hh) for the 4 gate rows of each hidden unit, then the
//       cell c' = s(f) c + s(i) tanh(g), h' = s(o) tanh(c') in the same kernel
//   joint (dec_mv_kernel<MV_JOINT>): f = ReLU(enc_proj[t_b] + W_pred g + b_pred)
//   logits (dec_mv_kernel<MV_PLAIN>): W_out f + b_out
//   greedy_rule_kernel: argmaxes, the TDT / RNNT rule of the per-item loops,
//       token records, state commit on emit.
// The matvecs are weight-streaming: each workgroup owns a few output rows,
// keeps the B input vectors in LDS and reads its rows of W once per round for
// all items (f32 weights; the quantisable joint projections are dequantised
// to f32 at load).  Every round recomputes the LSTM for all items: from an
// unchanged committed state it reproduces the same g bit for bit (the
// reference's g_valid cache skips that recomputation, with the same result).
// The host launches rounds in chunks and reads the active flags between
// chunks; rounds after the last item finished change nothing.
//
// Device state: X_l [B][2H] holds [x_l | committed h_l] for layer l (x_0 =
// embedding of the last token, zeros before the first emission; x_l = this
// round's h'_{l-1}), so a commit writes straight into the next round's input.
#include <algorithm>
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

enum { MV_LSTM = 0, MV_JOINT = 1, MV_PLAIN = 2 };
constexpr int MV_ITEMS = 16;   // items per LDS pass
constexpr int MV_KMAX = 8;     // K <= 256 MV_KMAX: a wave holds its whole weight rows in registers

struct MvArgs {
    const float* x;   // [B][ldx], K used
    int ldx, K, B;
    const float* W;   // [rows][K] f32
    const float* bias;
    int n_out;        // MV_LSTM: hidden units H (rows g*H + u); else output rows
    float* y;         // MV_JOINT / MV_PLAIN: [B][n_out]
    // MV_LSTM
    const float* c_in;
    float *out_h, *out_c, *x_next;
    int ld_next;
    // MV_JOINT
    const float* ep;
    int T_max;
};

// KS waves per output unit (MV_LSTM: the 4 gate rows of a hidden unit; else
// one row). With KS = 2 each takes every other 256-wide K slab: waves 0-3 the
// even slabs of units 4 bx + w, waves 4-7 the odd slabs of the same units, and
// the odd half's sums are added to the even half's through LDS (even + odd,
// one fixed order). Lanes stride a slab in float4; the items' inputs come
// from LDS.
template <int MODE, int KS>
__global__ __launch_bounds__(256 * KS) void dec_mv_kernel(MvArgs a, DecState st) {
    static_assert(KS == 1 || KS == 2, "one or two waves per unit");
    constexpr int G = MODE == MV_LSTM ? 4 : 1;
    constexpr int KH = MV_KMAX / KS;   // slabs per wave
    constexpr int NT = 256 * KS;
    extern __shared__ float xs[];   // [MV_ITEMS][K]
    __shared__ float zodd[4][MV_ITEMS][G];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int uw = w & 3, kh = w >> 2;
    const int u = blockIdx.x * 4 + uw;   // this wave's unit / row
    // the wave's half of the weight rows, all loads in flight at once, kept for
    // every item pass (rows past n_out read as zero)
    float4v wv[KH][G];
#pragma unroll
    for (int kj = 0; kj < KH; ++kj) {
        const int k = 4 * lane + 256 * (KS * kj + kh);
#pragma unroll
        for (int g = 0; g < G; ++g)
            wv[kj][g] = (u < a.n_out && k < a.K)
                            ? *(const float4v*)(a.W + (int64_t)(MODE == MV_LSTM ? g * a.n_out + u : u) * a.K + k)
                            : float4v{0.f, 0.f, 0.f, 0.f};
    }
    for (int m0 = 0; m0 < a.B; m0 += MV_ITEMS) {
        const int mc = min(MV_ITEMS, a.B - m0);
        // the epilogue's operands for item m0 + lane, loaded ahead of the
        // staging so that their latency overlaps it
        const bool epi = kh == 0 && u < a.n_out && lane < mc;
        const int b = m0 + lane;
        float pb[G], pc = 0.f;
#pragma unroll
        for (int g = 0; g < G; ++g) pb[g] = epi ? a.bias[g * a.n_out + u] : 0.f;
        if constexpr (MODE == MV_LSTM) {
            if (epi) pc = a.c_in[(int64_t)b * a.n_out + u];
        } else if constexpr (MODE == MV_JOINT) {
            if (epi) {
                int t = st.t[b];
                const int T = st.T[b];
                t = t > T - 1 ? T - 1 : t;   // inactive / boundary items (their logits are not used)
                t = t < 0 ? 0 : t;
                pc = a.ep[((int64_t)b * a.T_max + t) * a.n_out + u];
            }
        }
        __syncthreads();
        // the items' inputs into LDS, twelve 16-byte loads in flight per thread
        // (16 items at K <= 1536 in one round)
        const int n4 = mc * (a.K / 4);
        for (int i0 = threadIdx.x; i0 < n4; i0 += NT * 12) {
            float4v v[12];
#pragma unroll
            for (int j = 0; j < 12; ++j) {
                const int i = i0 + NT * j;
                if (i < n4) {
                    const int m = i / (a.K / 4), k4 = i - m * (a.K / 4);
                    v[j] = *(const float4v*)(a.x + (int64_t)(m0 + m) * a.ldx + 4 * k4);
                }
            }
#pragma unroll
            for (int j = 0; j < 12; ++j) {
                const int i = i0 + NT * j;
                if (i < n4) {
                    const int m = i / (a.K / 4), k4 = i - m * (a.K / 4);
                    *(float4v*)(xs + m * a.K + 4 * k4) = v[j];
                }
            }
        }
        __syncthreads();
        float acc[MV_ITEMS][G];
#pragma unroll
        for (int m = 0; m < MV_ITEMS; ++m)
#pragma unroll
            for (int g = 0; g < G; ++g) acc[m][g] = 0.f;
#pragma unroll
        for (int kj = 0; kj < KH; ++kj) {
            const int k = 4 * lane + 256 * (KS * kj + kh);
            if (256 * (KS * kj + kh) >= a.K) break;   // uniform over the wave
            if (k < a.K) {
#pragma unroll
                for (int m = 0; m < MV_ITEMS; ++m) {
                    if (m < mc) {
                        const float4v xv = *(const float4v*)(xs + m * a.K + k);
#pragma unroll
                        for (int g = 0; g < G; ++g)
                            acc[m][g] += (wv[kj][g][0] * xv[0] + wv[kj][g][1] * xv[1]) +
                                         (wv[kj][g][2] * xv[2] + wv[kj][g][3] * xv[3]);
                    }
                }
            }
        }
        // lane m finishes item m0 + m
        float z[G];
        if constexpr (G * MV_ITEMS == 64) {
            // recursive halving over the 64 (item, gate) sums: at each step a
            // lane keeps half of its values and adds its partner's copy of
            // them, so lane L ends with the total of value L = 4 m + g
            float t[64];
#pragma unroll
            for (int m = 0; m < MV_ITEMS; ++m)
#pragma unroll
                for (int g = 0; g < G; ++g) t[m * G + g] = acc[m][g];
#pragma unroll
            for (int step = 0; step < 6; ++step) {
                const int o = 32 >> step;
                const bool hi = (lane & o) != 0;
#pragma unroll
                for (int i = 0; i < (32 >> step); ++i) {
                    const float send = hi ? t[i] : t[i + o];
                    const float keep = hi ? t[i + o] : t[i];
                    t[i] = keep + __shfl_xor(send, o, 64);
                }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) z[g] = __shfl(t[0], (lane & (MV_ITEMS - 1)) * G + g, 64);
        } else {
            // butterfly sums: every lane ends with every item total
#pragma unroll
            for (int m = 0; m < MV_ITEMS; ++m)
#pragma unroll
                for (int g = 0; g < G; ++g)
                    for (int o = 32; o > 0; o >>= 1) acc[m][g] += __shfl_xor(acc[m][g], o, 64);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                z[g] = 0.f;
#pragma unroll
                for (int m = 0; m < MV_ITEMS; ++m)
                    if (m == lane) z[g] = acc[m][g];
            }
        }
        // the odd-slab half hands its sums to the even half (every wave reaches
        // this barrier; the next pass's staging waits behind the one above)
        if constexpr (KS == 2) {
            if (kh == 1 && lane < MV_ITEMS) {
#pragma unroll
                for (int g = 0; g < G; ++g) zodd[uw][lane][g] = z[g];
            }
            __syncthreads();
        }
        if (!epi) continue;
        if constexpr (KS == 2) {
#pragma unroll
            for (int g = 0; g < G; ++g) z[g] += zodd[uw][lane][g];
        }
        if constexpr (MODE == MV_LSTM) {
            const int H = a.n_out;
            const float zi = z[0] + pb[0], zf = z[1] + pb[1];
            const float zg = z[2] + pb[2], zo = z[3] + pb[3];
            const int64_t i = (int64_t)b * H + u;
            const float c = sigmoid_ref(zf) * pc + sigmoid_ref(zi) * tanhf(zg);
            const float h = sigmoid_ref(zo) * tanhf(c);
            a.out_c[i] = c;
            a.out_h[i] = h;
            a.x_next[(int64_t)b * a.ld_next + u] = h;
        } else if constexpr (MODE == MV_JOINT) {
            const float v = pc + (z[0] + pb[0]);
            a.y[(int64_t)b * a.n_out + u] = v > 0.f ? v : 0.f;
        } else {
            a.y[(int64_t)b * a.n_out + u] = z[0] + pb[0];
        }
    }
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

// workgroup-wide argmax (first max) over a[0, n)
__device__ __forceinline__ int block_argmax(const float* a, int n, float& vmax, float* rv, int* rk) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float v = -INFINITY;
    int k = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += 256)
        if (a[i] > v || (a[i] == v && i < k)) {
            v = a[i];
            k = i;
        }
    argmax_first(v, k);
    __syncthreads();
    if (lane == 0) {
        rv[w] = v;
        rk[w] = k;
    }
    __syncthreads();
    v = rv[0];
    k = rk[0];
    for (int j = 1; j < 4; ++j)
        if (rv[j] > v || (rv[j] == v && rk[j] < k)) {
            v = rv[j];
            k = rk[j];
        }
    vmax = v;
    return k < n ? k : 0;   // no value above -inf (NaN logits): index 0, as the scalar loop
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

// one workgroup per item: the per-item rule of transducer_batch.cpp:128-205
__global__ __launch_bounds__(256) void greedy_rule_kernel(RuleArgs a, DecState st) {
    __shared__ float rv[4];
    __shared__ int rk[4];
    __shared__ double rd[4];
    __shared__ int dur_s[32];
    const int b = blockIdx.x, tid = threadIdx.x;
    if (!st.active[b]) return;   // uniform over the workgroup
    // The item's state is read and written only by thread 0 of this workgroup:
    // its loads go out now, beside the logits', not after the commit stores.
    int t = 0, sym = 0, cnt = 0;
    if (tid == 0) {
        t = st.t[b];
        sym = st.sym[b];
        cnt = st.count[b];
    }
    if (tid < a.n_dur && tid < 32) dur_s[tid] = a.durations[tid];   // visible after block_argmax's barriers
    // this step's (h', c') rows, loaded now and stored by the commit if the item
    // emits (L <= 4, H <= 1024: at most 4 x 4 values of each per thread)
    float ph[4][4], pc[4][4];
#pragma unroll
    for (int l = 0; l < 4; ++l)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int j = tid + 256 * r;
            const bool ok = l < a.L && j < a.H;
            ph[l][r] = ok ? a.oh[l][(int64_t)b * a.H + j] : 0.f;
            pc[l][r] = ok ? a.oc[l][(int64_t)b * a.H + j] : 0.f;
        }
    const float* lz = a.logits + (int64_t)b * a.Vp;
    float v;
    const int k = block_argmax(lz, a.n_tok, v, rv, rk);
    int dk = 0;
    if (a.n_dur > 0) {
        float dv;
        dk = block_argmax(lz + a.n_tok, a.n_dur, dv, rv, rk);
    }
    const bool emit = k != a.blank;
    double den = 0.0;
    if (emit) {
        // max_prob confidence of the emitted token (decode_common.hpp:12-20), f64
        for (int i = tid; i < a.n_tok; i += 256) den += exp((double)lz[i] - (double)v);
        for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
        if ((tid & 63) == 0) rd[tid >> 6] = den;
        __syncthreads();
        den = (rd[0] + rd[1]) + (rd[2] + rd[3]);
        // commit: the step's (h', c') become the item's state; the token's
        // embedding is the next step's layer-0 input
#pragma unroll
        for (int l = 0; l < 4; ++l)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = tid + 256 * r;
                if (l < a.L && j < a.H) {
                    a.X[l][(int64_t)b * 2 * a.H + a.H + j] = ph[l][r];
                    a.cc[l][(int64_t)b * a.H + j] = pc[l][r];
                }
            }
        for (int j = tid; j < a.H; j += 256) a.X[0][(int64_t)b * 2 * a.H + j] = a.embed[(int64_t)k * a.H + j];
    }
    if (tid != 0) return;
    const int skip = a.n_dur > 0 ? (dk < 32 ? dur_s[dk] : a.durations[dk]) : 1;
    if (emit) {
        const int n = cnt;
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
    if (a.n_dur > 0) {
        // symbols_added += 1; t += skip; the frame is done unless skip == 0 and
        // symbols < max_symbols; a frame ended by max_symbols advances by 1
        sym += 1;
        t += skip;
        if (!(skip == 0 && sym < a.max_symbols)) {
            if (sym == a.max_symbols) t += 1;
            sym = 0;
        }
    } else if (!emit) {
        t += 1;   // RNNT blank: next frame
        sym = 0;
    } else if (++sym >= a.max_symbols) {
        t += 1;
        sym = 0;
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
    require(H % 4 == 0 && Hj % 4 == 0, "decode: pred_hidden and joint_hidden must be multiples of 4");
    require((size_t)MV_ITEMS * 2 * H * 4 <= 160 * 1024, "decode: pred_hidden too large for the LDS input stage");
    require(2 * H <= 256 * MV_KMAX && Hj <= 256 * MV_KMAX, "decode: pred_hidden above 1024 or joint_hidden above 2048");
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
    float* g = m.get<float>((size_t)B * H);
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

    const size_t lds_max = (size_t)MV_ITEMS * std::max(2 * H, std::max(H, Hj)) * sizeof(float);
    for (const void* fn : {(const void*)dec_mv_kernel<MV_LSTM, 2>, (const void*)dec_mv_kernel<MV_JOINT, 2>,
                           (const void*)dec_mv_kernel<MV_PLAIN, 1>})
        PKX_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_max));
    auto round = [&]() {
        for (int l = 0; l < L; ++l) {
            MvArgs a{};
            a.x = X[l];
            a.ldx = 2 * H;
            a.K = 2 * H;
            a.B = B;
            a.W = pred_.wcat[l];
            a.bias = pred_.bsum[l];
            a.n_out = H;
            a.c_in = cc[l];
            a.out_h = oh[l];
            a.out_c = oc[l];
            a.x_next = l + 1 < L ? X[l + 1] : g;
            a.ld_next = l + 1 < L ? 2 * H : H;
            launch(dec_mv_kernel<MV_LSTM, 2>, dim3(cdiv(H, 4)), dim3(512), (uint32_t)(MV_ITEMS * 2 * H * 4), s, a, st);
            PKX_LAUNCH_CHECK();
        }
        MvArgs j{};
        j.x = g;
        j.ldx = H;
        j.K = H;
        j.B = B;
        j.W = pred_.jpred;
        j.bias = heads_.jpred_b;
        j.n_out = Hj;
        j.y = f;
        j.ep = ep;
        j.T_max = T_max;
        launch(dec_mv_kernel<MV_JOINT, 2>, dim3(cdiv(Hj, 4)), dim3(512), (uint32_t)(MV_ITEMS * H * 4), s, j, st);
        PKX_LAUNCH_CHECK();
        MvArgs o{};
        o.x = f;
        o.ldx = Hj;
        o.K = Hj;
        o.B = B;
        o.W = pred_.jout;
        o.bias = heads_.jout_b;
        o.n_out = Vp;
        o.y = lg;
        launch(dec_mv_kernel<MV_PLAIN, 1>, dim3(cdiv(Vp, 4)), dim3(256), (uint32_t)(MV_ITEMS * Hj * 4), s, o, st);
        PKX_LAUNCH_CHECK();
        launch(greedy_rule_kernel, dim3(B), dim3(256), 0, s, ra, st);
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

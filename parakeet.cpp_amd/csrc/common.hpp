// Shared device/host helpers for the gfx950 encoder kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <tuple>

namespace pkx {

typedef _Float16 f16;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef int int2v __attribute__((ext_vector_type(2)));
typedef int int4v __attribute__((ext_vector_type(4)));

// ggml type ids (the GGUF weight layout)
enum GgmlType : int { GT_F32 = 0, GT_F16 = 1, GT_Q8_0 = 8, GT_Q4_K = 12 };

// Activation storage type of a compute precision mode.
enum Precision : int { PREC_F32 = 0, PREC_F16 = 1 };

struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void hip_check(hipError_t e, const char* what, const char* file, int line) {
    if (e != hipSuccess) {
        char buf[512];
        std::snprintf(buf, sizeof(buf), "%s failed: %s (%s:%d)", what, hipGetErrorString(e), file, line);
        throw HipError(buf);
    }
}
#define PKX_HIP(x) ::pkx::hip_check((x), #x, __FILE__, __LINE__)
#define PKX_LAUNCH_CHECK() ::pkx::hip_check(hipGetLastError(), "kernel launch", __FILE__, __LINE__)

// Per-launch timing.  When a hook is installed on the calling thread and it
// hands out an event pair, the launch carries those events on its own dispatch
// packet (hipExtLaunchKernel), so the elapsed time between them is the
// kernel's execution time, with no marker packets or host syncs in between.
struct LaunchHook {
    virtual bool take(hipEvent_t* start, hipEvent_t* stop) = 0;
    virtual ~LaunchHook() = default;
};
extern thread_local LaunchHook* tl_launch_hook;

template <typename... KA, typename... A>
inline void launch(void (*kernel)(KA...), dim3 grid, dim3 block, uint32_t shmem, hipStream_t s,
                   A... args) {
    static_assert(sizeof...(KA) == sizeof...(A), "kernel argument count");
    std::tuple<KA...> packed{static_cast<KA>(args)...};
    void* ptrs[sizeof...(KA) > 0 ? sizeof...(KA) : 1];
    std::apply([&](auto&... x) {
        int i = 0;
        ((ptrs[i++] = (void*)&x), ...);
    }, packed);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (tl_launch_hook && !tl_launch_hook->take(&e0, &e1)) e0 = e1 = nullptr;
    hip_check(hipExtLaunchKernel((const void*)kernel, grid, block, ptrs, shmem, s, e0, e1, 0),
              "kernel launch", __FILE__, __LINE__);
}

inline void require(bool ok, const std::string& msg) {
    if (!ok) throw std::invalid_argument(msg);
}

// v_rcp_f32 (1 ulp) instead of an IEEE division: the epilogues apply these to
// every GEMM output; exp overflow gives rcp(inf) = 0, the correct limit.
// e^-v as the bare v_exp_f32 of -v log2(e): without the denormal-range fix-up
// of __expf, whose results only differ where 1 + e^-v rounds to 1 anyway.
__device__ __forceinline__ float sigmoid_dev(float v) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f));
}
__device__ __forceinline__ float silu_dev(float v) { return v * sigmoid_dev(v); }

template <typename T> __device__ __forceinline__ T to_act(float v);
template <> __device__ __forceinline__ float to_act<float>(float v) { return v; }
template <> __device__ __forceinline__ f16 to_act<f16>(float v) { return (f16)v; }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Reductions over aligned groups of n consecutive lanes (n = 1, 2, 4, 8 or 16,
// wave-uniform), every lane of a group receiving the result: DPP steps
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror
// (each pairs a lane with one in the other half of its current group).
template <int CTRL> __device__ __forceinline__ float dpp_get(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float group_sum(float v, int n) {
    if (n > 1) v += dpp_get<0xB1>(v);    // quad_perm [1,0,3,2]
    if (n > 2) v += dpp_get<0x4E>(v);    // quad_perm [2,3,0,1]
    if (n > 4) v += dpp_get<0x141>(v);   // row_half_mirror
    if (n > 8) v += dpp_get<0x140>(v);   // row_mirror
    return v;
}
// XCD-aware block order: the hardware dispatches block b to XCD b % 8;
// xcd_tile gives each XCD a contiguous range of work positions (a bijection
// on [0, total)), so neighbouring work items share one XCD's L2.
__device__ __forceinline__ int xcd_tile(int bid, int total) {
    const int per = (int)((unsigned)total >> 3), rem = total & 7;
    const int x = bid & 7, loc = (int)((unsigned)bid >> 3);
    return x * per + (x < rem ? x : rem) + loc;
}

// x / d for 0 <= x < 2^22 and d >= 1, without the ~40-instruction integer
// division sequence: x times the reciprocal of d (v_rcp_f32, within 1 ulp)
// is within 0.75 of x / d at these sizes, so the truncated quotient is off by
// at most one either way and one remainder test corrects it.
__device__ __forceinline__ int udiv_small(int x, int d) {
    int q = (int)((float)x * __builtin_amdgcn_rcpf((float)d));
    const int r = x - q * d;
    q += (r >= d) - (r < 0);
    return q;
}

// MFMA row m of a 32-row tile <-> output column.  The 32x32 accumulator gives
// lane half q the rows 8 g + 4 q + e (register 4 g + e, e < 4); feeding row m
// from column 16 q + 4 g + e leaves column 16 q + r in register r, so each
// lane holds 16 consecutive columns.
__device__ __forceinline__ int tail_col(int m) { return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3); }

// Raw buffer resources: loads at offsets at or past num_records return zero,
// so an offset pushed to OOB (or a negative one, read as unsigned) is a
// zero fill with no branch.
constexpr uint32_t OOB = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    const int n = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, n, 0x00020000);
}
// Buffer load of 16 bytes per lane straight into LDS: lane L's data lands at
// lds + 16 L; soff is wave-uniform.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}
// s_waitcnt with only the vector-memory counter bounded (gfx9 encoding): the
// N most recent vector-memory operations of the wave may still be in flight.
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Sum over a whole wave, every lane receiving it: DPP within each row of 16
// lanes, then the four row sums read with v_readlane (no LDS round trips, as
// the ds_bpermute steps of wave_sum take).  Every lane of the wave must be
// active.
__device__ __forceinline__ float wave_sum_full(float v) {
    v = group_sum(v, 16);
    const int vi = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 48));
    return (r0 + r1) + (r2 + r3);
}

inline int cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Compute units of the current device (asked once per device, then cached).
inline int device_cu_count() {
    static std::atomic<int> cache[64];   // per device, 0 until first asked
    int dev = 0;
    PKX_HIP(hipGetDevice(&dev));
    require(dev >= 0 && dev < 64, "device index out of range");
    int cus = cache[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
        PKX_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        cache[dev].store(cus, std::memory_order_relaxed);
    }
    return cus;
}
__host__ __device__ __forceinline__ int cdiv_dev(int a, int b) { return (a + b - 1) / b; }

}  // namespace pkx

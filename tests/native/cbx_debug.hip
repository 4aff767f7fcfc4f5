// cbx_debug.hip -- test-only diagnostics (libcbx_debug.so): the device
// exponential, the device Philox uniforms and the two exact running-sum
// evaluations of the sampler, run on caller-given inputs so the tests can
// compare them with the host (tests/native/cbx_debug.h).
#include <hip/hip_runtime.h>

#include "../../chatterbox.cpp_amd/csrc/cbx_sampler_wave.h"
#include "cbx_debug.h"

namespace cbx {
namespace {

__global__ void debug_expf_kernel(const float* in, float* out, int64_t n) {
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 32) tab[threadIdx.x] = kExp2TabDev.t[threadIdx.x];
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = expf_libm_branchless(in[i], tab);
}

__global__ void debug_philox_kernel(uint64_t seed, const uint64_t* sid, uint64_t step, int32_t n,
                                    double* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = philox_uniform(seed, sid ? sid[i] : (uint64_t)i, step);
}

// One wave per case: the workgroup kernel's running sums (wave_run_sum over
// up to 8192 terms read from memory, the per-lane run length picked from n):
// sum[c] = 0 + t_0 + t_1 + ... and, for thr[c] > 0, hit[c] = the first index
// whose running sum is >= thr[c] (else -1).  desc[c] != 0: the terms do not
// increase, and the sums may stop once their adds are no-ops.
__global__ __launch_bounds__(64) void debug_runsum_kernel(const float* t, const int32_t* off,
                                                          const float* thr, const uint8_t* desc,
                                                          float* sum, int32_t* hit) {
    const int c = blockIdx.x;
    const int b = off[c], n = off[c + 1] - b;
    if (n <= 0 || n > 8192) return;
    const float th = thr ? thr[c] : 0.0f;
    auto term = [&](int i) { return t[b + i]; };
    int h = -1, unused;
    float s;
    if (desc && desc[c]) {
        s = wave_run_sum<8192, false, true>(term, n, 0.0f, 0.0f, unused, true);
        if (th > 0.0f) (void)wave_run_sum<8192, true, true>(term, n, 0.0f, th, h, true);
    } else {
        s = wave_run_sum<8192, false, false>(term, n, 0.0f, 0.0f, unused, true);
        if (th > 0.0f) (void)wave_run_sum<8192, true, false>(term, n, 0.0f, th, h, true);
    }
    if (threadIdx.x == 0) {
        sum[c] = s;
        hit[c] = h;
    }
}

// Case c: terms t[off[c] .. off[c+1]) (1..kWaveCap + 64, finite, >= 0) laid
// out as the sampler lays out its sorted exp terms (lane l holds C = the odd
// number >= n/64 consecutive terms); sum[c] by the sum the sampler uses for C,
// hit[c] the first index whose running sum is >= thr[c] (thr[c] > 0), else -1.
__global__ __launch_bounds__(64) void debug_chain_kernel(const float* t, const int32_t* off,
                                                         const float* thr, float* sum,
                                                         int32_t* hit) {
    constexpr int CM = kWaveRows + 1;
    const int c = blockIdx.x;
    const int lane = threadIdx.x;
    const int b = off[c], n = off[c + 1] - b;
    if (n <= 0 || n > 64 * CM) return;
    const int C = uni(((n + 63) >> 6) | 1);
    const int nl = uni((n + C - 1) / C);
    float tr[CM];
#pragma unroll
    for (int q = 0; q < CM; ++q) {
        const int i = lane * C + q;
        tr[q] = (q < C && i < n) ? t[b + i] : 0.0f;
    }
    const float th = thr ? thr[c] : 0.0f;
    float s = 0.0f;
    int h = -1;
    with_odd_c<1, CM>(C, [&](auto cc) {
        constexpr int CC = decltype(cc)::value;
        int unused;
        if constexpr (CC >= 7) s = chain_segments<CC>(tr, nl);
        else s = chain_sweeps<CC, false>(tr, nl, 0.0f, unused);
        if (th > 0.0f) (void)chain_sweeps<CC, true>(tr, nl, th, h);
    });
    if (lane == 0) {
        sum[c] = s;
        hit[c] = h;
    }
}

}  // namespace
}  // namespace cbx

namespace {
int launch_done(int device, hipError_t e) {
    (void)device;
    if (e != hipSuccess) return CBX_ERR_HIP;
    return CBX_OK;
}
struct DevGuard {
    int prev = -1;
    explicit DevGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DevGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};
}  // namespace

extern "C" {

int cbx_debug_expf(int32_t device, const float* in, float* out, int64_t n, void* stream) {
    if (!in || !out || n < 0) return CBX_ERR_INVALID;
    if (n == 0) return CBX_OK;
    DevGuard g(device);
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(cbx::debug_expf_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, in, out, n);
    return launch_done(device, hipGetLastError());
}

int cbx_debug_philox(int32_t device, uint64_t seed, const uint64_t* stream_ids, uint64_t step,
                     int32_t n, double* out, void* stream) {
    if (!out || n < 0) return CBX_ERR_INVALID;
    if (n == 0) return CBX_OK;
    DevGuard g(device);
    hipLaunchKernelGGL(cbx::debug_philox_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, seed, stream_ids, step, n, out);
    return launch_done(device, hipGetLastError());
}

int cbx_debug_runsum(int32_t device, const float* terms, const int32_t* offsets, const float* thr,
                     const uint8_t* desc, int32_t n_cases, float* sum, int32_t* hit,
                     void* stream) {
    if (!terms || !offsets || !sum || !hit || n_cases < 0) return CBX_ERR_INVALID;
    if (n_cases == 0) return CBX_OK;
    DevGuard g(device);
    hipLaunchKernelGGL(cbx::debug_runsum_kernel, dim3(n_cases), dim3(64), 0, (hipStream_t)stream,
                       terms, offsets, thr, desc, sum, hit);
    return launch_done(device, hipGetLastError());
}

int cbx_debug_chainsum(int32_t device, const float* terms, const int32_t* offsets,
                       const float* thr, int32_t n_cases, float* sum, int32_t* hit, void* stream) {
    if (!terms || !offsets || !sum || !hit || n_cases < 0) return CBX_ERR_INVALID;
    if (n_cases == 0) return CBX_OK;
    DevGuard g(device);
    hipLaunchKernelGGL(cbx::debug_chain_kernel, dim3(n_cases), dim3(64), 0, (hipStream_t)stream,
                       terms, offsets, thr, sum, hit);
    return launch_done(device, hipGetLastError());
}

}  // extern "C"

// cbx_sampler_kernel.hip -- launch dispatch by vocabulary class, LDS sizing,
// and the diagnostic kernels (device exponential, device Philox).
#include <hip/hip_runtime.h>

#include "cbx_sampler_impl.h"

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

// One wave per case: the exact left-to-right binary32 sum of the case's terms
// (starting from its first term; at most 2048 terms are read) and, for thr > 0, the first index whose
// running sum reaches thr.
__global__ __launch_bounds__(64) void debug_seqsum_kernel(const float* t, const int32_t* off,
                                                          const float* thr, float* sum,
                                                          int32_t* hit) {
    const int c = blockIdx.x;
    const int b = off[c], n = off[c + 1] - b;
    if (n <= 0) return;
    int h;
    const float th = thr ? thr[c] : 0.0f;
    const float s = seq_sum_wave<kFastMax / 64>(t + b, min(n, kFastMax), t[b], 1, th, h);
    if (threadIdx.x == 0) {
        sum[c] = s;
        hit[c] = (th > 0.0f && t[b] >= th) ? 0 : h;
    }
}

}  // namespace

size_t lds_bytes_for(int32_t cap, int32_t n_vocab) {
    const size_t Wp = (size_t)(((n_vocab + 31) / 32 + 3) & ~3);
    return 3 * Wp * 4 + region_bytes(cap);
}

int32_t max_cap_for_lds(int32_t n_vocab, size_t lds_bytes) {
    int32_t cap = 1 << 16;
    while (cap > 64 && lds_bytes_for(cap, n_vocab) + kStaticLds > lds_bytes) cap >>= 1;
    return cap;
}

bool uses_wave_kernel(const KernelArgs& a) {
    return a.cap <= kWaveCap && a.n_vocab <= kWaveMaxVocab;
}

hipError_t launch_sample(const KernelArgs& a, hipStream_t stream) {
    // one wave per row while the survivors fit its list
    if (uses_wave_kernel(a)) {
        if (a.n_vocab <= 256 * 16) return a.n_vocab > 256 * 15 ? launch_w16t(a, stream) : launch_w16(a, stream);
        if (a.n_vocab <= 256 * 26) return a.n_vocab > 256 * 25 ? launch_w26t(a, stream) : launch_w26(a, stream);
        if (a.n_vocab <= kWaveMaxVocab)
            return a.n_vocab > 256 * 32 ? launch_w33t(a, stream) : launch_w33(a, stream);
    }
    // registers per lane sized to the vocabulary (6563 -> 26 per lane)
    if (a.n_vocab <= 256 * 16) return launch_v256x16(a, stream);
    if (a.n_vocab <= 256 * 26) return launch_v256x26(a, stream);
    if (a.n_vocab <= 256 * 32) return launch_v256x32(a, stream);
    if (a.n_vocab <= 1024 * 16) return launch_v1024x16(a, stream);
    return launch_v1024x32(a, stream);
}

hipError_t launch_redo(const KernelArgs& a, hipStream_t stream) {
    if (a.n_vocab <= 256 * 16) return launch_redo_v256x16(a, stream);
    if (a.n_vocab <= 256 * 26) return launch_redo_v256x26(a, stream);
    if (a.n_vocab <= 256 * 32) return launch_redo_v256x32(a, stream);
    if (a.n_vocab <= 1024 * 16) return launch_redo_v1024x16(a, stream);
    return launch_redo_v1024x32(a, stream);
}

hipError_t launch_debug_expf(const float* in, float* out, int64_t n, hipStream_t stream) {
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(debug_expf_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, in, out, n);
    return hipGetLastError();
}

hipError_t launch_debug_seqsum(const float* terms, const int32_t* offsets, const float* thr,
                              int32_t n_cases, float* sum, int32_t* hit, hipStream_t stream) {
    hipLaunchKernelGGL(debug_seqsum_kernel, dim3(n_cases), dim3(64), 0, stream, terms, offsets,
                       thr, sum, hit);
    return hipGetLastError();
}

hipError_t launch_debug_philox(uint64_t seed, const uint64_t* stream_ids, uint64_t step,
                               int32_t n, double* out, hipStream_t stream) {
    const int blocks = (n + 255) / 256;
    hipLaunchKernelGGL(debug_philox_kernel, dim3(blocks), dim3(256), 0, stream, seed, stream_ids,
                       step, n, out);
    return hipGetLastError();
}

}  // namespace cbx

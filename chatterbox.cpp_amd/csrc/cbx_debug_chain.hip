// Diagnostic kernel: the one-wave sampler's exact running sums (DPP sweep
// chains and binade segments) on given term lists, one wavefront per list.
#include "cbx_sampler_wave.h"

namespace cbx {
namespace {

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

hipError_t launch_debug_chain(const float* terms, const int32_t* offsets, const float* thr,
                              int32_t n_cases, float* sum, int32_t* hit, hipStream_t stream) {
    hipLaunchKernelGGL(debug_chain_kernel, dim3(n_cases), dim3(64), 0, stream, terms, offsets, thr,
                       sum, hit);
    return hipGetLastError();
}

}  // namespace cbx

// cbx_sampler_kernel.hip -- launch dispatch by vocabulary class and LDS
// sizing.
#include <hip/hip_runtime.h>

#include "cbx_sampler_impl.h"

namespace cbx {

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
    return a.cap <= kWaveCap &&
           (a.n_vocab <= kWaveMaxVocab || (a.n_vocab <= kMaxVocab && a.uncond == nullptr));
}

hipError_t launch_sample(const KernelArgs& a, hipStream_t stream) {
    // one wave per row while the survivors fit its list
    if (uses_wave_kernel(a)) {
        if (a.n_vocab <= 256 * 16) return a.n_vocab > 256 * 15 ? launch_w16t(a, stream) : launch_w16(a, stream);
        if (a.n_vocab <= 256 * 26) return a.n_vocab > 256 * 25 ? launch_w26t(a, stream) : launch_w26(a, stream);
        if (a.n_vocab <= kWaveMaxVocab)
            return a.n_vocab > 256 * 32 ? launch_w33t(a, stream) : launch_w33(a, stream);
        return (int64_t)a.n_steps * a.n_rows <= kChunkTwoWaveRows ? launch_w128c2(a, stream)
                                                                  : launch_w128c(a, stream);
    }
    // registers per lane sized to the vocabulary (6563 -> 13 per lane)
    if (a.n_vocab <= 512 * 8) return launch_v512x8(a, stream);
    if (a.n_vocab <= 512 * 13) return launch_v512x13(a, stream);
    if (a.n_vocab <= 512 * 16) return launch_v512x16(a, stream);
    if (a.n_vocab <= 1024 * 16) return launch_v1024x16(a, stream);
    return launch_v1024x32(a, stream);
}

hipError_t launch_decode(const KernelArgs& a, hipStream_t stream) {
    if (a.n_vocab <= 512 * 8) return launch_decode_v512x8(a, stream);
    if (a.n_vocab <= 512 * 13) return launch_decode_v512x13(a, stream);
    if (a.n_vocab <= 512 * 16) return launch_decode_v512x16(a, stream);
    if (a.n_vocab <= 1024 * 16) return launch_decode_v1024x16(a, stream);
    return launch_decode_v1024x32(a, stream);
}

hipError_t launch_redo(const KernelArgs& a, hipStream_t stream) {
    if (a.n_vocab <= 512 * 8) return launch_redo_v512x8(a, stream);
    if (a.n_vocab <= 512 * 13) return launch_redo_v512x13(a, stream);
    if (a.n_vocab <= 512 * 16) return launch_redo_v512x16(a, stream);
    if (a.n_vocab <= 1024 * 16) return launch_redo_v1024x16(a, stream);
    return launch_redo_v1024x32(a, stream);
}

}  // namespace cbx

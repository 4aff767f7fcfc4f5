// One-wave sampler for vocabularies up to 32768 ids (no CFG rows), the row
// read once in chunks of 2048 ids.
#include "cbx_sampler_wave.h"

namespace cbx {
hipError_t launch_w128c(const KernelArgs& a, hipStream_t stream) {
    return launch_wave<128, 0, true>(a, stream);
}
// the same with each row's chunks split over two waves (launches of at most
// kChunkTwoWaveRows row-steps)
hipError_t launch_w128c2(const KernelArgs& a, hipStream_t stream) {
    return launch_wave<128, 0, true, true>(a, stream);
}
}  // namespace cbx

// One-wave sampler for vocabularies of 8193..8448 ids: only the last of the
// 33 vectors per lane holds padding.
#include "cbx_sampler_wave.h"

namespace cbx {
hipError_t launch_w33t(const KernelArgs& a, hipStream_t stream) { return launch_wave<33, 32>(a, stream); }
}  // namespace cbx

// One-wave sampler for vocabularies of 6401..6656 ids: only the last of the
// 26 vectors per lane holds padding.
#include "cbx_sampler_wave.h"

namespace cbx {
hipError_t launch_w26t(const KernelArgs& a, hipStream_t stream) { return launch_wave<26, 25>(a, stream); }
}  // namespace cbx

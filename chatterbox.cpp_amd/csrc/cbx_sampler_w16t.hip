// One-wave sampler for vocabularies of 3841..4096 ids: only the last of the
// 16 vectors per lane holds padding.
#include "cbx_sampler_wave.h"

namespace cbx {
hipError_t launch_w16t(const KernelArgs& a, hipStream_t stream) { return launch_wave<16, 15>(a, stream); }
}  // namespace cbx

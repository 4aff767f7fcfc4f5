// One-wave sampler for vocabularies up to 4096 ids (64 scores per lane).
#include "cbx_sampler_wave.h"

namespace cbx {
hipError_t launch_w16(const KernelArgs& a, hipStream_t stream) { return launch_wave<16, 0>(a, stream); }
}  // namespace cbx

// One-wave sampler for vocabularies up to 8448 ids (132 scores per lane).
#include "cbx_sampler_wave.h"

namespace cbx {
hipError_t launch_w33(const KernelArgs& a, hipStream_t stream) { return launch_wave<33, 26>(a, stream); }
}  // namespace cbx

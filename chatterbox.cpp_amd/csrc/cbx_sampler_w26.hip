// One-wave sampler for vocabularies up to 6656 ids (104 scores per lane).
#include "cbx_sampler_wave.h"

namespace cbx {
hipError_t launch_w26(const KernelArgs& a, hipStream_t stream) { return launch_wave<26, 16>(a, stream); }
}  // namespace cbx

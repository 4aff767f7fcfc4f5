// Sampler kernels for vocabularies up to 4096 ids (256 lanes x 16 scores).
#include "cbx_sampler_impl.h"

namespace cbx {
hipError_t launch_v256x16(const KernelArgs& a, hipStream_t stream) {
    return launch_for<256, 16>(a, stream);
}
hipError_t launch_redo_v256x16(const KernelArgs& a, hipStream_t stream) {
    return launch_redo_for<256, 16>(a, stream);
}
}  // namespace cbx

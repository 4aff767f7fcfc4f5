// Sampler kernels for vocabularies up to 6656 ids (256 lanes x 26 scores).
#include "cbx_sampler_impl.h"

namespace cbx {
hipError_t launch_v256x26(const KernelArgs& a, hipStream_t stream) {
    return launch_for<256, 26>(a, stream);
}
hipError_t launch_redo_v256x26(const KernelArgs& a, hipStream_t stream) {
    return launch_redo_for<256, 26>(a, stream);
}
}  // namespace cbx

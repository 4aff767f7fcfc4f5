// Sampler kernels for vocabularies up to 8192 ids (256 lanes x 32 scores).
#include "cbx_sampler_impl.h"

namespace cbx {
hipError_t launch_v256x32(const KernelArgs& a, hipStream_t stream) {
    return launch_for<256, 32>(a, stream);
}
hipError_t launch_redo_v256x32(const KernelArgs& a, hipStream_t stream) {
    return launch_redo_for<256, 32>(a, stream);
}
}  // namespace cbx

// Sampler kernels for vocabularies up to 16384 ids (1024 lanes x 16 scores).
#include "cbx_sampler_impl.h"

namespace cbx {
hipError_t launch_v1024x16(const KernelArgs& a, hipStream_t stream) {
    return launch_for<1024, 16>(a, stream);
}
hipError_t launch_redo_v1024x16(const KernelArgs& a, hipStream_t stream) {
    return launch_redo_for<1024, 16>(a, stream);
}
hipError_t launch_decode_v1024x16(const KernelArgs& a, hipStream_t stream) {
    return launch_decode_for<1024, 16>(a, stream);
}
}  // namespace cbx

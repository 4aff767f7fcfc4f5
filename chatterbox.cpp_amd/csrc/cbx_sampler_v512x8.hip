// Sampler kernels for vocabularies up to 4096 ids (512 lanes x 8 scores).
#include "cbx_sampler_impl.h"

namespace cbx {
hipError_t launch_v512x8(const KernelArgs& a, hipStream_t stream) {
    return launch_for<512, 8>(a, stream);
}
hipError_t launch_redo_v512x8(const KernelArgs& a, hipStream_t stream) {
    return launch_redo_for<512, 8>(a, stream);
}
hipError_t launch_decode_v512x8(const KernelArgs& a, hipStream_t stream) {
    return launch_decode_for<512, 8>(a, stream);
}
}  // namespace cbx

// Sampler kernels for vocabularies up to 8192 ids (512 lanes x 16 scores).
#include "cbx_sampler_impl.h"

namespace cbx {
hipError_t launch_v512x16(const KernelArgs& a, hipStream_t stream) {
    return launch_for<512, 16>(a, stream);
}
hipError_t launch_redo_v512x16(const KernelArgs& a, hipStream_t stream) {
    return launch_redo_for<512, 16>(a, stream);
}
hipError_t launch_decode_v512x16(const KernelArgs& a, hipStream_t stream) {
    return launch_decode_for<512, 16>(a, stream);
}
}  // namespace cbx

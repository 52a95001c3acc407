// Instantiations of the row-stationary kernel for shallow K (Kp <= 320): int16 rows and int8 planes,
// epilogues PLAIN, GEGLU and GELU, with int32 outputs or the int16 view.
#include "stripe_kernel.h"

namespace vk {
hipError_t launch_stripe(int src, int epi, const GemmParams& p, hipStream_t st) {
    if (src == SRC_I16) return launch_stripe_t<SRC_I16>(epi, p, st);
    if (src == SRC_I8) return launch_stripe_t<SRC_I8>(epi, p, st);
    return hipErrorInvalidValue;
}
hipError_t launch_stripe_view(int src, int epi, const GemmParams& p, hipStream_t st) {
    if (src == SRC_I16) return launch_stripe_view_t<SRC_I16>(epi, p, st);
    if (src == SRC_I8) return launch_stripe_view_t<SRC_I8>(epi, p, st);
    return hipErrorInvalidValue;
}
}  // namespace vk

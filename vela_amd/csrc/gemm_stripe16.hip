// Instantiations of the sixteen-rows-per-wave row-stationary kernel for shallow K (Kp <= 320): int16
// rows and int8 planes, epilogues PLAIN (no residual), GEGLU and GELU.
#include "stripe16_kernel.h"

namespace vk {
hipError_t launch_stripe16(int src, int epi, const GemmParams& p, hipStream_t st) {
    if (src == SRC_I16) return launch_stripe16_t<SRC_I16>(epi, p, st);
    if (src == SRC_I8) return launch_stripe16_t<SRC_I8>(epi, p, st);
    return hipErrorInvalidValue;
}
}  // namespace vk

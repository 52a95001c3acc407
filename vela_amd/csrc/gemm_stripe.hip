// Instantiations of the row-stationary kernel for shallow K: int16 rows and int8 planes, Kp <= 320
// (shape 0) and Kp <= 640 (shape 1), epilogues PLAIN, GEGLU and GELU.
#include "stripe_kernel.h"

namespace vk {
hipError_t launch_stripe(int src, int shape, int epi, const GemmParams& p, hipStream_t st) {
    if (src == SRC_I16) return shape == 0 ? launch_stripe_t<SRC_I16, StripeA>(epi, p, st) : launch_stripe_t<SRC_I16, StripeB>(epi, p, st);
    if (src == SRC_I8) return shape == 0 ? launch_stripe_t<SRC_I8, StripeA>(epi, p, st) : launch_stripe_t<SRC_I8, StripeB>(epi, p, st);
    return hipErrorInvalidValue;
}
}  // namespace vk

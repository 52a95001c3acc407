// Instantiations of the hi/lo GEMM kernel for the SRC_I16 source (all epilogues and tile variants).
#include "gemm_kernel.h"

namespace vk {
hipError_t launch_gemm_i16(int variant, int epi, const GemmParams& p, int batch, hipStream_t st) {
    return launch_gemm_src<SRC_I16>(variant, epi, p, batch, st);
}
}  // namespace vk

// Instantiations of the hi/lo GEMM kernel for the SRC_CONV16 source (all epilogues and tile
// variants), and of the halo-reuse 3x3 kernel that serves stride-1 convolutions with C % 64 == 0.
#include "conv_kernel.h"
#include "gemm_kernel.h"

namespace vk {
hipError_t launch_gemm_conv16(int variant, int epi, const GemmParams& p, int batch, hipStream_t st) {
    return launch_gemm_src<SRC_CONV16>(variant, epi, p, batch, st);
}

int conv_halo_bm(int epi, int H, int W, int C, int stride, int Ho, int Wo) {
    if (epi == EPI_GEGLU || epi == EPI_GELU || epi == EPI_QKV) return 0;
    return halo_fits(H, W, C, stride, Ho, Wo) ? HaloCfg::BM : 0;
}

hipError_t launch_gemm_conv16_halo(int bm, int epi, const GemmParams& p, hipStream_t st) {
    if (bm != HaloCfg::BM) return hipErrorInvalidValue;
    return launch_conv_halo(epi, p, st);
}
}  // namespace vk

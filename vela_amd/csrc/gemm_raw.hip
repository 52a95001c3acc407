// Single-plane int8 x int8 -> int32 GEMM (the Gemm::run replacement) and the split-K epilogue.
#include "gemm_kernel.h"

namespace vk {
hipError_t launch_gemm_raw(int variant, const GemmParams& p, int batch, hipStream_t st) {
    switch (variant) {
    case 1: return launch_dma_t<SRC_I8, EPI_RAW, TileD1>(p, batch, st);
    case 2: return launch_dma_t<SRC_I8, EPI_RAW, TileD2>(p, batch, st);
    case 3: return launch_dma_t<SRC_I8, EPI_RAW, TileD3>(p, batch, st);
    default: return launch_dma_t<SRC_I8, EPI_RAW, TileD0>(p, batch, st);
    }
}

hipError_t launch_splitk_epilogue(int epi, const GemmParams& p, hipStream_t st) {
    const int nout = epi == EPI_GEGLU ? (p.Nreal >> 1) : p.Nreal;
    const dim3 grid(unsigned((nout + 1023) / 1024), unsigned(p.Mreal < 65535 ? p.Mreal : 65535));
    switch (epi) {
    case EPI_PLAIN: hipLaunchKernelGGL(splitk_epilogue_kernel<EPI_PLAIN>, grid, dim3(256), 0, st, p); break;
    case EPI_SPLIT3: hipLaunchKernelGGL(splitk_epilogue_kernel<EPI_SPLIT3>, grid, dim3(256), 0, st, p); break;
    case EPI_GEGLU: hipLaunchKernelGGL(splitk_epilogue_kernel<EPI_GEGLU>, grid, dim3(256), 0, st, p); break;
    case EPI_GELU: hipLaunchKernelGGL(splitk_epilogue_kernel<EPI_GELU>, grid, dim3(256), 0, st, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
}  // namespace vk

// Single-plane int8 x int8 -> int32 GEMM (the Gemm::run replacement) and the split-K epilogue.
#include <algorithm>

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
    // one thread per (row, 4 columns), at most 16 blocks of 256 per CU (the kernel strides beyond)
    const long long threads = (long long)p.Mreal * ((nout + 3) / 4);
    const dim3 grid(unsigned(std::min<long long>((threads + 255) / 256, 4096)));
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

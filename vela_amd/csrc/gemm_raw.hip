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

// Sum of the K ranges' partial sums of a split single-plane GEMM: C[r][c] = sum over s of
// ws[s][r][c], four columns per thread (N % 4 == 0, ld and ldc multiples of 4).
__global__ void __launch_bounds__(256) raw_reduce_kernel(const v4i* __restrict__ ws, int splits, long long plane4, int ld4, int M, int N4,
                                                         v4i* __restrict__ C, int ldc4) {
    const long long total = (long long)M * N4;
    for (long long i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
        const int r = int(i / N4), c = int(i - (long long)r * N4);
        const v4i* src = ws + (long long)r * ld4 + c;
        v4i acc = src[0];
        for (int s = 1; s < splits; ++s) acc += src[s * plane4];
        C[(long long)r * ldc4 + c] = acc;
    }
}

// plane: bytes between K ranges in ws; ldw, ldc: row strides in int32 elements
hipError_t launch_raw_reduce(const int32_t* ws, int splits, long long plane, int ldw, int M, int N, int32_t* C, int ldc, hipStream_t st) {
    if (plane % 16 || ldw % 4 || ldc % 4 || N % 4) return hipErrorInvalidValue;
    const long long total = (long long)M * (N / 4);
    const dim3 grid(unsigned(std::min<long long>((total + 255) / 256, 4096)));
    hipLaunchKernelGGL(raw_reduce_kernel, grid, dim3(256), 0, st, reinterpret_cast<const v4i*>(ws), splits, plane / 16, ldw / 4, M, N / 4,
                       reinterpret_cast<v4i*>(C), ldc / 4);
    return hipGetLastError();
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

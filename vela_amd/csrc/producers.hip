// A-operand producers and the planar-path epilogues of the reference (src/kernels.cu), as HIP
// kernels for gfx950. They are memory-bound; all arithmetic is the reference's exact int64 form.
#include <climits>

#include "vk_common.h"

namespace vk {

__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
#pragma unroll
    for (int o = 32; o; o >>= 1) v = max(v, uint32_t(__shfl_xor(int(v), o)));
    return v;
}

__device__ __forceinline__ unsigned pack_hi4(int q0, int q1, int q2, int q3) {
    return (unsigned(uint8_t(q0 >> 8))) | (unsigned(uint8_t(q1 >> 8)) << 8) | (unsigned(uint8_t(q2 >> 8)) << 16) | (unsigned(uint8_t(q3 >> 8)) << 24);
}
__device__ __forceinline__ unsigned pack_lo4(int q0, int q1, int q2, int q3) {
    return (unsigned(uint8_t((q0 & 255) - 128))) | (unsigned(uint8_t((q1 & 255) - 128)) << 8) |
           (unsigned(uint8_t((q2 & 255) - 128)) << 16) | (unsigned(uint8_t((q3 & 255) - 128)) << 24);
}
constexpr unsigned PAD_HI4 = 0x00000000u, PAD_LO4 = 0x80808080u;   // value 0 = (hi 0, lo -128)

// k_quant_rows (src/kernels.cu:42-57, 727-731): one wave per row, rows [M, align32(M)) padded.
__global__ void __launch_bounds__(256) quant_rows_kernel(const int32_t* __restrict__ X, int M, int Mp, int K, int ldx,
                                                         int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                         int32_t* __restrict__ e, int Kp) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= Mp) return;
    unsigned* h = reinterpret_cast<unsigned*>(hi + size_t(r) * Kp);
    unsigned* l = reinterpret_cast<unsigned*>(lo + size_t(r) * Kp);
    const int K4 = Kp >> 2;
    if (r >= M) {
        for (int k = lane; k < K4; k += 64) { h[k] = PAD_HI4; l[k] = PAD_LO4; }
        return;
    }
    const int32_t* x = X + size_t(r) * ldx;
    uint32_t m = 0;
    for (int k = lane; k < K; k += 64) m = max(m, uabs(x[k]));
    const int ee = rowexp_u32(wave_umax(m));
    if (lane == 0) e[r] = ee;
    for (int k4 = lane; k4 < K4; k4 += 64) {
        int q[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) { const int k = 4 * k4 + j; q[j] = k < K ? quant16_32(x[k], ee) : 0; }
        h[k4] = pack_hi4(q[0], q[1], q[2], q[3]);
        l[k4] = pack_lo4(q[0], q[1], q[2], q[3]);
    }
}

// k_pixmax (src/kernels.cu:106-115): pm[row] = max_c |X[row, c]|, one wave per row.
__global__ void __launch_bounds__(256) pixmax_kernel(const int32_t* __restrict__ X, int rows, int C, uint32_t* __restrict__ pm) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int32_t* x = X + size_t(r) * C;
    uint32_t m = 0;
    for (int c = lane; c < C; c += 64) m = max(m, uabs(x[c]));
    m = wave_umax(m);
    if (lane == 0) pm[r] = m;
}

__device__ __forceinline__ uint32_t window_max(const uint32_t* __restrict__ pm, int b, int H, int W, int stride, int oy, int ox) {
    uint32_t m = 0;
    for (int ky = 0; ky < 3; ++ky)
        for (int kx = 0; kx < 3; ++kx) {
            const int iy = oy * stride - 1 + ky, ix = ox * stride - 1 + kx;
            if (iy >= 0 && iy < H && ix >= 0 && ix < W) m = max(m, pm[(size_t(b) * H + iy) * W + ix]);
        }
    return m;
}

// k_conv_e (src/gemm_hl.cu:335-349)
__global__ void __launch_bounds__(256) conv_e_kernel(const uint32_t* __restrict__ pm, int B, int H, int W, int stride, int Ho, int Wo,
                                                     int32_t* __restrict__ e) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= B * Ho * Wo) return;
    const int pp = r % (Ho * Wo), b = r / (Ho * Wo), oy = pp / Wo, ox = pp - oy * Wo;
    e[r] = rowexp_u32(window_max(pm, b, H, W, stride, oy, ox));
}

// k_im2col3 (src/kernels.cu:117-170, 740-744): one block per output row (tap-major K, C % 4 == 0);
// rows [rows, align32(rows)) get hi 0x00 / lo 0x80 (written here by a kernel, not a memset).
__global__ void __launch_bounds__(256) im2col3_kernel(const int32_t* __restrict__ X, const uint32_t* __restrict__ pm, int B, int H, int W,
                                                      int C, int stride, int Ho, int Wo, int rows, int8_t* __restrict__ hi,
                                                      int8_t* __restrict__ lo, int32_t* __restrict__ e, int Kp) {
    __shared__ int she;
    const int r = blockIdx.x;
    unsigned* h = reinterpret_cast<unsigned*>(hi + size_t(r) * Kp);
    unsigned* l = reinterpret_cast<unsigned*>(lo + size_t(r) * Kp);
    const int K4 = Kp >> 2;
    if (r >= rows) {
        for (int k = threadIdx.x; k < K4; k += 256) { h[k] = PAD_HI4; l[k] = PAD_LO4; }
        return;
    }
    const int b = r / (Ho * Wo), p = r % (Ho * Wo), oy = p / Wo, ox = p % Wo;
    if (threadIdx.x == 0) {
        she = rowexp_u32(window_max(pm, b, H, W, stride, oy, ox));
        e[r] = she;
    }
    __syncthreads();
    const int ee = she, C4 = C >> 2, K4r = 9 * C4;
    for (int idx = threadIdx.x; idx < K4; idx += 256) {
        if (idx >= K4r) { h[idx] = PAD_HI4; l[idx] = PAD_LO4; continue; }
        const int tap = idx / C4, c = (idx - tap * C4) * 4;
        const int iy = oy * stride - 1 + tap / 3, ix = ox * stride - 1 + tap % 3;
        int q[4] = {0, 0, 0, 0};
        if (iy >= 0 && iy < H && ix >= 0 && ix < W) {
            const int4 v = *reinterpret_cast<const int4*>(X + ((size_t(b) * H + iy) * W + ix) * C + c);
            q[0] = quant16_32(v.x, ee); q[1] = quant16_32(v.y, ee); q[2] = quant16_32(v.z, ee); q[3] = quant16_32(v.w, ee);
        }
        h[idx] = pack_hi4(q[0], q[1], q[2], q[3]);
        l[idx] = pack_lo4(q[0], q[1], q[2], q[3]);
    }
}

// k_epilogue (src/kernels.cu:70-95): four columns per thread. With GN, the per-(sample, group)
// sum, min and max of the outputs are gathered in LDS and flushed by one global atomic each per
// block; a block's 1024 elements lie in one sample ((T * N) % 1024 == 0, checked on the host).
// A group is flushed when it holds values (min or max moved from its initial value); the reference's
// test of min != INT_MAX alone would skip a block's group whose outputs all saturated to INT_MAX.
template <bool GN>
__global__ void __launch_bounds__(256) epilogue_kernel(const int32_t* __restrict__ Chi, const int32_t* __restrict__ Clo, int M, int N, int ldc,
                                                       const int4* __restrict__ cst, const int32_t* __restrict__ e, int32_t* Y, int ldy,
                                                       const int32_t* R, GnStat* gs, int T) {
    __shared__ long long gsum[32];
    __shared__ int gmin[32], gmax[32];
    if (GN) {
        if (threadIdx.x < 32) { gsum[threadIdx.x] = 0; gmin[threadIdx.x] = INT_MAX; gmax[threadIdx.x] = INT_MIN; }
        __syncthreads();
    }
    const int tpr = N >> 2;
    const size_t idx = size_t(blockIdx.x) * 256 + threadIdx.x;
    const bool live = idx < size_t(M) * tpr;
    if (!GN && !live) return;
    int r = 0, n = 0;
    int y[4] = {0, 0, 0, 0};
    if (live) {
        r = int(idx / tpr);
        n = int(idx - size_t(r) * tpr) * 4;
        const int er = e[r];
        const int4 hv = *reinterpret_cast<const int4*>(Chi + size_t(r) * ldc + n);
        const int4 lv = *reinterpret_cast<const int4*>(Clo + size_t(r) * ldc + n);
        const int hh[4] = {hv.x, hv.y, hv.z, hv.w}, ll[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) { const int4 c = cst[n + j]; y[j] = epi1_exact(hh[j], ll[j], c.x, c.y, c.z, c.w, er); }
        if (R) {
            const int4 rv = *reinterpret_cast<const int4*>(R + size_t(r) * ldy + n);
            y[0] = add_sat(y[0], rv.x); y[1] = add_sat(y[1], rv.y); y[2] = add_sat(y[2], rv.z); y[3] = add_sat(y[3], rv.w);
        }
        *reinterpret_cast<int4*>(Y + size_t(r) * ldy + n) = make_int4(y[0], y[1], y[2], y[3]);
    }
    if (GN) {
        if (live) {
            const int cg = N >> 5;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int g = (n + j) / cg;
                atomicAdd(reinterpret_cast<unsigned long long*>(&gsum[g]), static_cast<unsigned long long>(static_cast<long long>(y[j])));
                atomicMin(&gmin[g], y[j]);
                atomicMax(&gmax[g], y[j]);
            }
        }
        __syncthreads();
        if (threadIdx.x < 32 && (gmin[threadIdx.x] != INT_MAX || gmax[threadIdx.x] != INT_MIN)) {
            const int b = int(size_t(blockIdx.x) * 256 / size_t(tpr) / size_t(T));
            GnStat* s = gs + b * 32 + threadIdx.x;
            atomicAdd(reinterpret_cast<unsigned long long*>(&s->sum), static_cast<unsigned long long>(gsum[threadIdx.x]));
            atomicMin(&s->mn, gmin[threadIdx.x]);
            atomicMax(&s->mx, gmax[threadIdx.x]);
        }
    }
}

// k_epilogue_split (src/kernels.cu:97-104)
__global__ void __launch_bounds__(256) epilogue_split_kernel(const int32_t* __restrict__ Chi, const int32_t* __restrict__ Clo, int M, int N,
                                                             int ldc, const int4* __restrict__ cst, const int32_t* __restrict__ e, int Cs,
                                                             int32_t* __restrict__ Y0, int32_t* __restrict__ Y1, int32_t* __restrict__ Y2) {
    const size_t idx = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= size_t(M) * N) return;
    const int r = int(idx / N), n = int(idx - size_t(r) * N);
    const int part = n >= 2 * Cs ? 2 : (n >= Cs ? 1 : 0);
    int32_t* Y = part == 0 ? Y0 : (part == 1 ? Y1 : Y2);
    const int4 c = cst[n];
    Y[size_t(r) * Cs + (n - part * Cs)] = epi1_exact(Chi[size_t(r) * ldc + n], Clo[size_t(r) * ldc + n], c.x, c.y, c.z, c.w, e[r]);
}

// k_epilogue_geglu_q (src/kernels.cu:499-534 + quant_row_out :250-259): one block per row; the
// GEGLU values of the row are held in LDS (F <= 5120) for the row maximum and quantisation.
__global__ void __launch_bounds__(256) epilogue_geglu_q_kernel(const int32_t* __restrict__ Chi, const int32_t* __restrict__ Clo, int F, int ldc,
                                                               const int4* __restrict__ cst, const int32_t* __restrict__ e,
                                                               const int32_t* __restrict__ L, int8_t* __restrict__ hi,
                                                               int8_t* __restrict__ lo, int32_t* __restrict__ eo, int Kp) {
    __shared__ int v[5120];
    __shared__ uint32_t red[4];
    const int r = blockIdx.x, er = e[r];
    const size_t base = size_t(r) * ldc;
    uint32_t m = 0;
    for (int c = threadIdx.x; c < F; c += 256) {
        const int4 ca = cst[c], cg = cst[F + c];
        const int a = epi1_exact(Chi[base + c], Clo[base + c], ca.x, ca.y, ca.z, ca.w, er);
        const int g = epi1_exact(Chi[base + F + c], Clo[base + F + c], cg.x, cg.y, cg.z, cg.w, er);
        const int y = geglu_exact(a, g, L);
        v[c] = y;
        m = max(m, uabs(y));
    }
    m = wave_umax(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = max(max(red[0], red[1]), max(red[2], red[3]));
    const int ee = rowexp_u32(m);
    if (threadIdx.x == 0) eo[r] = ee;
    int8_t* h = hi + size_t(r) * Kp;
    int8_t* l = lo + size_t(r) * Kp;
    for (int c = threadIdx.x; c < Kp; c += 256) {
        const int q = c < F ? quant16_32(v[c], ee) : 0;
        h[c] = int8_t(q >> 8);
        l[c] = int8_t((q & 255) - 128);
    }
}

__global__ void __launch_bounds__(256) fill_u32_kernel(uint32_t* __restrict__ p, size_t n, uint32_t value) {
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256) p[i] = value;
}

// ---------------------------------------------------------------- host launchers

static inline unsigned blocks_for(size_t n, size_t per) { return unsigned((n + per - 1) / per); }

hipError_t launch_quant_rows(hipStream_t st, const int32_t* X, int M, int K, int ldx, int8_t* hi, int8_t* lo, int32_t* e, int Kp) {
    const int Mp = (M + 31) / 32 * 32;
    hipLaunchKernelGGL(quant_rows_kernel, dim3(blocks_for(Mp, 4)), dim3(256), 0, st, X, M, Mp, K, ldx, hi, lo, e, Kp);
    return hipGetLastError();
}
hipError_t launch_pixmax(hipStream_t st, const int32_t* X, int rows, int C, uint32_t* pm) {
    hipLaunchKernelGGL(pixmax_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, st, X, rows, C, pm);
    return hipGetLastError();
}
hipError_t launch_conv_e(hipStream_t st, const uint32_t* pm, int B, int H, int W, int stride, int32_t* e) {
    const int Ho = (H - 1) / stride + 1, Wo = (W - 1) / stride + 1, rows = B * Ho * Wo;
    hipLaunchKernelGGL(conv_e_kernel, dim3(blocks_for(rows, 256)), dim3(256), 0, st, pm, B, H, W, stride, Ho, Wo, e);
    return hipGetLastError();
}
hipError_t launch_im2col3(hipStream_t st, const int32_t* X, const uint32_t* pm, int B, int H, int W, int C, int stride, int8_t* hi, int8_t* lo,
                          int32_t* e, int Kp) {
    const int Ho = (H - 1) / stride + 1, Wo = (W - 1) / stride + 1, rows = B * Ho * Wo, Mp = (rows + 31) / 32 * 32;
    hipLaunchKernelGGL(im2col3_kernel, dim3(unsigned(Mp)), dim3(256), 0, st, X, pm, B, H, W, C, stride, Ho, Wo, rows, hi, lo, e, Kp);
    return hipGetLastError();
}
hipError_t launch_epilogue(hipStream_t st, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int4* cst, const int32_t* e,
                           int32_t* Y, int ldy, const int32_t* R, GnStat* gs, int T) {
    const dim3 grid(blocks_for(size_t(M) * (N / 4), 256));
    if (gs) hipLaunchKernelGGL(epilogue_kernel<true>, grid, dim3(256), 0, st, Chi, Clo, M, N, ldc, cst, e, Y, ldy, R, gs, T);
    else hipLaunchKernelGGL(epilogue_kernel<false>, grid, dim3(256), 0, st, Chi, Clo, M, N, ldc, cst, e, Y, ldy, R, gs, T);
    return hipGetLastError();
}
hipError_t launch_epilogue_split(hipStream_t st, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int4* cst,
                                 const int32_t* e, int Cs, int32_t* Y0, int32_t* Y1, int32_t* Y2) {
    hipLaunchKernelGGL(epilogue_split_kernel, dim3(blocks_for(size_t(M) * N, 256)), dim3(256), 0, st, Chi, Clo, M, N, ldc, cst, e, Cs, Y0, Y1, Y2);
    return hipGetLastError();
}
hipError_t launch_epilogue_geglu_q(hipStream_t st, const int32_t* Chi, const int32_t* Clo, int M, int F, int ldc, const int4* cst,
                                   const int32_t* e, const int32_t* L, int8_t* hi, int8_t* lo, int32_t* eo, int Kp) {
    hipLaunchKernelGGL(epilogue_geglu_q_kernel, dim3(unsigned(M)), dim3(256), 0, st, Chi, Clo, F, ldc, cst, e, L, hi, lo, eo, Kp);
    return hipGetLastError();
}
// k_gn_init (src/kernels.cu:173): sum 0, mn INT_MAX, mx INT_MIN, ss 0 for cnt statistics records
__global__ void __launch_bounds__(256) gn_init_kernel(GnStat* __restrict__ gs, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        gs[i].sum = 0;
        gs[i].mn = INT_MAX;
        gs[i].mx = INT_MIN;
        gs[i].ss = 0;
    }
}

hipError_t launch_gn_init(hipStream_t st, GnStat* gs, int n) {
    hipLaunchKernelGGL(gn_init_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, gs, n);
    return hipGetLastError();
}

hipError_t launch_fill_u32(hipStream_t st, uint32_t* p, size_t n, uint32_t value) {
    const unsigned g = unsigned(n / 256 + 1 < 4096 ? n / 256 + 1 : 4096);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(g), dim3(256), 0, st, p, n, value);
    return hipGetLastError();
}

}  // namespace vk

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

// The same for rows of at most 64 NV int4 words held in registers: one 16-byte load per word, the
// row read once (the general kernel above reads it twice). Needs ldx % 4 == 0 and a 16-byte aligned X.
template <int NV>
__global__ void __launch_bounds__(256) quant_rows_vec_kernel(const int32_t* __restrict__ X, int M, int Mp, int K, int ldx,
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
    const int4* x = reinterpret_cast<const int4*>(X + size_t(r) * ldx);
    int4 v[NV];
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int k4 = lane + 64 * j;
        v[j] = make_int4(0, 0, 0, 0);
        if (4 * k4 + 3 < K) v[j] = x[k4];
        else if (4 * k4 < K) {   // the row's last, partial word
            const int32_t* xs = reinterpret_cast<const int32_t*>(x + k4);
            v[j].x = xs[0];
            if (4 * k4 + 1 < K) v[j].y = xs[1];
            if (4 * k4 + 2 < K) v[j].z = xs[2];
        }
        m = max(max(m, max(uabs(v[j].x), uabs(v[j].y))), max(uabs(v[j].z), uabs(v[j].w)));
    }
    const int ee = rowexp_u32(wave_umax(m));
    if (lane == 0) e[r] = ee;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int k4 = lane + 64 * j;
        if (k4 < K4) {
            const int q0 = quant16_32(v[j].x, ee), q1 = quant16_32(v[j].y, ee), q2 = quant16_32(v[j].z, ee), q3 = quant16_32(v[j].w, ee);
            h[k4] = pack_hi4(q0, q1, q2, q3);
            l[k4] = pack_lo4(q0, q1, q2, q3);
        }
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

// k_conv_e (src/gemm_hl.cu:335-349): e[r] = row_exp of the maximum of pm over the 3x3 window of
// output pixel r (pad 1, image border excluded). Separable: a block takes one output row (b, oy) and
// a run of `oc` output columns; it first reduces the (at most three) input rows of the windows column
// by column into LDS, with 0 outside the image (pm >= 0, so 0 is the identity of the maximum), then
// each output column takes the maximum of three neighbouring column values. oc = min(256, 1024 /
// stride), so the (oc - 1) * stride + 3 input columns of a run fit the LDS row.
constexpr int CONVE_LDS = 1027;
__host__ __device__ inline int conv_e_run(int stride) { return stride >= 1024 ? 1 : min(256, 1024 / stride); }
__global__ void __launch_bounds__(256) conv_e_kernel(const uint32_t* __restrict__ pm, int H, int W, int stride, int Ho, int Wo, int runs,
                                                     int32_t* __restrict__ e) {
    __shared__ uint32_t colmax[CONVE_LDS];
    const int oc = conv_e_run(stride);
    const int row = blockIdx.x / runs, run = blockIdx.x - row * runs;   // row = b * Ho + oy
    const int oy = row % Ho, b = row / Ho;
    const int ox0 = run * oc;
    const int ix0 = ox0 * stride - 1;                  // first input column of the run's windows
    const int nx = min(oc, Wo - ox0);
    const int ncols = (nx - 1) * stride + 3;           // input columns its windows cover
    const int iy0 = oy * stride - 1;
    const uint32_t* img = pm + size_t(b) * H * W;
    for (int j = threadIdx.x; j < ncols; j += 256) {
        const int ix = ix0 + j;
        uint32_t m = 0;
        if (ix >= 0 && ix < W) {
#pragma unroll
            for (int ky = 0; ky < 3; ++ky) {
                const int iy = iy0 + ky;
                if (iy >= 0 && iy < H) m = max(m, img[size_t(iy) * W + ix]);
            }
        }
        colmax[j] = m;
    }
    __syncthreads();
    const int t = threadIdx.x;
    if (t < nx) {
        const int j = t * stride;
        const uint32_t m = max(max(colmax[j], colmax[j + 1]), colmax[j + 2]);
        e[size_t(row) * Wo + ox0 + t] = rowexp_u32(m);
    }
}

// k_im2col3 (src/kernels.cu:117-170, 740-744): the materialised 3x3 im2col, tap-major K
// (k = tap*C + c, tap = 3*ky + kx), quantised per output row with e = row_exp(window maximum of pm),
// pad columns [9C, Kp) and pad rows [rows, align32(rows)) set to the value 0 = (hi 0, lo -128).
// One wave per output row, four rows per block: lanes 0..8 fetch the window's nine pm values, a
// wave maximum gives e (no LDS), then the wave walks the nine taps, each lane quantising four
// consecutive channels per step (C % 4 == 0: 16-byte loads, 4-byte hi/lo stores).
__global__ void __launch_bounds__(256) im2col3_kernel(const int32_t* __restrict__ X, const uint32_t* __restrict__ pm, int H, int W,
                                                      int C, int stride, int Ho, int Wo, int rows, int rows_pad,
                                                      int8_t* __restrict__ hi, int8_t* __restrict__ lo, int32_t* __restrict__ e, int Kp) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows_pad) return;
    unsigned* h = reinterpret_cast<unsigned*>(hi + size_t(r) * Kp);
    unsigned* l = reinterpret_cast<unsigned*>(lo + size_t(r) * Kp);
    const int K4 = Kp >> 2, C4 = C >> 2;
    if (r >= rows) {
        for (int k = lane; k < K4; k += 64) { h[k] = PAD_HI4; l[k] = PAD_LO4; }
        return;
    }
    const int ox = r % Wo, oy = (r / Wo) % Ho, b = r / (Wo * Ho);
    const int iy0 = oy * stride - 1, ix0 = ox * stride - 1;
    // the window maximum: lane t < 9 holds tap t's pixel maximum (0 outside the image)
    uint32_t m = 0;
    if (lane < 9) {
        const int iy = iy0 + lane / 3, ix = ix0 + lane % 3;
        if (iy >= 0 && iy < H && ix >= 0 && ix < W) m = pm[(size_t(b) * H + iy) * W + ix];
    }
#pragma unroll
    for (int o = 8; o; o >>= 1) m = max(m, uint32_t(__shfl_xor(int(m), o)));   // lanes 0..15 hold all nine
    const int ee = rowexp_u32(uint32_t(__shfl(int(m), 0)));
    if (lane == 0) e[r] = ee;
    for (int tap = 0; tap < 9; ++tap) {
        const int iy = iy0 + tap / 3, ix = ix0 + tap % 3;
        const bool inside = iy >= 0 && iy < H && ix >= 0 && ix < W;
        const int4* src = reinterpret_cast<const int4*>(X + ((size_t(b) * H + (inside ? iy : 0)) * W + (inside ? ix : 0)) * C);
        for (int c4 = lane; c4 < C4; c4 += 64) {
            int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
            if (inside) {
                const int4 v = src[c4];
                q0 = quant16_32(v.x, ee); q1 = quant16_32(v.y, ee); q2 = quant16_32(v.z, ee); q3 = quant16_32(v.w, ee);
            }
            h[tap * C4 + c4] = pack_hi4(q0, q1, q2, q3);
            l[tap * C4 + c4] = pack_lo4(q0, q1, q2, q3);
        }
    }
    for (int k = 9 * C4 + lane; k < K4; k += 64) { h[k] = PAD_HI4; l[k] = PAD_LO4; }
}

// k_epilogue (src/kernels.cu:70-95, 732-736): y = epi1 of the cuBLASLt-path plane sums (+ residual,
// saturated). The output [M x N] is processed in spans of 1024 consecutive row-major elements, one
// wave per span; per step lane l takes the four consecutive columns at element span + 256 j + 4 l
// (N % 4 == 0, so they lie in one row), so each load/store instruction of a wave covers 1 KB.
// With GN the span is also the region the statistics are gathered over, as in the reference: the
// wave's sum/min/max per group go to a table of its own in LDS (each lane first merges its four
// values by group) and are flushed to GnStat[(first row of the span / T) * 32 + group] when the
// min is not INT_MAX (a span whose outputs of a group are all INT_MAX adds nothing).
struct GnTable {
    long long sum[32];
    int mn[32], mx[32];
};

template <bool GN>
__global__ void __launch_bounds__(256) epilogue_kernel(const int32_t* __restrict__ Chi, const int32_t* __restrict__ Clo, int M, int N, int ldc,
                                                       const int4* __restrict__ cst, const int32_t* __restrict__ e, int32_t* Y, int ldy,
                                                       const int32_t* R, GnStat* gs, int T) {
    __shared__ GnTable tab[GN ? 4 : 1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    GnTable& t = tab[GN ? wave : 0];
    if (GN && lane < 32) { t.sum[lane] = 0; t.mn[lane] = INT_MAX; t.mx[lane] = INT_MIN; }
    const unsigned long long total = (unsigned long long)M * unsigned(N);
    const unsigned long long s0 = ((unsigned long long)blockIdx.x * 4 + wave) * 1024ull;
    const int cg = N >> 5;
    if (GN) __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned long long el = s0 + 256ull * j + 4ull * lane;
        if (el >= total) break;
        const int r = int(el / unsigned(N)), n = int(el - (unsigned long long)r * unsigned(N));
        const int er = e[r];
        const int4 hv = *reinterpret_cast<const int4*>(Chi + size_t(r) * ldc + n);
        const int4 lv = *reinterpret_cast<const int4*>(Clo + size_t(r) * ldc + n);
        const int4 c0 = cst[n], c1 = cst[n + 1], c2 = cst[n + 2], c3 = cst[n + 3];
        int y[4] = {epi1_exact(hv.x, lv.x, c0.x, c0.y, c0.z, c0.w, er), epi1_exact(hv.y, lv.y, c1.x, c1.y, c1.z, c1.w, er),
                    epi1_exact(hv.z, lv.z, c2.x, c2.y, c2.z, c2.w, er), epi1_exact(hv.w, lv.w, c3.x, c3.y, c3.z, c3.w, er)};
        if (R) {
            const int4 rv = *reinterpret_cast<const int4*>(R + size_t(r) * ldy + n);
            y[0] = add_sat(y[0], rv.x); y[1] = add_sat(y[1], rv.y); y[2] = add_sat(y[2], rv.z); y[3] = add_sat(y[3], rv.w);
        }
        *reinterpret_cast<int4*>(Y + size_t(r) * ldy + n) = make_int4(y[0], y[1], y[2], y[3]);
        if constexpr (GN) {
            // runs of equal group among the four columns: one atomic triple per run
            int v = 0;
            while (v < 4) {
                const int g = (n + v) / cg;
                long long sm = 0;
                int mn = INT_MAX, mx = INT_MIN;
                for (; v < 4 && (n + v) / cg == g; ++v) { sm += y[v]; mn = min(mn, y[v]); mx = max(mx, y[v]); }
                atomicAdd(reinterpret_cast<unsigned long long*>(&t.sum[g]), static_cast<unsigned long long>(sm));
                atomicMin(&t.mn[g], mn);
                atomicMax(&t.mx[g], mx);
            }
        }
    }
    if constexpr (GN) {
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (s0 < total && lane < 32 && t.mn[lane] != INT_MAX) {
            GnStat* d = gs + int((s0 / unsigned(N)) / unsigned(T)) * 32 + lane;
            atomicAdd(reinterpret_cast<unsigned long long*>(&d->sum), static_cast<unsigned long long>(t.sum[lane]));
            atomicMin(&d->mn, t.mn[lane]);
            atomicMax(&d->mx, t.mx[lane]);
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

// rows: the rows written, M and the pad rows [M, rows) (k_quant_rows: align32(M))
hipError_t launch_quant_rows(hipStream_t st, const int32_t* X, int M, int K, int ldx, int8_t* hi, int8_t* lo, int32_t* e, int Kp, int rows) {
    const int Mp = rows;
    const dim3 grid(blocks_for(Mp, 4));
    const int words = (Kp / 4 + 63) / 64;   // int4 words per lane
    if (ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0 && words <= 8) {
        switch (words) {
        case 1: hipLaunchKernelGGL(quant_rows_vec_kernel<1>, grid, dim3(256), 0, st, X, M, Mp, K, ldx, hi, lo, e, Kp); break;
        case 2: hipLaunchKernelGGL(quant_rows_vec_kernel<2>, grid, dim3(256), 0, st, X, M, Mp, K, ldx, hi, lo, e, Kp); break;
        case 3:
        case 4: hipLaunchKernelGGL(quant_rows_vec_kernel<4>, grid, dim3(256), 0, st, X, M, Mp, K, ldx, hi, lo, e, Kp); break;
        default: hipLaunchKernelGGL(quant_rows_vec_kernel<8>, grid, dim3(256), 0, st, X, M, Mp, K, ldx, hi, lo, e, Kp); break;
        }
        return hipGetLastError();
    }
    hipLaunchKernelGGL(quant_rows_kernel, grid, dim3(256), 0, st, X, M, Mp, K, ldx, hi, lo, e, Kp);
    return hipGetLastError();
}
hipError_t launch_pixmax(hipStream_t st, const int32_t* X, int rows, int C, uint32_t* pm) {
    hipLaunchKernelGGL(pixmax_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, st, X, rows, C, pm);
    return hipGetLastError();
}
hipError_t launch_conv_e(hipStream_t st, const uint32_t* pm, int B, int H, int W, int stride, int32_t* e) {
    const int Ho = (H - 1) / stride + 1, Wo = (W - 1) / stride + 1;
    const int runs = int(blocks_for(Wo, conv_e_run(stride)));
    const long long nb = (long long)B * Ho * runs;
    if (nb > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(conv_e_kernel, dim3(unsigned(nb)), dim3(256), 0, st, pm, H, W, stride, Ho, Wo, runs, e);
    return hipGetLastError();
}
hipError_t launch_im2col3(hipStream_t st, const int32_t* X, const uint32_t* pm, int B, int H, int W, int C, int stride, int8_t* hi, int8_t* lo,
                          int32_t* e, int Kp) {
    const int Ho = (H - 1) / stride + 1, Wo = (W - 1) / stride + 1, rows = B * Ho * Wo, Mp = (rows + 31) / 32 * 32;
    hipLaunchKernelGGL(im2col3_kernel, dim3(blocks_for(Mp, 4)), dim3(256), 0, st, X, pm, H, W, C, stride, Ho, Wo, rows, Mp, hi, lo, e, Kp);
    return hipGetLastError();
}
hipError_t launch_epilogue(hipStream_t st, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int4* cst, const int32_t* e,
                           int32_t* Y, int ldy, const int32_t* R, GnStat* gs, int T) {
    const dim3 grid(unsigned((size_t(M) * N + 4095) / 4096));   // four 1024-element spans per block
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
// Fix-up of the int16 view the row-stationary kernel writes (stripe_kernel.h, VIEW): one wave per
// row, lanes over its 4-column words (coalesced). The row's exponent e = row_exp(max |y|) goes to
// e[r]. A word of a 32-column group that was quantised at a running exponent ec < e is rewritten
// from what it holds: with d the kept correction bit, y >> ec = q - d exactly; floor shifts compose,
// so y >> (e - 1) = (y >> ec) >> (e - 1 - ec), and quant16_32(y, e) = clamp(((y >> (e - 1)) + 1)
// >> 1). Exponents and masks are group-major ([group][row]). Words [F / 4, ld / 4) get the pad
// value (0, -128).
__global__ void __launch_bounds__(256) view_fix_kernel(const uint32_t* __restrict__ vmax, const uint8_t* __restrict__ vexp,
                                                       const uint32_t* __restrict__ vmask, int M, int F, int G,
                                                       int8_t* __restrict__ hi, int8_t* __restrict__ lo, int ld, int32_t* __restrict__ e) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= M) return;
    const int ef = rowexp_u32(vmax[r]);
    if (lane == 0) e[r] = ef;
    unsigned* h = reinterpret_cast<unsigned*>(hi + size_t(r) * ld);
    unsigned* l = reinterpret_cast<unsigned*>(lo + size_t(r) * ld);
    const int F4 = F >> 2;
    if (ef > 0) {
        for (int w = lane; w < F4; w += 64) {
            const int grp = w >> 3;
            const int ec = vexp[size_t(grp) * M + r];
            if (ec >= ef) continue;
            const unsigned bits = vmask[size_t(grp) * M + r] >> (4 * (w & 7));
            const int sh = ef - 1 - ec;
            const unsigned hw = h[w], lw = l[w];
            int q[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int q0 = (int(int8_t(hw >> (8 * v))) << 8) | int(((lw >> (8 * v)) & 255u) ^ 0x80u);
                const int fl = q0 - int((bits >> v) & 1u);
                q[v] = min(max(((fl >> sh) + 1) >> 1, -32767), 32767);
            }
            h[w] = pack_hi4(q[0], q[1], q[2], q[3]);
            l[w] = pack_lo4(q[0], q[1], q[2], q[3]);
        }
    }
    for (int w = F4 + lane; w < (ld >> 2); w += 64) { h[w] = PAD_HI4; l[w] = PAD_LO4; }
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

hipError_t launch_view_fix(hipStream_t st, const uint32_t* vmax, const uint8_t* vexp, const uint32_t* vmask, int M, int F, int G, int8_t* hi,
                           int8_t* lo, int ld, int32_t* e) {
    hipLaunchKernelGGL(view_fix_kernel, dim3(blocks_for(M, 4)), dim3(256), 0, st, vmax, vexp, vmask, M, F, G, hi, lo, ld, e);
    return hipGetLastError();
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

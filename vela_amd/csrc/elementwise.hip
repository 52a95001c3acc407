// The integer elementwise kernels between the GEMMs of the reference engine (src/kernels.cu:537-566,
// launchers :763-771, header src/kernels.h:31-35), bit-exact:
//   k_act       x = sat32(rshr(x lut16i(x, L), 16))                      in place (SiLU, GELU)
//   k_geglu     a = sat32(rshr(a sat32(rshr(g lut16i(g, L), 16)), 16))   in place
//   k_add       x = sat32(x + y)                                         in place
//   k_concat    out[r] = [A[r] | B[r]] (+ the GroupNorm sum/min/max of out, per 256-element region
//               with the reference's flush rule)
//   k_upsample2 nearest-neighbour x2 of an NHWC image
//
// All are HBM-bound streams. Each thread moves 16-byte pieces where the layout allows (n % 4 == 0 and
// aligned pointers for the flat ones, channel counts % 4 == 0 for concat / upsample) and single
// elements otherwise; grids are sized to a few blocks per CU with grid-stride loops. The activation
// table (2049 int32, 8 KB) is staged in LDS once per block and interpolated exactly as lut16i does
// (32-bit wrapping arithmetic), so any table gives the reference's bytes.
#include "vk_common.h"

namespace vk {

namespace {

constexpr int EW_NT = 256;       // threads per block
constexpr int LUT_ENTRIES = 2049;

unsigned ew_grid(size_t work) {
    const size_t g = (work + EW_NT - 1) / EW_NT;
    return unsigned(g < 2048 ? (g ? g : 1) : 2048);
}

// lut16i (src/intops.cuh:42-50) on a table in LDS
__device__ __forceinline__ int lut16i_lds(int x, const int32_t* __restrict__ L) {
    const i64 z = i64(x) + (16LL << 16);
    if (z < 0) return 0;
    if (z >= (32LL << 16)) return 65536;
    const int i = int(z >> 10), f = int(z & 1023);
    const int a = L[i], b = L[i + 1];
    return int(unsigned(a) + unsigned(int((unsigned(b) - unsigned(a)) * unsigned(f)) >> 10));
}

// sat32(rshr(v, 16)) for v = a b (|v| < 2^62: the rounding add does not wrap)
__device__ __forceinline__ int mul_rshr16(int a, int b) { return int(sat32((i64(a) * i64(b) + 32768) >> 16)); }

__device__ __forceinline__ int act1(int x, const int32_t* L) { return mul_rshr16(x, lut16i_lds(x, L)); }
__device__ __forceinline__ int geglu1(int a, int g, const int32_t* L) { return mul_rshr16(a, mul_rshr16(g, lut16i_lds(g, L))); }

__device__ __forceinline__ void load_table(int32_t* s, const int32_t* __restrict__ L) {
    for (int i = threadIdx.x; i < LUT_ENTRIES; i += EW_NT) s[i] = L[i];
    __syncthreads();
}

// VEC: n % 4 == 0 and 16-byte aligned operands, one int4 per step
template <bool VEC>
__global__ void __launch_bounds__(EW_NT) act_kernel(int32_t* X, size_t n, const int32_t* __restrict__ L) {
    __shared__ int32_t s_lut[LUT_ENTRIES];
    load_table(s_lut, L);
    const size_t stride = size_t(gridDim.x) * EW_NT;
    if constexpr (VEC) {
        int4* X4 = reinterpret_cast<int4*>(X);
        for (size_t i = size_t(blockIdx.x) * EW_NT + threadIdx.x; i < n / 4; i += stride) {
            int4 v = X4[i];
            v.x = act1(v.x, s_lut); v.y = act1(v.y, s_lut); v.z = act1(v.z, s_lut); v.w = act1(v.w, s_lut);
            X4[i] = v;
        }
    } else {
        for (size_t i = size_t(blockIdx.x) * EW_NT + threadIdx.x; i < n; i += stride) X[i] = act1(X[i], s_lut);
    }
}

template <bool VEC>
__global__ void __launch_bounds__(EW_NT) geglu_kernel(int32_t* A, const int32_t* __restrict__ G, size_t n, const int32_t* __restrict__ L) {
    __shared__ int32_t s_lut[LUT_ENTRIES];
    load_table(s_lut, L);
    const size_t stride = size_t(gridDim.x) * EW_NT;
    if constexpr (VEC) {
        int4* A4 = reinterpret_cast<int4*>(A);
        const int4* G4 = reinterpret_cast<const int4*>(G);
        for (size_t i = size_t(blockIdx.x) * EW_NT + threadIdx.x; i < n / 4; i += stride) {
            int4 a = A4[i];
            const int4 g = G4[i];
            a.x = geglu1(a.x, g.x, s_lut); a.y = geglu1(a.y, g.y, s_lut); a.z = geglu1(a.z, g.z, s_lut); a.w = geglu1(a.w, g.w, s_lut);
            A4[i] = a;
        }
    } else {
        for (size_t i = size_t(blockIdx.x) * EW_NT + threadIdx.x; i < n; i += stride) A[i] = geglu1(A[i], G[i], s_lut);
    }
}

template <bool VEC>
__global__ void __launch_bounds__(EW_NT) add_kernel(int32_t* X, const int32_t* __restrict__ Y, size_t n) {
    const size_t stride = size_t(gridDim.x) * EW_NT;
    if constexpr (VEC) {
        int4* X4 = reinterpret_cast<int4*>(X);
        const int4* Y4 = reinterpret_cast<const int4*>(Y);
        for (size_t i = size_t(blockIdx.x) * EW_NT + threadIdx.x; i < n / 4; i += stride) {
            int4 x = X4[i];
            const int4 y = Y4[i];
            x.x = add_sat(x.x, y.x); x.y = add_sat(x.y, y.y); x.z = add_sat(x.z, y.z); x.w = add_sat(x.w, y.w);
            X4[i] = x;
        }
    } else {
        for (size_t i = size_t(blockIdx.x) * EW_NT + threadIdx.x; i < n; i += stride) X[i] = add_sat(X[i], Y[i]);
    }
}

// concat without statistics: VEC when Ca % 4 == Cb % 4 == 0 and 16-byte aligned rows (a quad of
// output columns then comes from one source)
template <bool VEC>
__global__ void __launch_bounds__(EW_NT) concat_kernel(const int32_t* __restrict__ A, int Ca, const int32_t* __restrict__ B, int Cb, size_t rows,
                                                       int32_t* __restrict__ out) {
    const int Co = Ca + Cb;
    const size_t stride = size_t(gridDim.x) * EW_NT;
    if constexpr (VEC) {
        const int q = Co / 4;
        for (size_t i = size_t(blockIdx.x) * EW_NT + threadIdx.x; i < rows * size_t(q); i += stride) {
            const size_t r = i / unsigned(q);
            const int c = int(i - r * unsigned(q)) * 4;
            const int4 v = c < Ca ? *reinterpret_cast<const int4*>(A + r * Ca + c) : *reinterpret_cast<const int4*>(B + r * Cb + (c - Ca));
            *reinterpret_cast<int4*>(out + r * Co + c) = v;
        }
    } else {
        for (size_t i = size_t(blockIdx.x) * EW_NT + threadIdx.x; i < rows * size_t(Co); i += stride) {
            const size_t r = i / unsigned(Co);
            const int c = int(i - r * unsigned(Co));
            out[i] = c < Ca ? A[r * Ca + c] : B[r * Cb + (c - Ca)];
        }
    }
}

// concat with the GroupNorm sum/min/max of out (src/kernels.cu:542-556 with gnacc_*, :64-69): the
// reference gathers per block of 256 consecutive output elements (a region), group c / (Co / 32),
// and adds a region's record for a group to gs[sample * 32 + group] only when the region's minimum
// of that group is not INT_MAX; the region's sample is (its first element's row) / T. Here one wave
// per region, each lane four consecutive elements of one row (Co % 32 == 0), a 32-group table per
// wave in LDS.
__global__ void __launch_bounds__(EW_NT) concat_gn_kernel(const int32_t* __restrict__ A, int Ca, const int32_t* __restrict__ B, int Cb, size_t rows,
                                                          int32_t* __restrict__ out, GnStat* gs, int T, bool vec) {
    __shared__ long long s_sum[EW_NT / 64][32];
    __shared__ int s_mn[EW_NT / 64][32], s_mx[EW_NT / 64][32];
    const int Co = Ca + Cb, cg = Co >> 5;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const size_t tot = rows * size_t(Co);
    const size_t nreg = (tot + 255) / 256;   // the last region may be partial when rows % T != 0
    for (size_t reg = size_t(blockIdx.x) * (EW_NT / 64) + w; reg < nreg; reg += size_t(gridDim.x) * (EW_NT / 64)) {
        if (lane < 32) { s_sum[w][lane] = 0; s_mn[w][lane] = INT_MAX; s_mx[w][lane] = INT_MIN; }
        __builtin_amdgcn_wave_barrier();
        const size_t e0 = reg * 256 + size_t(lane) * 4;
        // Co % 32 == 0 and tot % 4 == 0: a lane's four elements are all inside or all outside
        const bool live = e0 < tot;
        const size_t r = live ? e0 / unsigned(Co) : 0;
        const int c = live ? int(e0 - r * unsigned(Co)) : 0;
        int v[4] = {0, 0, 0, 0};
        if (!live) {
        } else if (vec) {
            const int4 x = c < Ca ? *reinterpret_cast<const int4*>(A + r * Ca + c) : *reinterpret_cast<const int4*>(B + r * Cb + (c - Ca));
            v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
            *reinterpret_cast<int4*>(out + e0) = x;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int cc = c + j;
                v[j] = cc < Ca ? A[r * Ca + cc] : B[r * Cb + (cc - Ca)];
                out[e0 + j] = v[j];
            }
        }
        // the lane's four elements by group (consecutive columns: at most four groups, in order)
        if (live) {
        int g = c / cg;
        long long sum = v[0];
        int mn = v[0], mx = v[0];
#pragma unroll
        for (int j = 1; j < 4; ++j) {
            const int gj = (c + j) / cg;
            if (gj != g) {
                atomicAdd(reinterpret_cast<unsigned long long*>(&s_sum[w][g]), static_cast<unsigned long long>(sum));
                atomicMin(&s_mn[w][g], mn);
                atomicMax(&s_mx[w][g], mx);
                g = gj; sum = 0; mn = INT_MAX; mx = INT_MIN;
            }
            sum += v[j]; mn = min(mn, v[j]); mx = max(mx, v[j]);
        }
        atomicAdd(reinterpret_cast<unsigned long long*>(&s_sum[w][g]), static_cast<unsigned long long>(sum));
        atomicMin(&s_mn[w][g], mn);
        atomicMax(&s_mx[w][g], mx);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (lane < 32 && s_mn[w][lane] != INT_MAX) {
            GnStat* s = gs + (reg * 256 / unsigned(Co) / unsigned(T)) * 32 + lane;
            atomicAdd(reinterpret_cast<unsigned long long*>(&s->sum), static_cast<unsigned long long>(s_sum[w][lane]));
            atomicMin(&s->mn, s_mn[w][lane]);
            atomicMax(&s->mx, s_mx[w][lane]);
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// out[b, y, x, c] = X[b, y / 2, x / 2, c] (src/kernels.cu:557-561); VEC: C % 4 == 0 and 16-byte aligned
template <bool VEC>
__global__ void __launch_bounds__(EW_NT) upsample2_kernel(const int32_t* __restrict__ X, int B, int H, int W, int C, int32_t* __restrict__ out) {
    const int cq = VEC ? C / 4 : C;
    const size_t tot = size_t(B) * 4 * H * W * cq;
    const size_t stride = size_t(gridDim.x) * EW_NT;
    for (size_t i = size_t(blockIdx.x) * EW_NT + threadIdx.x; i < tot; i += stride) {
        size_t p = i / unsigned(cq);
        const int c = int(i - p * unsigned(cq));
        const int x = int(p % unsigned(2 * W));
        p /= unsigned(2 * W);
        const int y = int(p % unsigned(2 * H));
        const size_t b = p / unsigned(2 * H);
        const size_t src = ((b * H + (y >> 1)) * W + (x >> 1)) * C;
        if constexpr (VEC) reinterpret_cast<int4*>(out)[i] = *reinterpret_cast<const int4*>(X + src + 4 * c);
        else out[i] = X[src + c];
    }
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

hipError_t launch_act(hipStream_t st, int32_t* X, size_t n, const int32_t* L) {
    if (n % 4 == 0 && a16(X)) hipLaunchKernelGGL(act_kernel<true>, dim3(ew_grid(n / 4)), dim3(EW_NT), 0, st, X, n, L);
    else hipLaunchKernelGGL(act_kernel<false>, dim3(ew_grid(n)), dim3(EW_NT), 0, st, X, n, L);
    return hipGetLastError();
}

hipError_t launch_geglu(hipStream_t st, int32_t* A, const int32_t* G, size_t n, const int32_t* L) {
    if (n % 4 == 0 && a16(A) && a16(G)) hipLaunchKernelGGL(geglu_kernel<true>, dim3(ew_grid(n / 4)), dim3(EW_NT), 0, st, A, G, n, L);
    else hipLaunchKernelGGL(geglu_kernel<false>, dim3(ew_grid(n)), dim3(EW_NT), 0, st, A, G, n, L);
    return hipGetLastError();
}

hipError_t launch_add(hipStream_t st, int32_t* X, const int32_t* Y, size_t n) {
    if (n % 4 == 0 && a16(X) && a16(Y)) hipLaunchKernelGGL(add_kernel<true>, dim3(ew_grid(n / 4)), dim3(EW_NT), 0, st, X, Y, n);
    else hipLaunchKernelGGL(add_kernel<false>, dim3(ew_grid(n)), dim3(EW_NT), 0, st, X, Y, n);
    return hipGetLastError();
}

hipError_t launch_concat(hipStream_t st, const int32_t* A, int Ca, const int32_t* B, int Cb, int rows, int32_t* out, GnStat* gs, int T) {
    const int Co = Ca + Cb;
    const bool vec = Ca % 4 == 0 && Cb % 4 == 0 && a16(A) && a16(B) && a16(out);
    if (gs) {
        const size_t nreg = (size_t(rows) * Co + 255) / 256;
        const size_t g = (nreg + EW_NT / 64 - 1) / (EW_NT / 64);
        hipLaunchKernelGGL(concat_gn_kernel, dim3(unsigned(g < 4096 ? (g ? g : 1) : 4096)), dim3(EW_NT), 0, st, A, Ca, B, Cb, size_t(rows), out, gs, T, vec);
    } else if (vec) {
        hipLaunchKernelGGL(concat_kernel<true>, dim3(ew_grid(size_t(rows) * (Co / 4))), dim3(EW_NT), 0, st, A, Ca, B, Cb, size_t(rows), out);
    } else {
        hipLaunchKernelGGL(concat_kernel<false>, dim3(ew_grid(size_t(rows) * Co)), dim3(EW_NT), 0, st, A, Ca, B, Cb, size_t(rows), out);
    }
    return hipGetLastError();
}

hipError_t launch_upsample2(hipStream_t st, const int32_t* X, int B, int H, int W, int C, int32_t* out) {
    const size_t tot = size_t(B) * 4 * H * W * C;
    if (C % 4 == 0 && a16(X) && a16(out)) hipLaunchKernelGGL(upsample2_kernel<true>, dim3(ew_grid(tot / 4)), dim3(EW_NT), 0, st, X, B, H, W, C, out);
    else hipLaunchKernelGGL(upsample2_kernel<false>, dim3(ew_grid(tot)), dim3(EW_NT), 0, st, X, B, H, W, C, out);
    return hipGetLastError();
}

}  // namespace vk

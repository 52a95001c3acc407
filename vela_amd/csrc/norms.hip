// The integer normalisations on either side of the GEMM path (the GroupNorm that consumes the
// statistics a GEMM epilogue gathers, and the LayerNorm rows that feed the next GEMM), bit-exact
// with src/kernels.cu:172-305,349-420 and src/intops.cuh:18-56:
//
//   GroupNorm over X[B, T, C] with `groups` groups of cg = C / groups channels, per (b, group):
//     fin1   mean = floor((sum + n/2) / n), e = max(0, row_exp(max(mx - mean, mean - mn)) - 5)
//     stats2 ss = sum of (rounding shift of (x - mean) by e)^2   (no saturation)
//     fin2   var = floor(ss / n), eps = floor((2^(32 - 2e) + den/2) / den), sd = isqrt((var + eps) << 16)
//     apply  y = sat32(rshr(floor((x - mean) 2^(25 - e) + sd) / 2 sd) * g[c], 16) + beta[c])
//            (+ SiLU y = sat32(rshr(y * lut16i(y, Lsig), 16))), then int32 Y and the row maximum, or
//            the row's int16 view (quant_row_out)
//   LayerNorm per row of C: the same with the row as the group and rshr (saturating) deviations.
//
// Design. The reductions (sum/min/max and the squared deviations) read X once: 1024-thread blocks,
// a thread owning four adjacent channels of a run of rows with its loads issued before the
// arithmetic, one LDS atomic per (thread, group) and one global atomic per (block, group); blocks
// are sized so that about one lands on each CU, which keeps the same-address global atomics per
// record few. The row kernels are one wave per row with the row in registers (16-byte loads, the
// next row's loads in flight while the current one is computed). Their per-element arithmetic is in
// double wherever the double result is provably exact -- integers below 2^53, products by powers
// of two, and the normalised quotient by a bound on its rounding error (see NormK) -- because on
// this GPU double adds and FMAs issue at the full vector rate while 32-bit integer multiplies issue
// at a quarter of it; the few elements the bounds do not cover take the exact integer form.
#include <algorithm>
#include <climits>

#include "vk_common.h"

namespace vk {

// floor(a / b) for b != 0 (src/intops.cuh:18)
__device__ __forceinline__ i64 floor_div64(i64 a, i64 b) {
    i64 q = a / b;
    if (a % b != 0 && ((a < 0) != (b < 0))) --q;
    return q;
}

// e = #{k in [15, 32): m >= 2^k} for a 64-bit m (src/intops.cuh:37-38)
__device__ __forceinline__ int row_exp64(i64 m) {
    if (m < (1LL << 15)) return 0;
    if (m >= (1LL << 32)) return 17;
    return 32 - __clz(unsigned(m)) - 15;
}

// floor(sqrt(v)) for v >= 0 (0 for v <= 0): a double estimate, then exact integer corrections
__device__ __forceinline__ i64 isqrt64(i64 v) {
    if (v <= 0) return 0;
    i64 s = i64(sqrt(double(v)));
    while (s > 0 && s * s > v) --s;
    while ((s + 1) * (s + 1) <= v) ++s;
    return s;
}

// (x - mean) rounded and shifted right by e, no saturation (src/kernels.cu:197)
__device__ __forceinline__ i64 dev_shift(i64 d, int e) { return e ? ((d >> e) + ((d >> (e - 1)) & 1)) : d; }

__device__ __forceinline__ double clamp32d(double v) { return fmin(fmax(v, -2147483648.0), 2147483647.0); }

// ---------------------------------------------------------------- wave reductions (DPP)
//
// Four in-row DPP steps (lane ^ 1, lane ^ 2, the half-row mirror, the row mirror) leave every lane
// of a 16-lane row with the row's total; the four row totals are then read into scalar registers.
// Every lane of the wave must be active.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp32(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ double dppf64(double v) {
    const u64 b = __builtin_bit_cast(u64, v);
    const unsigned lo = unsigned(dpp32<CTRL>(int(b))), hi = unsigned(dpp32<CTRL>(int(b >> 32)));
    return __builtin_bit_cast(double, (u64(hi) << 32) | lo);
}
__device__ __forceinline__ double readlanef64(double v, int l) {
    const u64 b = __builtin_bit_cast(u64, v);
    const unsigned lo = unsigned(__builtin_amdgcn_readlane(int(b), l)), hi = unsigned(__builtin_amdgcn_readlane(int(b >> 32), l));
    return __builtin_bit_cast(double, (u64(hi) << 32) | lo);
}

// sum of integer-valued doubles whose partial sums stay below 2^53 (exact in any order)
__device__ __forceinline__ double wave_sumf64(double v) {
    v += dppf64<DPP_XOR1>(v);
    v += dppf64<DPP_XOR2>(v);
    v += dppf64<DPP_HALF_MIRROR>(v);
    v += dppf64<DPP_MIRROR>(v);
    return (readlanef64(v, 0) + readlanef64(v, 16)) + (readlanef64(v, 32) + readlanef64(v, 48));
}
__device__ __forceinline__ int wave_min32(int v) {
    v = min(v, dpp32<DPP_XOR1>(v));
    v = min(v, dpp32<DPP_XOR2>(v));
    v = min(v, dpp32<DPP_HALF_MIRROR>(v));
    v = min(v, dpp32<DPP_MIRROR>(v));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)), min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int wave_max32(int v) {
    v = max(v, dpp32<DPP_XOR1>(v));
    v = max(v, dpp32<DPP_XOR2>(v));
    v = max(v, dpp32<DPP_HALF_MIRROR>(v));
    v = max(v, dpp32<DPP_MIRROR>(v));
    return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)), max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ uint32_t wave_umax32(uint32_t v) {
    v = max(v, uint32_t(dpp32<DPP_XOR1>(int(v))));
    v = max(v, uint32_t(dpp32<DPP_XOR2>(int(v))));
    v = max(v, uint32_t(dpp32<DPP_HALF_MIRROR>(int(v))));
    v = max(v, uint32_t(dpp32<DPP_MIRROR>(int(v))));
    const uint32_t a = uint32_t(__builtin_amdgcn_readlane(int(v), 0)), b = uint32_t(__builtin_amdgcn_readlane(int(v), 16));
    const uint32_t c = uint32_t(__builtin_amdgcn_readlane(int(v), 32)), d = uint32_t(__builtin_amdgcn_readlane(int(v), 48));
    return max(max(a, b), max(c, d));
}

// ---------------------------------------------------------------- the normalised value
//
// yy = floor((d 2^s + sd) / (2 sd)) with d = x - mean, s = 25 - e (src/kernels.cu:217,296,380) equals
// floor(d K + 1/2) for the exact K = 2^(s - 1) / sd. In double, with d exact (|mean| < 2^36) and K
// correctly rounded, t = fma(d, K, 1/2) differs from d K + 1/2 by at most 2^-52 (|t| + 1): below 2^-30
// for |t| < 2^21, so floor(t) is exact whenever t lies at least 2^-16 from an integer. Then with
// |yy| < 2^21 and an int32 g, yy g is below 2^52 and rshr(yy g, 16) = floor(yy g 2^-16 + 1/2) is one
// exact FMA, a scaling by 2^-16 and a floor, and the saturations and the add of beta are exact double
// operations. The other elements (about one in 2^15 on any data, and those with |yy| >= 2^21), and
// every group whose record is outside the double form's range, take the exact integer form.
struct NormK {
    double mean;   // NaN: every element takes the exact form
    double K;      // 0 for sd = 0 (yy = 0)
};

__device__ __forceinline__ NormK norm_const(i64 mean, int e, i64 sd) {
    const bool ok = mean > -(1LL << 36) && mean < (1LL << 36) && e >= 0 && e <= 25 && sd >= 0 && sd < (1LL << 52);
    NormK k;
    k.mean = ok ? double(mean) : __builtin_nan("");
    k.K = (ok && sd > 0) ? (e <= 24 ? double(1 << (24 - e)) : 0.5) / double(sd) : 0.0;
    return k;
}

// the exact integer form (0 for sd = 0); the shift and the additions wrap in 64 bits
__device__ __forceinline__ i64 norm_exact(int x, i64 mean, int e, i64 sd) {
    if (sd == 0) return 0;
    const i64 d = i64(u64(i64(x)) - u64(mean));
    return floor_div64(i64((u64(d) << (25 - e)) + u64(sd)), i64(2 * u64(sd)));
}

// the general form: yy g wraps in 64 bits (src/kernels.cu:218)
__device__ __forceinline__ int norm_affine64(i64 yy, i64 g, i64 beta) {
    return int(sat32(i64(u64(rshr(i64(u64(yy) * u64(g)), 16)) + u64(beta))));
}

// SiLU by the Q16 sigmoid table: sat32(rshr(y lut16i(y), 16)) (src/kernels.cu:300), exact for any
// table (lut16i's 32-bit wrapping interpolation)
__device__ __forceinline__ int silu32(int y, const int32_t* L) {
    const i64 r = (i64(y) * lut16i(y, L) + (1LL << 15)) >> 16;
    return int(r < INT_MIN ? INT_MIN : (r > INT_MAX ? INT_MAX : r));
}
// ---------------------------------------------------------------- per-record finalisation

// src/kernels.cu:185-192
__global__ void __launch_bounds__(256) gn_fin1_kernel(GnStat* __restrict__ gs, int cnt, i64 n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= cnt) return;
    const i64 mean = floor_div64(gs[i].sum + n / 2, n);
    const i64 m = max(i64(gs[i].mx) - mean, mean - i64(gs[i].mn));
    gs[i].mean = mean;
    gs[i].e = max(0, row_exp64(m) - 5);
}

// src/kernels.cu:203-210
__global__ void __launch_bounds__(256) gn_fin2_kernel(GnStat* __restrict__ gs, int cnt, i64 n, i64 den) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= cnt) return;
    const i64 var = floor_div64(gs[i].ss, n);
    const int sh = 32 - 2 * gs[i].e;
    const i64 one = sh >= 0 ? (1LL << sh) : 0;
    const i64 eps = floor_div64(one + den / 2, den);
    gs[i].sd = isqrt64(i64(u64(var + eps) << 16));
}

// ---------------------------------------------------------------- GroupNorm reductions

constexpr int GN_MAXG = 64;        // groups a block can accumulate
constexpr int GN_THREADS = 1024;   // threads of a reduction block
constexpr int GN_CHUNK = 8;        // rows a thread loads before it accumulates

// SQ = false: sum, min, max of each (sample, group) region (src/kernels.cu:175-183); SQ = true: the
// squared shifted deviations from the record's mean (src/kernels.cu:193-201). A thread owns four
// adjacent channels: a block's threads cover a slab of qs channel quads (grid.y over the slabs)
// times R = GN_THREADS / qs rows, and a run of R * rpt consecutive rows of one sample (grid.x =
// B * runs), each thread rpt rows (a multiple of GN_CHUNK). C % 4 == 0, C % groups == 0, groups <=
// GN_MAXG.
template <bool SQ>
__global__ void __launch_bounds__(GN_THREADS) gn_reduce_kernel(const int32_t* __restrict__ X, int T, int C, int groups, int qs, int rpt, int runs,
                                                               GnStat* __restrict__ gs) {
    __shared__ long long s_sum[GN_MAXG];
    __shared__ int s_mn[GN_MAXG], s_mx[GN_MAXG];
    const int tid = threadIdx.x;
    const int Q = C >> 2, R = GN_THREADS / qs;
    const int tr = tid / qs, tq = tid - tr * qs;
    const int b = blockIdx.x / runs, run = blockIdx.x - b * runs;
    const int t0 = run * R * rpt + tr, t1 = min(T, (run + 1) * R * rpt);
    const int q4 = blockIdx.y * qs + tq, c0 = 4 * q4;
    const int cg = C / groups;
    if (tid < groups) { s_sum[tid] = 0; s_mn[tid] = INT_MAX; s_mx[tid] = INT_MIN; }
    __syncthreads();
    if (tr < R && q4 < Q) {
        int gi[4];
        i64 mean[4];
        int ev[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            gi[k] = (c0 + k) / cg;
            if constexpr (SQ) {
                mean[k] = gs[b * groups + gi[k]].mean;
                ev[k] = gs[b * groups + gi[k]].e;
            }
        }
        i64 acc[4] = {0, 0, 0, 0};
        int mn[4] = {INT_MAX, INT_MAX, INT_MAX, INT_MAX}, mx[4] = {INT_MIN, INT_MIN, INT_MIN, INT_MIN};
        const size_t step = size_t(R) * C;
        const int32_t* x = X + (size_t(b) * T + t0) * C + c0;
        for (int t = t0; t < t1; t += GN_CHUNK * R, x += GN_CHUNK * step) {
            int4 v[GN_CHUNK];
#pragma unroll
            for (int i = 0; i < GN_CHUNK; ++i)
                if (t + i * R < t1) v[i] = *reinterpret_cast<const int4*>(x + i * step);
#pragma unroll
            for (int i = 0; i < GN_CHUNK; ++i) {
                if (t + i * R >= t1) break;
                const int vv[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if constexpr (SQ) {
                        const i64 dd = dev_shift(i64(vv[k]) - mean[k], ev[k]);
                        acc[k] = i64(u64(acc[k]) + u64(dd) * u64(dd));
                    } else {
                        acc[k] += vv[k];
                        mn[k] = min(mn[k], vv[k]);
                        mx[k] = max(mx[k], vv[k]);
                    }
                }
            }
        }
        // the four channels fall in one to four groups
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (k > 0 && gi[k] == gi[k - 1]) continue;
            i64 a = 0;
            int lo = INT_MAX, hi = INT_MIN;
#pragma unroll
            for (int j = k; j < 4; ++j)
                if (gi[j] == gi[k]) { a = i64(u64(a) + u64(acc[j])); lo = min(lo, mn[j]); hi = max(hi, mx[j]); }
            atomicAdd(reinterpret_cast<unsigned long long*>(&s_sum[gi[k]]), (unsigned long long)a);
            if constexpr (!SQ) { atomicMin(&s_mn[gi[k]], lo); atomicMax(&s_mx[gi[k]], hi); }
        }
    }
    __syncthreads();
    // the groups this slab touches
    const int cs0 = min(C, int(blockIdx.y) * qs * 4), cs1 = min(C, int(blockIdx.y + 1) * qs * 4);
    const int g0 = cs0 / cg, g1 = (cs1 - 1) / cg;
    if (tid >= g0 && tid <= g1 && tid < groups) {
        GnStat* s = gs + b * groups + tid;
        if constexpr (SQ) {
            atomicAdd(reinterpret_cast<unsigned long long*>(&s->ss), (unsigned long long)s_sum[tid]);
        } else {
            atomicAdd(reinterpret_cast<unsigned long long*>(&s->sum), (unsigned long long)s_sum[tid]);
            atomicMin(&s->mn, s_mn[tid]);
            atomicMax(&s->mx, s_mx[tid]);
        }
    }
}

// ---------------------------------------------------------------- GroupNorm apply

// src/kernels.cu:211-219: elementwise, 64-bit g and beta
__global__ void __launch_bounds__(256) gn_apply_kernel(const int32_t* __restrict__ X, int B, int T, int C, int groups, const GnStat* __restrict__ gs,
                                                       const i64* __restrict__ g, const i64* __restrict__ beta, int32_t* __restrict__ Y) {
    const size_t tot = size_t(B) * T * C;
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < tot; i += size_t(gridDim.x) * 256) {
        const int c = int(i % C), b = int(i / (size_t(T) * C)), grp = c / (C / groups);
        const GnStat& s = gs[b * groups + grp];
        Y[i] = norm_affine64(norm_exact(X[i], s.mean, s.e, s.sd), g[c], beta[c]);   // (sd = 0: no defined quotient, 0)
    }
}

// ---------------------------------------------------------------- row tiles
//
// The row kernels work on tiles of RT consecutive rows (RT = 1, 2, 4 or 8): the LR = 64 / RT lanes
// lr * LR .. lr * LR + LR - 1 of a wave own row lr of the tile, lane lq of them the channel quads
// lq + LR j (slot j < NV) of that row. The host picks RT so that the quads fill the NV slots best
// (C = 320: four rows of 16 lanes, five slots each, every lane busy). Every lane's slots lie in one
// row, so a per-row quantity (a sum, an extreme) is a reduction over the row's LR lanes: in-row DPP
// steps, then for LR >= 32 one swizzle across rows and for LR = 64 a read of both halves.
__device__ __forceinline__ int swz_xor16(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x401F); }

__device__ __forceinline__ double rows_sumf64(double v, int LR) {
    v += dppf64<DPP_XOR1>(v);
    v += dppf64<DPP_XOR2>(v);
    v += dppf64<DPP_HALF_MIRROR>(v);
    if (LR >= 16) v += dppf64<DPP_MIRROR>(v);
    if (LR >= 32) {
        const u64 b = __builtin_bit_cast(u64, v);
        v += __builtin_bit_cast(double, (u64(unsigned(swz_xor16(int(b >> 32)))) << 32) | unsigned(swz_xor16(int(b))));
    }
    if (LR == 64) v = readlanef64(v, 0) + readlanef64(v, 32);
    return v;
}
__device__ __forceinline__ int rows_min32(int v, int LR) {
    v = min(v, dpp32<DPP_XOR1>(v));
    v = min(v, dpp32<DPP_XOR2>(v));
    v = min(v, dpp32<DPP_HALF_MIRROR>(v));
    if (LR >= 16) v = min(v, dpp32<DPP_MIRROR>(v));
    if (LR >= 32) v = min(v, swz_xor16(v));
    if (LR == 64) v = min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 32));
    return v;
}
__device__ __forceinline__ int rows_max32(int v, int LR) {
    v = max(v, dpp32<DPP_XOR1>(v));
    v = max(v, dpp32<DPP_XOR2>(v));
    v = max(v, dpp32<DPP_HALF_MIRROR>(v));
    if (LR >= 16) v = max(v, dpp32<DPP_MIRROR>(v));
    if (LR >= 32) v = max(v, swz_xor16(v));
    if (LR == 64) v = max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 32));
    return v;
}
__device__ __forceinline__ uint32_t rows_umax32(uint32_t v, int LR) {
    v = max(v, uint32_t(dpp32<DPP_XOR1>(int(v))));
    v = max(v, uint32_t(dpp32<DPP_XOR2>(int(v))));
    v = max(v, uint32_t(dpp32<DPP_HALF_MIRROR>(int(v))));
    if (LR >= 16) v = max(v, uint32_t(dpp32<DPP_MIRROR>(int(v))));
    if (LR >= 32) v = max(v, uint32_t(swz_xor16(int(v))));
    if (LR == 64) v = max(uint32_t(__builtin_amdgcn_readlane(int(v), 0)), uint32_t(__builtin_amdgcn_readlane(int(v), 32)));
    return v;
}

struct RowLane {
    int lr, lq, LR;   // row in the tile, lane in the row, lanes per row
};
__device__ __forceinline__ RowLane row_lane(int lane, int RT) {
    const int LR = 64 / RT;
    return RowLane{lane / LR, lane % LR, LR};
}

// The int16 view of the lane's row (quant_row_out, src/kernels.cu:317-331): e from the row's max |y|,
// the lane's slots quantised at e, the row's pads (0, -128) by its lanes.
template <int NV>
__device__ __forceinline__ void row_view_store(const int (&y)[NV][4], uint32_t m, const RowLane& rl, int Q, bool live, int8_t* h8, int8_t* l8,
                                               int32_t* e, int Kp) {
    const int ee = rowexp_u32(rows_umax32(m, rl.LR));
    if (!live) return;
    if (rl.lq == 0) *e = ee;
    unsigned* h = reinterpret_cast<unsigned*>(h8);
    unsigned* l = reinterpret_cast<unsigned*>(l8);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int q4 = rl.lq + rl.LR * j;
        if (q4 < Q) {
            int q[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) q[k] = quant16_32(y[j][k], ee);
            h[q4] = __builtin_amdgcn_perm(unsigned(q[1]), unsigned(q[0]), 0x0c0c0501u) | __builtin_amdgcn_perm(unsigned(q[3]), unsigned(q[2]), 0x05010c0cu);
            l[q4] = (__builtin_amdgcn_perm(unsigned(q[1]), unsigned(q[0]), 0x0c0c0400u) | __builtin_amdgcn_perm(unsigned(q[3]), unsigned(q[2]), 0x04000c0cu)) ^ 0x80808080u;
        }
    }
    for (int q4 = Q + rl.lq; q4 < (Kp >> 2); q4 += rl.LR) { h[q4] = 0u; l[q4] = 0x80808080u; }
}

// the lane's slots of its row; slots past the row's end load the row's first quad instead
template <int NV>
__device__ __forceinline__ void load_slots(int4 (&xv)[NV], const int32_t* x, const RowLane& rl, int Q) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int q4 = rl.lq + rl.LR * j;
        xv[j] = *reinterpret_cast<const int4*>(x + 4 * (q4 < Q ? q4 : 0));
    }
}

// the normalised value's double form (see NormK): f = floor(t), exact when ok
__device__ __forceinline__ double norm_floor(int x, const NormK& k, bool& ok) {
    const double t = fma(double(x) - k.mean, k.K, 0.5);
    const double f = floor(t);
    ok = fabs(t) < 0x1p21 && fabs((t - f) - 0.5) <= 0.5 - 0x1p-16;   // false for NaN
    return f;
}
// sat32(sat32(rshr(yy g, 16)) + beta) in double: with |yy g| < 2^52, (yy 2^-16) g + 1/2 is exact in one FMA
__device__ __forceinline__ double affine_d(double yy, int g, int beta) {
    return clamp32d(clamp32d(floor(fma(yy * 0x1p-16, double(g), 0.5))) + double(beta));
}
// SiLU for a table whose entries all lie in (-2^20, 2^20), on y held both as int and as an integer-valued
// double: the interpolated value l lies in that range too (no wrap: |(b - a) f| < 2^31), lut16i's index
// and fraction come from 32-bit arithmetic on y clamped to the table's range, and |y l| < 2^51 makes
// rshr(y l, 16) one exact FMA, a scaling and a floor.
__device__ __forceinline__ int silu_dd(int y, double yd, const int32_t* L) {
    const int z = min(max(y, -(1 << 20)), (1 << 20) - 1) + (1 << 20);
    const int a = L[z >> 10], b = L[(z >> 10) + 1];
    const int dba = ((b - a) << 8) >> 8;   // |b - a| < 2^21 for table entries below 2^20: a 24-bit product
    const int li = a + ((dba * (z & 1023)) >> 10);
    const int l = y < -(1 << 20) ? 0 : (y >= (1 << 20) ? 65536 : li);
    return int(clamp32d(floor(fma(yd, double(l), 32768.0) * 0x1p-16)));
}

constexpr int GN_SLOTS = 8;     // samples the rows of one apply block may span
constexpr int LUT_N = 2049;     // entries of a Q16 activation table
constexpr int LUT_SAFE = 1 << 20;

struct GnApplyArgs {
    const int32_t* X;
    int M, T, C, groups, RT, tiles_per_block;
    const GnStat* gs;
    const int32_t *g, *beta;
    int32_t* Y;
    uint32_t* pm;
    int8_t *hi, *lo;
    int32_t* e;
    int Kp;
};

// The tiles of one GroupNorm apply block; ACT: 0 none, 1 SiLU in double (table within 2^20), 2 SiLU exact.
template <int NV, bool VIEW, int ACT>
__device__ __forceinline__ void gn_apply_tiles(const GnApplyArgs& a, const NormK* s_k, const int4* s_g, const int4* s_b, const int32_t* s_lut, int b0) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int C = a.C, Q = C >> 2, T = a.T;
    const RowLane rl = row_lane(lane, a.RT);
    const int cg = C / a.groups;
    int gi[NV];   // the slot's four channel groups, 8 bits each
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        gi[j] = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) gi[j] |= (min(4 * (rl.lq + rl.LR * j) + k, C - 1) / cg) << (8 * k);
    }
    const int t_begin = blockIdx.x * a.tiles_per_block;
    for (int tile = t_begin + wave; tile < t_begin + a.tiles_per_block; tile += 4) {
        const int row0 = tile * a.RT;
        if (row0 >= a.M) break;
        const int row = min(row0 + rl.lr, a.M - 1);
        const bool live = row0 + rl.lr < a.M;
        const int32_t* x = a.X + size_t(row) * C;
        int4 xv[NV];
        load_slots<NV>(xv, x, rl, Q);
        const int kb = (row / T - b0) * a.groups;   // the row's first record in s_k
        int y[NV][4];
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int q4 = rl.lq + rl.LR * j;
            const bool sl = live && q4 < Q;
            const int c0 = 4 * (q4 < Q ? q4 : 0);
            const int xs[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
            const int4 gg = s_g[c0 >> 2], bb = s_b[c0 >> 2];
            const int g4[4] = {gg.x, gg.y, gg.z, gg.w}, b4[4] = {bb.x, bb.y, bb.z, bb.w};
            unsigned slow = 0;   // bit k: element k needs the exact form
            double yd[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                bool ok;
                const double f = norm_floor(xs[k], s_k[kb + ((gi[j] >> (8 * k)) & 255)], ok);
                yd[k] = affine_d(f, g4[k], b4[k]);
                y[j][k] = int(yd[k]);
                slow |= (sl && !ok) ? 1u << k : 0u;
            }
            if (__builtin_amdgcn_ballot_w64(slow != 0)) {
                while (slow) {
                    const int k = __builtin_ctz(slow);
                    slow &= slow - 1;
                    int xk = 0;
#pragma unroll
                    for (int k2 = 0; k2 < 4; ++k2) xk = k == k2 ? xs[k2] : xk;
                    const GnStat& s = a.gs[b0 * a.groups + kb + ((gi[j] >> (8 * k)) & 255)];
                    const int r = norm_affine64(norm_exact(xk, s.mean, s.e, s.sd), a.g[c0 + k], a.beta[c0 + k]);
#pragma unroll
                    for (int k2 = 0; k2 < 4; ++k2) {
                        y[j][k2] = k == k2 ? r : y[j][k2];
                        yd[k2] = k == k2 ? double(r) : yd[k2];
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (ACT == 1) y[j][k] = silu_dd(y[j][k], yd[k], s_lut);
                if constexpr (ACT == 2) y[j][k] = silu32(y[j][k], s_lut);
            }
            if (sl) m = max(m, max(max(uabs(y[j][0]), uabs(y[j][1])), max(uabs(y[j][2]), uabs(y[j][3]))));
            if constexpr (!VIEW)
                if (sl) *reinterpret_cast<int4*>(a.Y + size_t(row) * C + c0) = make_int4(y[j][0], y[j][1], y[j][2], y[j][3]);
        }
        if constexpr (VIEW) {
            row_view_store<NV>(y, m, rl, Q, live, a.hi + size_t(row) * a.Kp, a.lo + size_t(row) * a.Kp, a.e + row, a.Kp);
        } else if (a.pm) {
            m = rows_umax32(m, rl.LR);
            if (live && rl.lq == 0) a.pm[row] = m;
        }
    }
}

// src/kernels.cu:287-305 (k_gn_apply_row): a block of four waves owns tiles_per_block tiles of RT rows
// (spanning at most GN_SLOTS samples), a wave one tile at a time with the tile in registers
// (C <= 2560, C % 4 == 0, 16-byte loads). Dynamic LDS: the (sample, group) constants of the
// quotient, g, beta and the SiLU table. Outputs: Y and pm[row] = max |y| (pm may
// be NULL), or the int16 view (VIEW).
template <int NV, bool VIEW>
__global__ void __launch_bounds__(256) gn_apply_row_kernel(GnApplyArgs a, const int32_t* __restrict__ Lsig) {
    extern __shared__ int4 s_dyn[];
    NormK* s_k = reinterpret_cast<NormK*>(s_dyn);                 // GN_SLOTS * GN_MAXG
    int4* s_g = s_dyn + GN_SLOTS * GN_MAXG;                       // C / 4
    int4* s_b = s_g + (a.C >> 2);                                 // C / 4
    int32_t* s_lut = reinterpret_cast<int32_t*>(s_b + (a.C >> 2)); // LUT_N when Lsig
    const int r0 = blockIdx.x * a.tiles_per_block * a.RT, r1 = min(a.M, r0 + a.tiles_per_block * a.RT);
    const int b0 = r0 / a.T, nrec = ((r1 - 1) / a.T - b0 + 1) * a.groups;
    for (int i = threadIdx.x; i < nrec; i += 256) {
        const GnStat& s = a.gs[b0 * a.groups + i];
        s_k[i] = norm_const(s.mean, s.e, s.sd);
    }
    for (int i = threadIdx.x; i < (a.C >> 2); i += 256) {
        s_g[i] = reinterpret_cast<const int4*>(a.g)[i];
        s_b[i] = reinterpret_cast<const int4*>(a.beta)[i];
    }
    // SiLU in its double form needs every table entry (and so every interpolated value) below 2^20
    bool lut_ok = true;
    if (Lsig)
        for (int i = threadIdx.x; i < LUT_N; i += 256) {
            const int v = Lsig[i];
            s_lut[i] = v;
            lut_ok = lut_ok && v > -LUT_SAFE && v < LUT_SAFE;
        }
    lut_ok = __syncthreads_and(lut_ok);
    if (!Lsig) gn_apply_tiles<NV, VIEW, 0>(a, s_k, s_g, s_b, s_lut, b0);
    else if (lut_ok) gn_apply_tiles<NV, VIEW, 1>(a, s_k, s_g, s_b, s_lut, b0);
    else gn_apply_tiles<NV, VIEW, 2>(a, s_k, s_g, s_b, s_lut, b0);
}

// ---------------------------------------------------------------- LayerNorm

// eps = floor((2^(32 - 2 ex) + den / 2) / den) for every shift ex the statistics can give (0..12),
// computed on the host from den
struct LnEps {
    long long v[13];
};

// src/kernels.cu:221-246 (k_lnorm, 64-bit g/beta, int32 Y) and :349-390 (k_lnorm_q, int32 g/beta in
// dynamic LDS, int16 view): a block of four waves owns tiles_per_block tiles of RT rows, a
// wave one tile at a time with the tile in registers (C <= 2560, C % 4 == 0), reading each row once
// for the mean, the deviations and the output; every lane of a row computes the row's statistics
// from the row reductions. They are exact in double: |sum| < 2^43; mean = floor((sum + n/2) / n)
// from the correctly rounded quotient (its error, below 2^-21, is smaller than the 1/n gap of a
// non-integer quotient to the next integer); the deviation rshr(x - mean, ex) = floor((x - mean)
// 2^-ex + 1/2) is at most 2^20 in magnitude (|x - mean| <= max(mx - mean, mean - mn), which is below
// 2^(20 + ex), or below 2^33 with ex = 12), so ss < C 2^40 < 2^52 and var = floor(ss / n) likewise.
template <int NV, bool Q>
__global__ void __launch_bounds__(256) lnorm_kernel(const int32_t* __restrict__ X, int M, int C, int RT, int tiles_per_block, const void* __restrict__ gp,
                                                    const void* __restrict__ bp, LnEps eps, int32_t* __restrict__ Y, int8_t* __restrict__ hi,
                                                    int8_t* __restrict__ lo, int32_t* __restrict__ e, int Kp) {
    extern __shared__ int4 s_dyn[];
    int4* s_g = s_dyn;              // C / 4 (Q)
    int4* s_b = s_dyn + (C >> 2);   // C / 4 (Q)
    __shared__ long long s_eps[13];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if constexpr (Q) {
        for (int i = threadIdx.x; i < (C >> 2); i += 256) {
            s_g[i] = static_cast<const int4*>(gp)[i];
            s_b[i] = static_cast<const int4*>(bp)[i];
        }
    }
    if (threadIdx.x < 13) s_eps[threadIdx.x] = eps.v[threadIdx.x];
    __syncthreads();
    const int Qd = C >> 2;
    const RowLane rl = row_lane(lane, RT);
    const double n = double(C);
    const int t_begin = blockIdx.x * tiles_per_block;
    for (int tile = t_begin + wave; tile < t_begin + tiles_per_block; tile += 4) {
        const int row0 = tile * RT;
        if (row0 >= M) break;
        const int row = min(row0 + rl.lr, M - 1);
        const bool live = row0 + rl.lr < M;
        const int32_t* x = X + size_t(row) * C;
        int4 xv[NV];
        load_slots<NV>(xv, x, rl, Qd);
        int v[NV][4];
        double s = 0.0;
        int mn = INT_MAX, mx = INT_MIN;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const bool in = rl.lq + rl.LR * j < Qd;
            v[j][0] = xv[j].x; v[j][1] = xv[j].y; v[j][2] = xv[j].z; v[j][3] = xv[j].w;
            s += in ? (double(v[j][0]) + double(v[j][1])) + (double(v[j][2]) + double(v[j][3])) : 0.0;
            mn = in ? min(mn, min(min(v[j][0], v[j][1]), min(v[j][2], v[j][3]))) : mn;
            mx = in ? max(mx, max(max(v[j][0], v[j][1]), max(v[j][2], v[j][3]))) : mx;
        }
        s = rows_sumf64(s, rl.LR);
        mn = rows_min32(mn, rl.LR);
        mx = rows_max32(mx, rl.LR);
        const double mean_d = floor((s + double(C / 2)) / n);
        const i64 mean = i64(mean_d);
        const int ex = max(0, row_exp64(max(i64(mx) - mean, mean - i64(mn))) - 5);
        const double sc = double(1 << (12 - ex)) * 0x1p-12;   // 2^-ex (ex <= 12)
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const bool in = rl.lq + rl.LR * j < Qd;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const double dd = floor(fma(double(v[j][k]) - mean_d, sc, 0.5));
                ss = in ? fma(dd, dd, ss) : ss;
            }
        }
        ss = rows_sumf64(ss, rl.LR);
        const i64 sd = isqrt64(i64(u64(i64(floor(ss / n)) + s_eps[ex]) << 16));
        const NormK kk = norm_const(mean, ex, sd);
        int y[NV][4];
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int q4 = rl.lq + rl.LR * j;
            const bool sl = live && q4 < Qd;
            const int c0 = 4 * (q4 < Qd ? q4 : 0);
            unsigned slow = 0;   // bit k: element k needs the exact form
            int g4[4] = {0, 0, 0, 0}, b4[4] = {0, 0, 0, 0};
            if constexpr (Q) {
                const int4 gg = s_g[c0 >> 2], bb = s_b[c0 >> 2];
                g4[0] = gg.x; g4[1] = gg.y; g4[2] = gg.z; g4[3] = gg.w;
                b4[0] = bb.x; b4[1] = bb.y; b4[2] = bb.z; b4[3] = bb.w;
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                bool ok;
                const double f = norm_floor(v[j][k], kk, ok);
                if constexpr (Q) {
                    y[j][k] = int(affine_d(f, g4[k], b4[k]));
                } else {
                    y[j][k] = norm_affine64(ok ? i64(f) : 0, static_cast<const i64*>(gp)[c0 + k], static_cast<const i64*>(bp)[c0 + k]);
                }
                slow |= (sl && !ok) ? 1u << k : 0u;
            }
            if (__builtin_amdgcn_ballot_w64(slow != 0)) {
                while (slow) {
                    const int k = __builtin_ctz(slow);
                    slow &= slow - 1;
                    int xk = 0;
#pragma unroll
                    for (int k2 = 0; k2 < 4; ++k2) xk = k == k2 ? v[j][k2] : xk;
                    const i64 yy = norm_exact(xk, mean, ex, sd);
                    int r;
                    if constexpr (Q) r = norm_affine64(yy, static_cast<const int32_t*>(gp)[c0 + k], static_cast<const int32_t*>(bp)[c0 + k]);
                    else r = norm_affine64(yy, static_cast<const i64*>(gp)[c0 + k], static_cast<const i64*>(bp)[c0 + k]);
#pragma unroll
                    for (int k2 = 0; k2 < 4; ++k2) y[j][k2] = k == k2 ? r : y[j][k2];
                }
            }
            if (sl) m = max(m, max(max(uabs(y[j][0]), uabs(y[j][1])), max(uabs(y[j][2]), uabs(y[j][3]))));
            if constexpr (!Q)
                if (sl) *reinterpret_cast<int4*>(Y + size_t(row) * C + c0) = make_int4(y[j][0], y[j][1], y[j][2], y[j][3]);
        }
        if constexpr (Q) row_view_store<NV>(y, m, rl, Qd, live, hi + size_t(row) * Kp, lo + size_t(row) * Kp, e + row, Kp);
    }
}

// ---------------------------------------------------------------- launchers

static inline unsigned nblocks(size_t n, size_t per) { return unsigned((n + per - 1) / per); }

hipError_t launch_gn_fin1(hipStream_t st, GnStat* gs, int cnt, i64 n) {
    hipLaunchKernelGGL(gn_fin1_kernel, dim3(nblocks(cnt, 256)), dim3(256), 0, st, gs, cnt, n);
    return hipGetLastError();
}
hipError_t launch_gn_fin2(hipStream_t st, GnStat* gs, int cnt, i64 n, i64 den) {
    hipLaunchKernelGGL(gn_fin2_kernel, dim3(nblocks(cnt, 256)), dim3(256), 0, st, gs, cnt, n, den);
    return hipGetLastError();
}

// Reduction grid: slabs of at most 256 channel quads (an equal split of C / 4), R = 1024 / slab rows
// per block step, and rows per thread (a multiple of GN_CHUNK, at most 64) chosen so that the grid is
// about one block per CU: deep per-thread load queues and few same-address atomics per record.
hipError_t launch_gn_reduce(hipStream_t st, bool sq, const int32_t* X, int B, int T, int C, int groups, GnStat* gs) {
    const int Q = C / 4, nslab = (Q + 255) / 256, qs = (Q + nslab - 1) / nslab, R = GN_THREADS / qs;
    const long long target = 256;   // blocks
    const long long rows_per_block = std::max<long long>(1, (1LL * B * T * nslab + target - 1) / target);
    int rpt = int(std::min<long long>(64, (rows_per_block + R - 1) / R));
    rpt = std::max(GN_CHUNK, (rpt + GN_CHUNK - 1) / GN_CHUNK * GN_CHUNK);
    const int runs = int(nblocks(T, size_t(R) * rpt));
    const dim3 grid(unsigned(B * runs), unsigned(nslab));
    if (sq) {
        // ss accumulates onto the records' value, as the reference's k_gn_stats2 does (src/kernels.cu:201):
        // gn_init / k_gn_stats1 zero it
        hipLaunchKernelGGL(gn_reduce_kernel<true>, grid, dim3(GN_THREADS), 0, st, X, T, C, groups, qs, rpt, runs, gs);
    } else {
        hipLaunchKernelGGL(gn_reduce_kernel<false>, grid, dim3(GN_THREADS), 0, st, X, T, C, groups, qs, rpt, runs, gs);
    }
    return hipGetLastError();
}
hipError_t launch_gn_apply(hipStream_t st, const int32_t* X, int B, int T, int C, int groups, const GnStat* gs, const i64* g, const i64* beta, int32_t* Y) {
    const size_t tot = size_t(B) * T * C;
    hipLaunchKernelGGL(gn_apply_kernel, dim3(std::min<unsigned>(nblocks(tot, 256), 65536u)), dim3(256), 0, st, X, B, T, C, groups, gs, g, beta, Y);
    return hipGetLastError();
}

// Tile shape of the row kernels: RT in {1, 2, 4, 8} rows (at most rt_max) of 64 / RT lanes each, and
// the NV template whose slots the row's C / 4 quads fill best (ties to the smaller RT).
static void tile_shape(int C, int rt_max, int& RT, int& NV) {
    const int Q = C / 4;
    double best = -1.0;
    RT = 1;
    NV = 10;
    for (int rt = 1; rt <= 8 && rt <= rt_max; rt *= 2) {
        const int lr = 64 / rt, slots = (Q + lr - 1) / lr;
        const int nv = slots <= 2 ? 2 : (slots <= 5 ? 5 : (slots <= 10 ? 10 : 0));
        if (!nv) continue;
        const double util = double(Q) / (double(lr) * nv);
        if (util > best + 1e-9) { best = util; RT = rt; NV = nv; }
    }
}

// tiles per block: about 32 rows, and for the GroupNorm apply at most 6 T + 1 so that a block's rows
// span at most GN_SLOTS samples (n consecutive rows span at most ceil((n - 1) / T) + 1 samples)
static int tiles_per_block(int RT, long long row_cap) { return int(std::max<long long>(1, std::min<long long>(32, row_cap) / RT)); }

hipError_t launch_gn_apply_row(hipStream_t st, const int32_t* X, int M, int T, int C, int groups, const GnStat* gs, const int32_t* g, const int32_t* beta,
                               const int32_t* Lsig, int32_t* Y, uint32_t* pm, int8_t* hi, int8_t* lo, int32_t* e, int Kp) {
    int RT, NV;
    tile_shape(C, int(std::min<long long>(8, 6LL * T + 1)), RT, NV);
    const int tpb = tiles_per_block(RT, 6LL * T + 1);
    const GnApplyArgs a{X, M, T, C, groups, RT, tpb, gs, g, beta, Y, pm, hi, lo, e, Kp};
    const dim3 grid(nblocks(nblocks(M, RT), tpb));
    const size_t lds = sizeof(NormK) * GN_SLOTS * GN_MAXG + 2 * sizeof(int32_t) * C + (Lsig ? sizeof(int32_t) * LUT_N : 0);
#define VK_GNA(N, V) hipLaunchKernelGGL((gn_apply_row_kernel<N, V>), grid, dim3(256), lds, st, a, Lsig)
    if (hi) {
        if (NV == 2) VK_GNA(2, true);
        else if (NV == 5) VK_GNA(5, true);
        else VK_GNA(10, true);
    } else {
        if (NV == 2) VK_GNA(2, false);
        else if (NV == 5) VK_GNA(5, false);
        else VK_GNA(10, false);
    }
#undef VK_GNA
    return hipGetLastError();
}

hipError_t launch_lnorm(hipStream_t st, bool q, const int32_t* X, int M, int C, const void* g, const void* beta, i64 den, int32_t* Y, int8_t* hi, int8_t* lo,
                        int32_t* e, int Kp) {
    LnEps eps;
    for (int ex = 0; ex < 13; ++ex) eps.v[ex] = ((1LL << (32 - 2 * ex)) + den / 2) / den;   // positive operands: the quotient is the floor
    int RT, NV;
    tile_shape(C, 8, RT, NV);
    const int tpb = tiles_per_block(RT, 32);
    const dim3 grid(nblocks(nblocks(M, RT), tpb));
    const size_t lds = q ? 2 * sizeof(int32_t) * C : 0;
#define VK_LNORM(N, QQ) hipLaunchKernelGGL((lnorm_kernel<N, QQ>), grid, dim3(256), lds, st, X, M, C, RT, tpb, g, beta, eps, Y, hi, lo, e, Kp)
    if (q) {
        if (NV == 2) VK_LNORM(2, true);
        else if (NV == 5) VK_LNORM(5, true);
        else VK_LNORM(10, true);
    } else {
        if (NV == 2) VK_LNORM(2, false);
        else if (NV == 5) VK_LNORM(5, false);
        else VK_LNORM(10, false);
    }
#undef VK_LNORM
    return hipGetLastError();
}

}  // namespace vk

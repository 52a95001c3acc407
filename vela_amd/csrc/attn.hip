// Exact integer attention for gfx950 and its operand producers, bit-exact with the reference's
// fused attention (src/attn.cu:1-6, whose unfused form is src/kernels.cu:673-722) and its operand
// kernels (src/kernels.cu:611-672,799-805). Heads of 64 values, G = B * heads groups.
//
// Semantics per query row q of group g, over the valid keys k (k < Tk, and k <= q when causal):
//   S = sum_d Q_d K_d (Q, K the int16 values of the planes: 256 hi + lo + 128)
//   s = rshr(S, 19 - eq - ek); mx = max s; E = lutexp(mx - s); sumE = sum E; r = floor(2^62 / sumE)
//   P = min(32767, (E r + 2^46) >> 47); O_d = sum_k P_k V_kd; out = rshr(O, 15 - ev_d)
//
// Design. A block owns 64 queries of one group, a wave 16 of them with their Q fragments in
// registers, and makes three passes over the key tiles (64 keys each): the row maximum, the sum of
// E, then P and P.V -- recomputing the scores each pass instead of storing them, so nothing of size
// Tq x Tk touches memory and the row statistics stay in registers. Scores are 16x16x64 int8 MFMAs of
// the signed planes (hh, hl + lh, ll) with the unsigned-offset terms restored from the query's plane
// sums and the key's value sum: S = 65536 hh + 256 (hl + lh) + ll + 32768 qhs + 128 qls + 128 ksum,
// assembled exactly in double (every term an integer below 2^37). A wave's 16 queries x 16 keys of
// a subtile land four queries per lane and one key per lane of a 16-lane row, so the per-query max
// and sum over keys are in-row DPP reductions. P goes to LDS as two signed planes (P >> 8 and
// (P & 255) - 128) and returns as the B operand of the P.V MFMAs against the transposed V planes;
// the plane offsets come back through the sum of P per query and the sum of V per dimension.
#include <climits>

#include "attn.h"

namespace vk {

namespace {

constexpr int AT_Q = 64;      // queries per block (16 per wave)
constexpr int AT_K = 64;      // keys per tile
constexpr int PSTRIDE = 80;   // LDS row stride of a P plane (bytes)

__device__ __forceinline__ v4i ld16(const int8_t* p) { return *reinterpret_cast<const v4i*>(p); }

__device__ __forceinline__ double clampd32(double v) { return fmin(fmax(v, -2147483648.0), 2147483647.0); }

// reductions over the 16 lanes of a DPP row (the lanes that share a query in the score layout)
template <int CTRL>
__device__ __forceinline__ int dpp(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
__device__ __forceinline__ int row16_max(int v) {
    v = max(v, dpp<0xB1>(v));
    v = max(v, dpp<0x4E>(v));
    v = max(v, dpp<0x141>(v));
    return max(v, dpp<0x140>(v));
}
__device__ __forceinline__ double dppd(double v, int which) {
    const u64 b = __builtin_bit_cast(u64, v);
    int lo = int(b), hi = int(b >> 32);
    switch (which) {
    case 0: lo = dpp<0xB1>(lo); hi = dpp<0xB1>(hi); break;
    case 1: lo = dpp<0x4E>(lo); hi = dpp<0x4E>(hi); break;
    case 2: lo = dpp<0x141>(lo); hi = dpp<0x141>(hi); break;
    default: lo = dpp<0x140>(lo); hi = dpp<0x140>(hi); break;
    }
    return __builtin_bit_cast(double, (u64(unsigned(hi)) << 32) | unsigned(lo));
}
__device__ __forceinline__ double row16_sum(double v) {
    v += dppd(v, 0);
    v += dppd(v, 1);
    v += dppd(v, 2);
    return v + dppd(v, 3);
}

// floor(2^62 / s) for an integer-valued double 0 < s < 2^53: a double estimate, then exact
// corrections on the 64-bit remainder
__device__ __forceinline__ u64 recip62(double s) {
    const u64 d = u64(s);
    u64 q = u64(0x1p62 / s);
    const u64 N = u64(1) << 62;
    while (q * d > N) --q;
    while (N - q * d >= d) ++q;
    return q;
}

struct LutE {
    double v, slope;   // L[i], (L[i + 1] - L[i]) * 2^-10
};

// Orders a wave's LDS writes before its later LDS reads of them (a wave's LDS instructions execute
// in order; this keeps the compiler from moving them).
__device__ __forceinline__ void wave_order_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace

// grid (Tqp / 64, G), 256 threads. SMALL: at most two key tiles (Tkp <= 128, cross-attention): the
// first pass keeps the rounded scores in registers and the other two passes reuse them.
template <bool SMALL>
__global__ void __launch_bounds__(256) attn_kernel(const AttnArgs a) {
    __shared__ LutE s_lut[1024];
    __shared__ __attribute__((aligned(16))) int8_t s_p[4][2][16 * PSTRIDE];   // per wave: P planes [query][key]
    __shared__ int s_red[4][64 + 16];                                         // per wave: sum of V per dimension, sum of P per query
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int fr = lane & 15, fg = lane >> 4;
    const int g = blockIdx.y, q0 = blockIdx.x * AT_Q;
    const int b = g / a.heads, h = g - b * a.heads;

    // exp table (src/attn.cu:85-91): entry i and the slope to entry i + 1, scaled by 2^-10
    for (int i = tid; i < 1024; i += 256) {
        const long long l0 = a.Lexp[i], l1 = a.Lexp[i + 1];
        s_lut[i] = LutE{double(l0), double(l1 - l0) * 0x1p-10};
    }

    // this wave's queries: Q fragment rows (A operand) and, in the score layout, queries 4 fg + j
    const size_t qrow = size_t(g) * a.Tqp + q0 + 16 * wave;
    const v4i qa_h = ld16(a.qh + (qrow + fr) * 64 + 16 * fg), qa_l = ld16(a.ql + (qrow + fr) * 64 + 16 * fg);
    double cq[4];
    int shq[4], qpos[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const size_t r = qrow + 4 * fg + j;
        cq[j] = 32768.0 * double(a.qhs[r]) + 128.0 * double(a.qls[r]);
        shq[j] = 19 - a.eq[r];
        qpos[j] = q0 + 16 * wave + 4 * fg + j;
    }
    __syncthreads();

    const int nT = a.Tkp / AT_K;
    // the key is valid for the query: inside the keys, and not after the query when causal
    auto valid = [&](int kt, int ks, int j) -> bool {
        const int key = kt * AT_K + 16 * ks + fr;
        return key < a.Tk && !(a.causal && key > qpos[j]);
    };
    // scores of key tile kt: sv[ks][j] for query 4 fg + j and key 16 ks + fr of the tile (any value
    // where the key is not valid)
    auto scores = [&](int kt, int (&sv)[4][4]) {
        const int k0 = kt * AT_K;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const size_t krow = size_t(g) * a.Tkp + k0 + 16 * ks + fr;
            const v4i kb_h = ld16(a.kh + krow * 64 + 16 * fg), kb_l = ld16(a.kl + krow * 64 + 16 * fg);
            v4i hh = v4i{0, 0, 0, 0}, hl = v4i{0, 0, 0, 0}, ll = v4i{0, 0, 0, 0};
            hh = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa_h, kb_h, hh, 0, 0, 0);
            hl = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa_h, kb_l, hl, 0, 0, 0);
            hl = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa_l, kb_h, hl, 0, 0, 0);
            ll = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa_l, kb_l, ll, 0, 0, 0);
            const int ekk = a.ek[krow];
            const double k128 = 128.0 * double(a.ksum[krow]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // |hl| <= 2^21, |ll| <= 2^20: T fits int32; S below 2^37 is exact in double
                const int T = (hl[j] << 8) + ll[j];
                const double S = fma(double(hh[j]), 65536.0, double(T) + (cq[j] + k128));
                sv[ks][j] = int(clampd32(floor(ldexp(S, ekk - shq[j]) + 0.5)));   // rshr(S, 19 - eq - ek), saturated
            }
        }
    };
    // E = lutexp(mx - s) (src/attn.cu:85-91) as an integer-valued double: exact for tables of
    // int32 entries (products below 2^42)
    auto lutE = [&](unsigned z) -> double {
        const unsigned zc = z < (1u << 20) ? z : (1u << 20) - 1;
        const LutE e = s_lut[zc >> 10];
        const double v = e.v + floor(e.slope * double(zc & 1023u));
        return z < (1u << 20) ? v : 0.0;
    };

    // the scores of tile kt: recomputed, or (SMALL) the ones pass 0 kept
    constexpr int NKEEP = SMALL ? 2 : 1;
    int keep[NKEEP][4][4];
    auto tile_scores = [&](int kt, int (&sv)[4][4]) __attribute__((always_inline)) {
        if constexpr (SMALL) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int j = 0; j < 4; ++j) sv[ks][j] = kt ? keep[NKEEP - 1][ks][j] : keep[0][ks][j];
        } else {
            scores(kt, sv);
        }
    };

    // ---- pass 0: the row maximum
    int mx[4] = {INT_MIN, INT_MIN, INT_MIN, INT_MIN};
    for (int kt = 0; kt < nT; ++kt) {
        int sv[4][4];
        scores(kt, sv);
        if constexpr (SMALL) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (kt == 0) keep[0][ks][j] = sv[ks][j];
                    else keep[NKEEP - 1][ks][j] = sv[ks][j];
                }
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (valid(kt, ks, j)) mx[j] = max(mx[j], sv[ks][j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) mx[j] = row16_max(mx[j]);

    // ---- pass 1: sum of E, then r = floor(2^62 / sumE) (0 for sumE <= 0)
    double se[4] = {0.0, 0.0, 0.0, 0.0};
    for (int kt = 0; kt < nT; ++kt) {
        int sv[4][4];
        tile_scores(kt, sv);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (valid(kt, ks, j)) se[j] += lutE(unsigned(mx[j]) - unsigned(sv[ks][j]));
    }
    u64 rr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        se[j] = row16_sum(se[j]);
        rr[j] = se[j] > 0.0 ? recip62(se[j]) : 0;
    }

    // ---- pass 2: P (two signed planes through LDS) and P.V
    v4i ohh[4], ohl[4], oll[4];
    int vsum_p[4] = {0, 0, 0, 0};   // sum over this lane's keys of 256 vh + vl, dimension 16 ds + fr
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) { ohh[ds] = v4i{0, 0, 0, 0}; ohl[ds] = v4i{0, 0, 0, 0}; oll[ds] = v4i{0, 0, 0, 0}; }
    int psum[4] = {0, 0, 0, 0};
    int8_t* ph = s_p[wave][0];
    int8_t* pl = s_p[wave][1];
    for (int kt = 0; kt < nT; ++kt) {
        const int k0 = kt * AT_K;
        int sv[4][4];
        tile_scores(kt, sv);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int P = 0;
                if (valid(kt, ks, j)) {
                    const double E = lutE(unsigned(mx[j]) - unsigned(sv[ks][j]));
                    if (E > 0.0) {
                        const u64 pp = (u64(E) * rr[j] + (u64(1) << 46)) >> 47;   // (E r + 2^46) >> 47 mod 2^64
                        P = pp > 32767u ? 32767 : int(pp);
                    }
                }
                psum[j] += P;
                const int o = (4 * fg + j) * PSTRIDE + 16 * ks + fr;
                ph[o] = int8_t(P >> 8);
                pl[o] = int8_t((P & 255) - 128);
            }
        wave_order_lds();
        const v4i pb_h = *reinterpret_cast<const v4i*>(ph + fr * PSTRIDE + 16 * fg);
        const v4i pb_l = *reinterpret_cast<const v4i*>(pl + fr * PSTRIDE + 16 * fg);
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) {
            const size_t vrow = (size_t(g) * 64 + 16 * ds + fr) * a.Tkp + k0 + 16 * fg;
            const v4i va_h = ld16(a.vth + vrow), va_l = ld16(a.vtl + vrow);
            ohh[ds] = __builtin_amdgcn_mfma_i32_16x16x64_i8(va_h, pb_h, ohh[ds], 0, 0, 0);
            ohl[ds] = __builtin_amdgcn_mfma_i32_16x16x64_i8(va_h, pb_l, ohl[ds], 0, 0, 0);
            ohl[ds] = __builtin_amdgcn_mfma_i32_16x16x64_i8(va_l, pb_h, ohl[ds], 0, 0, 0);
            oll[ds] = __builtin_amdgcn_mfma_i32_16x16x64_i8(va_l, pb_l, oll[ds], 0, 0, 0);
            int sh = 0, sl = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                sh = __builtin_amdgcn_sdot4(va_h[c], 0x01010101, sh, false);
                sl = __builtin_amdgcn_sdot4(va_l[c], 0x01010101, sl, false);
            }
            vsum_p[ds] += 256 * sh + sl;
        }
        wave_order_lds();   // the P planes are read before the next tile writes them
    }

    // ---- sums for the plane offsets: P per query (score layout), V per dimension (over the four key chunks)
    int* red = s_red[wave];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = int(row16_sum(double(psum[j])));
        if (fr == 0) red[64 + 4 * fg + j] = t;
    }
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
        int v = vsum_p[ds];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (fg == 0) red[16 * ds + fr] = v;
    }
    wave_order_lds();

    // ---- output: lane holds dimensions 16 ds + 4 fg + j of query fr of the wave
    // O = 65536 hh + 256 (hl + lh) + ll + 128 (sum P) + 128 (sum of 256 vh + vl), below 2^43: exact in double
    const int qi = 16 * wave + fr, q = q0 + qi;
    const double p128 = 128.0 * double(red[64 + fr]);
    uint32_t am = 0;
    int32_t* orow = a.out + (size_t(b) * a.Tq + (q < a.Tq ? q : 0)) * a.C + h * 64;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
        int o4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = 16 * ds + 4 * fg + j;
            const double O = fma(double(ohh[ds][j]), 65536.0, fma(double(ohl[ds][j]), 256.0, double(oll[ds][j]))) + (p128 + 128.0 * double(red[d]));
            const int e = a.ev[g * 64 + d];
            o4[j] = int(clampd32(floor(ldexp(O, e - 15) + 0.5)));   // rshr(O, 15 - ev), saturated
            am = max(am, uabs(o4[j]));
        }
        if (q < a.Tq) *reinterpret_cast<int4*>(orow + 16 * ds + 4 * fg) = make_int4(o4[0], o4[1], o4[2], o4[3]);
    }
    if (a.rowmax) {
        am = max(am, uint32_t(__shfl_xor(int(am), 16)));
        am = max(am, uint32_t(__shfl_xor(int(am), 32)));
        if (fg == 0 && q < a.Tq && am) atomicMax(a.rowmax + size_t(b) * a.Tq + q, am);
    }
}

// ---------------------------------------------------------------- operands

// src/kernels.cu:611-631 (k_quant_heads): one wave per (g, t) row of 64 values, lane d owning value d
__global__ void __launch_bounds__(256) quant_heads_kernel(const int32_t* __restrict__ X, int B, int T, int C, int heads, int Tp, int8_t* __restrict__ hi,
                                                          int8_t* __restrict__ lo, int32_t* __restrict__ e, long long* __restrict__ hs,
                                                          long long* __restrict__ ls, long long* __restrict__ tsum) {
    const int lane = threadIdx.x & 63;
    const long long w = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int G = B * heads;
    if (w >= (long long)G * Tp) return;
    const int g = int(w / Tp), t = int(w - (long long)g * Tp), b = g / heads, h = g - b * heads;
    const size_t o = size_t(w) * 64 + lane;
    if (t >= T) {
        hi[o] = 0;
        lo[o] = -128;
        if (lane == 0) { e[w] = 0; hs[w] = 0; ls[w] = -128 * 64; tsum[w] = 0; }
        return;
    }
    const int x = X[(size_t(b) * T + t) * C + h * 64 + lane];
    uint32_t m = uabs(x);
#pragma unroll
    for (int s = 32; s; s >>= 1) m = max(m, uint32_t(__shfl_xor(int(m), s)));
    const int ee = rowexp_u32(m);
    const int q = quant16_32(x, ee);
    const int hv = q >> 8, lv = (q & 255) - 128;
    hi[o] = int8_t(hv);
    lo[o] = int8_t(lv);
    int sh = hv, sl = lv, st = q;
#pragma unroll
    for (int s = 32; s; s >>= 1) { sh += __shfl_xor(sh, s); sl += __shfl_xor(sl, s); st += __shfl_xor(st, s); }
    if (lane == 0) { e[w] = ee; hs[w] = sh; ls[w] = sl; tsum[w] = st; }
}

// src/kernels.cu:799-805: rows t in [T, Tp) of every group take the value 0
__global__ void __launch_bounds__(256) quant_heads_pad_kernel(int G, int T, int Tp, int8_t* __restrict__ hi, int8_t* __restrict__ lo, int32_t* __restrict__ e,
                                                              long long* __restrict__ hs, long long* __restrict__ ls, long long* __restrict__ tsum) {
    const int lane = threadIdx.x & 63, npad = Tp - T;
    const long long w = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= (long long)G * npad) return;
    const int g = int(w / npad);
    const size_t row = size_t(g) * Tp + T + (w - (long long)g * npad);
    hi[row * 64 + lane] = 0;
    lo[row * 64 + lane] = -128;
    if (lane == 0) { e[row] = 0; hs[row] = 0; ls[row] = -128 * 64; tsum[row] = 0; }
}

// src/kernels.cu:632-650 (k_quant_v, exponents): one block per group, thread (d, slice) scanning
// rows slice, slice + 4, ...; ev = row_exp(max |x|) per dimension; vsum cleared for the write pass
__global__ void __launch_bounds__(256) quant_v_exp_kernel(const int32_t* __restrict__ X, int Tk, int C, int heads, int32_t* __restrict__ ev,
                                                          long long* __restrict__ vsum) {
    __shared__ uint32_t s_m[4][64];
    const int g = blockIdx.x, b = g / heads, h = g - b * heads, d = threadIdx.x & 63, sl = threadIdx.x >> 6;
    const int32_t* x = X + size_t(b) * Tk * C + h * 64 + d;
    uint32_t m = 0;
    for (int t = sl; t < Tk; t += 4) m = max(m, uabs(x[size_t(t) * C]));
    s_m[sl][d] = m;
    __syncthreads();
    if (sl == 0) {
        m = max(max(s_m[0][d], s_m[1][d]), max(s_m[2][d], s_m[3][d]));
        ev[g * 64 + d] = rowexp_u32(m);
        vsum[g * 64 + d] = 0;
    }
}

// src/kernels.cu:651-672 (k_quant_v, transposed write): block per (64-row tile, group): the tile in
// LDS, then thread (d, quarter) quantises 16 consecutive rows of dimension d, writes them as 16
// bytes of each plane of vt[g * 64 + d], and adds its part of vsum
__global__ void __launch_bounds__(256) quant_v_write_kernel(const int32_t* __restrict__ X, int Tk, int C, int heads, int Tkp,
                                                            const int32_t* __restrict__ ev, int8_t* __restrict__ vth, int8_t* __restrict__ vtl,
                                                            long long* __restrict__ vsum) {
    __shared__ int32_t tile[64][65];
    __shared__ long long s_s[4][64];
    const int g = blockIdx.y, t0 = blockIdx.x * 64, b = g / heads, h = g - b * heads;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < 64; r += 4) {
        const int t = t0 + r;
        tile[r][tx] = t < Tk ? X[(size_t(b) * Tk + t) * C + h * 64 + tx] : 0;
    }
    __syncthreads();
    const int d = threadIdx.x >> 2, qt = threadIdx.x & 3;
    const int e = ev[g * 64 + d];
    unsigned hw[4], lw[4];
    long long s = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        unsigned hv = 0, lv = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int r = 16 * qt + 4 * c + k;
            const int q = t0 + r < Tk ? quant16_32(tile[r][d], e) : 0;
            s += q;
            hv |= unsigned(q >> 8 & 255) << (8 * k);
            lv |= unsigned(((q & 255) - 128) & 255) << (8 * k);
        }
        hw[c] = hv;
        lw[c] = lv;
    }
    const size_t o = (size_t(g) * 64 + d) * Tkp + t0 + 16 * qt;
    *reinterpret_cast<v4i*>(vth + o) = v4i{int(hw[0]), int(hw[1]), int(hw[2]), int(hw[3])};
    *reinterpret_cast<v4i*>(vtl + o) = v4i{int(lw[0]), int(lw[1]), int(lw[2]), int(lw[3])};
    s_s[qt][d] = s;
    __syncthreads();
    if (threadIdx.x < 64) {
        const long long t = s_s[0][threadIdx.x] + s_s[1][threadIdx.x] + s_s[2][threadIdx.x] + s_s[3][threadIdx.x];
        atomicAdd(reinterpret_cast<unsigned long long*>(vsum + g * 64 + threadIdx.x), (unsigned long long)t);
    }
}

// ---------------------------------------------------------------- launchers

hipError_t launch_attention(hipStream_t st, const AttnArgs& a, int G) {
    if (a.Tkp <= 2 * AT_K) hipLaunchKernelGGL(attn_kernel<true>, dim3(unsigned(a.Tqp / AT_Q), unsigned(G)), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(attn_kernel<false>, dim3(unsigned(a.Tqp / AT_Q), unsigned(G)), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_quant_heads(hipStream_t st, const int32_t* X, int B, int T, int C, int heads, int Tp, int8_t* hi, int8_t* lo, int32_t* e, long long* hs,
                              long long* ls, long long* tsum) {
    const long long rows = (long long)B * heads * Tp;
    hipLaunchKernelGGL(quant_heads_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, st, X, B, T, C, heads, Tp, hi, lo, e, hs, ls, tsum);
    return hipGetLastError();
}

hipError_t launch_quant_heads_pad(hipStream_t st, int G, int T, int Tp, int8_t* hi, int8_t* lo, int32_t* e, long long* hs, long long* ls, long long* tsum) {
    const long long rows = (long long)G * (Tp - T);
    hipLaunchKernelGGL(quant_heads_pad_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, st, G, T, Tp, hi, lo, e, hs, ls, tsum);
    return hipGetLastError();
}

hipError_t launch_quant_v(hipStream_t st, const int32_t* X, int B, int Tk, int C, int heads, int Tkp, int8_t* vth, int8_t* vtl, int32_t* ev, long long* vsum) {
    const int G = B * heads;
    hipLaunchKernelGGL(quant_v_exp_kernel, dim3(unsigned(G)), dim3(256), 0, st, X, Tk, C, heads, ev, vsum);
    hipLaunchKernelGGL(quant_v_write_kernel, dim3(unsigned(Tkp / 64), unsigned(G)), dim3(256), 0, st, X, Tk, C, heads, Tkp, ev, vth, vtl, vsum);
    return hipGetLastError();
}

}  // namespace vk

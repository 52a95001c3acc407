// The W8A16 hi/lo-split GEMM kernels for gfx950 (CDNA4), templated on the A source, the epilogue
// and the tile shape. Each source file gemm_src_*.hip instantiates them for one source.
//
// Arithmetic: the int16 activation q = 256*hi + lo + 128 is split into a signed hi byte and an
// offset lo byte (lo - 128 = (q & 255) ^ 0x80) with byte permutes; both planes run through
// v_mfma_i32_16x16x64_i8 against the same W fragment (W is the MFMA's A operand, the activations its
// B operand, so each lane ends up holding four consecutive output columns of one output row).
//
// Two main loops:
//  * gemm_dma_kernel (int8 planes, int16 rows, int16 NHWC image, plain int8 GEMM): every operand
//    byte goes HBM -> LDS by buffer_load ... lds into a ring of LDS stages, two K steps ahead of the
//    MFMAs, with no register staging; out-of-range offsets read as zero (pad rows/columns and the
//    image border of the implicit im2col cost no branches). int16 data sits raw in LDS and is split
//    (and for the image source clamped/quantised) as each MFMA fragment is read. Waves are stacked
//    along M (4 x 1), so each activation row is split once per block and its row maximum is
//    complete inside one wave.
//  * gemm_hl_kernel (int32 rows, int32 NHWC image): register-staged loads, quantise + split at the
//    LDS store, double-buffered.
//
// Epilogue: acc = 256*Chi + Clo + 128*wsum, y = sat32(rshr(acc*m, s-e) + b) (src/gemm_hl.cu:40-52).
// When the block's columns satisfy Kp*|m| < 2^30 (so |acc*m| < 2^52) and every shift s-e lies in
// [1, 52], it runs in FP64, where it is exact: acc*m*2^-(s-e) + 1/2 is a dyadic rational with a
// numerator below 2^53, one FMA produces it without rounding, and floor() then gives the rounding
// shift. Otherwise it runs the reference's int64 formula element by element.
#pragma once
#include <climits>
#include <type_traits>

#include "vk_common.h"

namespace vk {

template <int BM_, int BN_, int WM_, int WN_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
    static constexpr int WTM = BM / WM, WTN = BN / WN;   // wave sub-tile (rows x columns)
    static constexpr int MS = WTM / 16, NS = WTN / 16;   // 16x16 MFMA tiles per wave
    static constexpr int WT = BN * 4 / 256;              // 16-byte W chunks per thread per K step (register path)
    static constexpr int AT = BM * 4 / 256;              // 16-value A chunks per thread per K step (register path)
    static constexpr int STAGE = (BN + 2 * BM) * 64;     // LDS bytes per stage: W, hi, lo planes
    static constexpr int NW = WM * WN;                   // waves per block
    static constexpr int NT = 64 * NW;                   // threads per block
    static_assert(NW == 4 || NW == 8, "four or eight waves");
    static_assert(MS >= 1 && NS >= 2 && (NS % 2) == 0, "wave tile");
};

// register-path tiles (waves 2 x 2 / 1 x 4)
typedef Tile<128, 128, 2, 2> TileV0;
typedef Tile<64, 128, 1, 4> TileV1;
typedef Tile<128, 64, 2, 2> TileV2;
// DMA-path tiles (waves stacked along M)
typedef Tile<128, 128, 4, 1> TileD0;
typedef Tile<64, 128, 4, 1> TileD1;
typedef Tile<128, 64, 4, 1> TileD2;
// eight waves, 4 x 2: each A stripe feeds 256 columns (half the A traffic of 128-column tiles)
typedef Tile<128, 256, 4, 2> TileD3;

// LDS layouts of the K-step tiles. A fragment load (ds_read_b128) has each group of 16 lanes read
// one 16-byte chunk of 16 consecutive rows. Measured on gfx950 (a probe with SQ_LDS_BANK_CONFLICT):
// 128-byte rows under swz16 read conflict-free, while 64-byte rows under any XOR swizzle of their
// four chunks cost four conflict cycles per instruction (the load takes twice as long).
//
// Byte offset of 16-byte chunk `chunk` (0..3) of a 64-byte LDS row, XOR-swizzled (the register-staged
// kernel, which writes its tiles from registers)
__device__ __forceinline__ int swz(int row, int chunk) { return row * 64 + ((chunk ^ (((row >> 1) + (row >> 3)) & 3)) << 4); }
// byte offset of 16-byte chunk `chunk` (0..7) of a 128-byte LDS row (raw int16 activations): conflict-free
__device__ __forceinline__ int swz16(int row, int chunk) { return row * 128 + ((chunk ^ ((row & 7) ^ ((row >> 3) & 1))) << 4); }
// 64-byte rows (W, int8 planes) stored in pairs as 128-byte rows under swz16: chunk c (0..3) of row r
// is chunk 4 (r & 1) + c of LDS row r / 2. The DMA still reads two whole 64-byte rows per 8 lanes.
__device__ __forceinline__ int pswz(int row, int chunk) { return swz16(row >> 1, 4 * (row & 1) + chunk); }
// byte offset of 16-byte chunk `chunk` (0..15) of a 256-byte LDS row (raw int32 image values): the 16
// rows read together by one fragment load hit 16 distinct chunk positions
__device__ __forceinline__ int swz32(int row, int chunk) { return row * 256 + ((chunk ^ (row & 15)) << 4); }
__device__ __forceinline__ int swz_key(int row) { return ((row >> 1) + (row >> 3)) & 3; }
__device__ __forceinline__ int swz16_key(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// LDS row of W-tile row `row`. For GEGLU the a-columns (even) go to the first half and the
// g-columns (odd) to the second half, so a wave's a- and g-subtiles hold matching columns.
template <int EPI, int BN>
__device__ __forceinline__ int wrow_lds(int row) {
    if constexpr (EPI == EPI_GEGLU) return (row & 1) ? (BN / 2 + (row >> 1)) : (row >> 1);
    else return row;
}
// inverse: W-tile row stored at LDS row `lr`
template <int EPI, int BN>
__device__ __forceinline__ int wrow_of_lds(int lr) {
    if constexpr (EPI == EPI_GEGLU) return lr < BN / 2 ? 2 * lr : 2 * (lr - BN / 2) + 1;
    else return lr;
}

// first LDS row of MFMA column-subtile ns of wave column wn
template <int EPI, class T>
__device__ __forceinline__ int wsub_row(int wn, int ns) {
    if constexpr (EPI == EPI_GEGLU) {
        constexpr int H = T::NS / 2;
        return ns < H ? (wn * H + ns) * 16 : T::BN / 2 + (wn * H + ns - H) * 16;
    } else {
        return (wn * T::NS + ns) * 16;
    }
}

// four int16 pairs (d[0..7], two per dword) -> 16 hi bytes and 16 offset lo bytes
__device__ __forceinline__ void split16x16(const unsigned* d, v4i& h, v4i& l) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h[j] = int(__builtin_amdgcn_perm(d[2 * j + 1], d[2 * j], 0x07050301u));
        l[j] = int(__builtin_amdgcn_perm(d[2 * j + 1], d[2 * j], 0x06040200u) ^ 0x80808080u);
    }
}

// quant16_32(v, e) for e in [0, 17] in four VALU instructions, from sh1 = max(e - 1, 0) and
// c1 = (e > 0): the rounding shift as ((v >> (e - 1)) + 1) >> 1, which equals (v >> e) +
// ((v >> (e - 1)) & 1) for e >= 1 because floor shifts compose (v >> e = (v >> (e - 1)) >> 1); the
// add saturates, so that its one overflowing case (e = 1, v = INT_MAX) still clamps to 32767 as the
// reference's form does; e = 0 leaves v as it is.
__device__ __forceinline__ int quant16_sh(int v, int sh1, int c1) {
    const int t = __builtin_elementwise_add_sat(v >> sh1, c1);
    return min(max(t >> c1, -32767), 32767);
}

// 16 int32 values quantised with shift e (quant16_32), packed to int16 pairs
__device__ __forceinline__ void quant_pack16(const v4i* x, int e, unsigned* d) {
    const int sh1 = e > 0 ? e - 1 : 0, c1 = e > 0 ? 1 : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q0 = quant16_sh(x[j >> 1][(2 * j) & 3], sh1, c1);
        const int q1 = quant16_sh(x[j >> 1][(2 * j + 1) & 3], sh1, c1);
        d[j] = __builtin_amdgcn_perm(unsigned(q1), unsigned(q0), 0x05040100u);
    }
}

// quant16_32(v, e) for 0 <= e <= 16 in three instructions: with r = 2^(e-1) (0 for e = 0),
// clamp(sat(v + r) >> e). Where v + r does not saturate, floor((v + r) / 2^e) is exactly
// (v >> e) + ((v >> (e-1)) & 1); where it does, both forms clamp to 32767 (INT_MAX >> e >= 32767
// for e <= 16). e = 17 (a row holding INT_MIN) keeps quant_pack16.
__device__ __forceinline__ void quant_pack16_e16(const v4i* x, int e, unsigned* d) {
    const int r = e > 0 ? 1 << (e - 1) : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q0 = min(max(__builtin_elementwise_add_sat(x[j >> 1][(2 * j) & 3], r) >> e, -32767), 32767);
        const int q1 = min(max(__builtin_elementwise_add_sat(x[j >> 1][(2 * j + 1) & 3], r) >> e, -32767), 32767);
        d[j] = __builtin_amdgcn_perm(unsigned(q1), unsigned(q0), 0x05040100u);
    }
}

// 16 int32 values quantised with shift 0 (quant16_32(v, 0) = v clamped to +-32767), packed to int16 pairs
__device__ __forceinline__ void clamp_pack16(const v4i* x, unsigned* d) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int a = min(max(x[j >> 1][(2 * j) & 3], -32767), 32767);
        const int b = min(max(x[j >> 1][(2 * j + 1) & 3], -32767), 32767);
        d[j] = __builtin_amdgcn_perm(unsigned(b), unsigned(a), 0x05040100u);
    }
}

// 16 int16 image values (two per dword, in place) quantised with shift 0: quant16_32(v, 0) =
// max(v, -32767) for int16 v
__device__ __forceinline__ void clamp16_pairs(unsigned* d) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const unsigned w = d[j];
        s2 v = __builtin_bit_cast(s2, w);
        v = __builtin_elementwise_max(v, s2{-32767, -32767});
        d[j] = __builtin_bit_cast(unsigned, v);
    }
}

// the same with any shift e in [0, 17] (quant16_32)
__device__ __forceinline__ void quant16_pairs(unsigned* d, int e) {
    const int sh1 = e > 0 ? e - 1 : 0, c1 = e > 0 ? 1 : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int w = int(d[j]);
        const int q0 = quant16_sh(int(short(w & 0xffff)), sh1, c1);
        const int q1 = quant16_sh(w >> 16, sh1, c1);
        d[j] = __builtin_amdgcn_perm(unsigned(q1), unsigned(q0), 0x05040100u);
    }
}

// ---------------------------------------------------------------- epilogue shared state

// GroupNorm accumulators of a block (EPI_PLAIN_GN only): [region][group]. A region is one
// gnBM x gnBN tile of the reference's GEMM (the granularity its statistics are flushed at); a
// block of at most 128 x 256 outputs holds at most 2 x 4 of them, region (tr, tc) at slot 4 tr + tc.
constexpr int GN_REGIONS = 8;
template <bool GN>
struct GnShared {};
template <>
struct GnShared<true> {
    long long gsum[GN_REGIONS][32];
    int gmin[GN_REGIONS][32], gmax[GN_REGIONS][32];
    int gm0;   // first output row of the block
};

// Per-block epilogue constants, GELU table and exactness flags, in LDS.
template <int BN, bool LUT, bool GN = false>
struct EpiShared : GnShared<GN> {
    double ms[BN];      // m * 2^-s
    double wm[BN];      // 128 * wsum * m * 2^-s; + 1/2 when e == 0, and + b as well when the block folds b
    int b[BN];
    int2 lut[LUT ? 2050 : 1];   // lut[i + 1] = (L[i], L[i+1] - L[i]); lut[0] below the table, lut[2049] above
    int4 wslot[8];      // per wave of the set-up: min e, max e, min s, max s over its rows / columns
    int wbits[8];       // per wave: bit 0 a column bound failed, bit 1 a table entry lies outside [0, 65536], bit 2 b not foldable
};

// GroupNorm statistics of a block (src/gemm_hl.cu:175-177, 285-287, 306-309). The reference gathers
// the sum, min and max of its tile's outputs per group and flushes them to
// GnStat[(tile row 0 / gnT) * 32 + group] only when the min is not INT_MAX, so a tile whose outputs
// of a group all saturated to INT_MAX adds nothing for that group. The statistics here are gathered
// per region = one such tile (the host picks a block shape made of whole regions and passes the
// reference's tile as gnBM x gnBN), cleared before the epilogue, fed by one LDS atomic per group and
// lane, and flushed by the same rule with one global atomic each.
template <class S>
__device__ __forceinline__ void gn_clear(const GemmParams& p, int m0, S& sh) {
    const int tid = threadIdx.x;
    if (tid < GN_REGIONS * 32) {
        sh.gsum[tid >> 5][tid & 31] = 0;
        sh.gmin[tid >> 5][tid & 31] = INT_MAX;
        sh.gmax[tid >> 5][tid & 31] = INT_MIN;
    }
    if (tid == 0) sh.gm0 = m0;
}

template <class S>
__device__ __forceinline__ void gn_flush(const GemmParams& p, S& sh) {
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < GN_REGIONS * 32) {
        const int slot = tid >> 5, g = tid & 31;
        if (sh.gmin[slot][g] != INT_MAX) {   // the reference's test: a region of INT_MAX values (or none) adds nothing
            const int r0 = sh.gm0 + (slot >> 2) * p.gnBM;   // the region's first row gives its sample
            GnStat* gs = p.gnstat + (r0 / p.gnT) * 32 + g;
            atomicAdd(reinterpret_cast<unsigned long long*>(&gs->sum), static_cast<unsigned long long>(sh.gsum[slot][g]));
            atomicMin(&gs->mn, sh.gmin[slot][g]);
            atomicMax(&gs->mx, sh.gmax[slot][g]);
        }
    }
}

struct EpiFlags {
    bool fast, ezero, fold;
};

// Shift of output row r (src/gemm_hl.cu:102,335-341): SRC_X32 from the row's maximum |x|; a
// convolution source given per-pixel maxima instead of an e vector takes k_conv_e's rule in-kernel
// (row_exp of the largest maximum over the in-bounds pixels of the row's 3x3 window, nine cached
// loads per row); otherwise e[r], or 0 without an e vector.
__device__ __forceinline__ int conv_window_shift(const GemmParams& p, int r) {
    const int HoWo = p.Ho * p.Wo;
    const int b = r / HoWo, pp = r - b * HoWo, oy = pp / p.Wo, ox = pp - oy * p.Wo;
    const int iy0 = oy * p.stride - 1, ix0 = ox * p.stride - 1;
    uint32_t m = 0;
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
        const int iy = iy0 + ky;
        if (iy < 0 || iy >= p.H) continue;
        const uint32_t* row = p.pm + (size_t(b) * p.H + iy) * p.W;
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
            const int ix = ix0 + kx;
            if (ix >= 0 && ix < p.W) m = max(m, row[ix]);
        }
    }
    return rowexp_u32(m);
}

template <int SRC>
__device__ __forceinline__ int row_shift(const GemmParams& p, int r) {
    if constexpr (SRC == SRC_X32) return rowexp_u32(p.xrowmax[r]);
    if constexpr (SRC == SRC_CONV32 || SRC == SRC_CONV16) {
        if (p.pm) return conv_window_shift(p, r);
    }
    return p.e ? p.e[r] : 0;
}

// Wave-wide minimum / maximum (every lane active): within each 16-lane row by DPP (xor 1, xor 2, the
// half-row mirror, the row mirror), then over the four rows by readlane.
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
__device__ __forceinline__ int wave_min_i32(int v) {
    v = min(v, dpp_i32<0xB1>(v));
    v = min(v, dpp_i32<0x4E>(v));
    v = min(v, dpp_i32<0x141>(v));
    v = min(v, dpp_i32<0x140>(v));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int wave_max_i32(int v) {
    v = max(v, dpp_i32<0xB1>(v));
    v = max(v, dpp_i32<0x4E>(v));
    v = max(v, dpp_i32<0x141>(v));
    v = max(v, dpp_i32<0x140>(v));
    return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// A thread's share of the block's exactness test: the shift range of its rows and columns and the
// failed tests of its columns and table entries. Each wave reduces its threads' shares and writes
// one slot; after a barrier every thread combines the slots (setup_flags).
struct SetupPart {
    int emn = INT_MAX, emx = INT_MIN, smn = INT_MAX, smx = INT_MIN;
    bool bad = false, lbad = false, nofold = false;
};
template <class S>
__device__ __forceinline__ void setup_publish(S& sh, const SetupPart& v) {
    const int emn = wave_min_i32(v.emn), emx = wave_max_i32(v.emx), smn = wave_min_i32(v.smn), smx = wave_max_i32(v.smx);
    const int bits = (__builtin_amdgcn_ballot_w64(v.bad) ? 1 : 0) | (__builtin_amdgcn_ballot_w64(v.lbad) ? 2 : 0) |
                     (__builtin_amdgcn_ballot_w64(v.nofold) ? 4 : 0);
    if ((threadIdx.x & 63) == 0) {
        sh.wslot[threadIdx.x >> 6] = make_int4(emn, emx, smn, smx);
        sh.wbits[threadIdx.x >> 6] = bits;
    }
}
// The block's forms from the waves' slots. fast: the FP64 form is exact for every element (columns
// with |m| Kp < 2^30 and |s| <= 1000, 1 <= s - e <= 52 for every row and column, the table in
// [0, 65536]); ezero: every row has e = 0; fold: also no element can saturate and b folds exactly
// into the FMA constant (every column with 2^22 Kp |m| 2^-s < 2^30, |b| < 2^30 and |b| 2^s < 2^51).
template <bool NEEDLUT, int NW, class S>
__device__ __forceinline__ EpiFlags setup_flags(const S& sh) {
    int emin = INT_MAX, emax = INT_MIN, smin = INT_MAX, smax = INT_MIN, bits = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const int4 q = sh.wslot[w];
        emin = min(emin, q.x); emax = max(emax, q.y); smin = min(smin, q.z); smax = max(smax, q.w);
        bits |= sh.wbits[w];
    }
    EpiFlags f;
    f.fast = !(bits & 1) && (i64(smin) - emax >= 1) && (i64(smax) - emin <= 52) && emin >= -1000 && emax <= 1000;
    if (NEEDLUT && (bits & 2)) f.fast = false;
    f.ezero = emin > emax || (emin == 0 && emax == 0);
    f.fold = f.fast && f.ezero && !(bits & 4);
    return f;
}

// a column's FP64 constants m 2^-s, 128 wsum m 2^-s and its share of the exactness test
__device__ __forceinline__ void setup_column(const GemmParams& p, const int4& c, double& ms, double& wmv, SetupPart& sp) {
    const i64 mag = (c.x < 0 ? -i64(c.x) : i64(c.x)) * i64(p.Kp);
    sp.bad |= mag >= (1LL << 30) || c.y < -1000 || c.y > 1000;
    sp.smn = min(sp.smn, c.y);
    sp.smx = max(sp.smx, c.y);
    if (c.y >= -1000 && c.y <= 1000) {
        ms = ldexp(double(c.x), -c.y);
        wmv = ldexp(128.0 * (double(c.w) * double(c.x)), -c.y);
        // |acc*m*2^-s| <= 2^22*Kp*|m|*2^-s, since |acc| <= 32768*128*Kp; with that below 2^30 and
        // |b| < 2^30 no element saturates; wm + 1/2 + b is exact when |b|*2^s < 2^51
        const double um = ldexp(4194304.0 * double(p.Kp) * fabs(double(c.x)), -c.y);
        sp.nofold |= !(um < 1073741824.0) || uabs(c.z) >= (1u << 30) || ldexp(fabs(double(c.z)), c.y) >= 2251799813685248.0;
    } else {
        ms = 0.0;
        wmv = 0.0;
    }
}

// Fill the epilogue constants of columns [n0, n0 + BN) (in LDS-row order) and decide whether the
// FP64 epilogue is exact for every element of this block.
template <int EPI, int SRC, int BM, int BN, class S>
__device__ __forceinline__ EpiFlags block_prologue(const GemmParams& p, int m0, int n0, S& sh) {
    constexpr bool NEEDLUT = EPI == EPI_GEGLU || EPI == EPI_GELU;
    const int tid = threadIdx.x;
    if constexpr (EPI == EPI_PLAIN_GN) {
        gn_clear(p, m0, sh);
        __syncthreads();
    }
    SetupPart sp;
    for (int i = tid; i < BM; i += 256) {
        const int r = m0 + i;
        if (r < p.Mreal) {
            const int er = row_shift<SRC>(p, r);
            sp.emn = min(sp.emn, er);
            sp.emx = max(sp.emx, er);
        }
    }
    for (int j = tid; j < BN; j += 256) {
        const int n = n0 + wrow_of_lds<EPI, BN>(j);
        double ms = 0.0, wmv = 0.0;
        int bb = 0;
        if (n < p.Nreal) {
            const int4 c = p.cst[n];
            setup_column(p, c, ms, wmv, sp);
            bb = c.z;
        }
        sh.ms[j] = ms; sh.wm[j] = wmv; sh.b[j] = bb;
    }
    if constexpr (NEEDLUT) {
        for (int i = tid; i < 2050; i += 256) {
            int2 v;
            if (i == 0) v = make_int2(0, 0);
            else if (i == 2049) v = make_int2(65536, 0);
            else {
                const int a = p.Lphi[i - 1], nx = p.Lphi[i];
                v = make_int2(a, nx - a);
                sp.lbad |= unsigned(a) > 65536u || unsigned(nx) > 65536u;
            }
            sh.lut[i] = v;
        }
    }
    setup_publish(sh, sp);
    __syncthreads();
    const EpiFlags f = setup_flags<NEEDLUT, 4>(sh);
    if (f.ezero) {
        // the FMA constant of the e == 0 forms: wm + 1/2, and + b when folded (exact, see above)
        for (int j = tid; j < BN; j += 256) sh.wm[j] = (sh.wm[j] + 0.5) + (f.fold ? double(sh.b[j]) : 0.0);
        __syncthreads();
    }
    return f;
}

// ---- the same set-up for a kernel that loads its inputs before the K loop and builds the
// tables after it, so that no load latency sits between the loads of the first K steps and the
// first MFMA: the cst entry of table column tid and the shift of tile row tid are held in
// registers (TilePre), and the GELU table arrives in LDS by DMA, raw, in the upper half of
// sh.lut, and is expanded to (L[i], L[i+1] - L[i]) pairs here.
struct TilePre {
    int4 c;
    int e;
    bool cok, eok;
    int m0;
};

template <int EPI, int SRC, int BM, int BN>
__device__ __forceinline__ TilePre load_tile_pre(const GemmParams& p, int m0, int n0) {
    // one table row and one table column per thread (blocks have at least max(BM, BN) threads)
    const int tid = threadIdx.x;
    TilePre t;
    const int n = n0 + wrow_of_lds<EPI, BN>(tid < BN ? tid : 0);
    t.cok = tid < BN && n < p.Nreal;
    t.c = t.cok ? p.cst[n] : make_int4(0, 0, 0, 0);
    const int r = m0 + tid;
    t.eok = tid < BM && r < p.Mreal;
    t.e = t.eok ? (row_shift<SRC>(p, r)) : 0;
    t.m0 = m0;
    return t;
}

// byte offset inside sh.lut of the raw table copy (entries 0..2047; entry 2048 comes in a register)
constexpr unsigned LUT_RAW_OFF = 8192;

template <int EPI, int SRC, int BM, int BN, int NT, class S>
__device__ __forceinline__ EpiFlags epi_setup(const GemmParams& p, const TilePre& t, int L2048, S& sh) {
    constexpr bool NEEDLUT = EPI == EPI_GEGLU || EPI == EPI_GELU;
    static_assert(NT >= BM && NT >= BN, "one table row and column per thread");
    const int tid = threadIdx.x;
    // ---- phase 1: everything that reads LDS or needs no LDS (the raw table is still in place)
    constexpr int LPT = NEEDLUT ? (2050 + NT - 1) / NT : 1;   // table entries per thread
    SetupPart sp;
    int2 lv[LPT];
    if constexpr (NEEDLUT) {
        const int* raw = reinterpret_cast<const int*>(reinterpret_cast<const char*>(sh.lut) + LUT_RAW_OFF);
#pragma unroll
        for (int q = 0; q < LPT; ++q) {
            const int i = tid + NT * q;
            int2 v = make_int2(0, 0);
            if (i == 2049) v = make_int2(65536, 0);
            else if (i >= 1 && i <= 2049) {
                const int a = raw[i - 1], nx = i - 1 == 2047 ? L2048 : raw[i];
                v = make_int2(a, nx - a);
                sp.lbad |= unsigned(a) > 65536u || unsigned(nx) > 65536u;
            }
            lv[q] = v;
        }
    }
    double ms = 0.0, wmv = 0.0;
    const int bb = t.cok ? t.c.z : 0;
    if (t.cok) setup_column(p, t.c, ms, wmv, sp);
    if (t.eok) { sp.emn = t.e; sp.emx = t.e; }
    setup_publish(sh, sp);
    if constexpr (EPI == EPI_PLAIN_GN) gn_clear(p, t.m0, sh);
    __syncthreads();   // raw table read by everyone, every wave's slot in
    // ---- phase 2: the block's forms, the column tables (with the e == 0 FMA constant: wm + 1/2, and
    // + b when folded, exact as above) and the expanded GELU table
    const EpiFlags f = setup_flags<NEEDLUT, NT / 64>(sh);
    if (tid < BN) {
        sh.ms[tid] = ms;
        sh.wm[tid] = f.ezero ? (wmv + 0.5) + (f.fold ? double(bb) : 0.0) : wmv;
        sh.b[tid] = bb;
    }
    if constexpr (NEEDLUT) {
#pragma unroll
        for (int q = 0; q < LPT; ++q) {
            const int i = tid + NT * q;
            if (i < 2050) sh.lut[i] = lv[q];
        }
    }
    __syncthreads();
    return f;
}

// The requantising epilogue of one wave. Subtile (ns, ms) of the wave holds rows
// rbase + ms*16 + (lane & 15) and LDS-table rows wsub_row(wn, ns) + 4*(lane >> 4) + v, v = 0..3.
template <int EPI, int SRC, class T, bool EZERO, bool SMALLK, bool FOLD, class S>
__device__ __forceinline__ void fused_epilogue_t(const GemmParams& p, const v4i (&acc_h)[T::NS][T::MS], const v4i (&acc_l)[T::NS][T::MS],
                                                 int rbase, int n0, int wn, const S& sh, bool fast, const int (&er)[T::MS]) {
    static_assert(!FOLD || EZERO, "folding b assumes e == 0");
    constexpr int MS = T::MS, NS = T::NS;
    const int lane = threadIdx.x & 63, fr = lane & 15, fg = lane >> 4;
    double pr[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) pr[ms] = EZERO ? 1.0 : ldexp(1.0, min(max(er[ms], -1000), 1000));
    // running max and min of y per row: max |y| = max(ymax, -ymin), two instructions per value
    int ymax[MS], ymin[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) { ymax[ms] = 0; ymin[ms] = 0; }

    // A = 256*Chi + Clo as an exact double
    auto comb = [&](int h, int l) -> double {
        if constexpr (SMALLK) return double((h << 8) + l);
        else return __builtin_fma(double(h), 256.0, double(l));
    };
    // floor(acc*m*2^-(s-e) + 1/2) saturated, + b saturated: exact under the block conditions
    auto epi_fast = [&](double A, double ms_, double wm_, double wmh_, int b_, double prr) -> int {
        double X;
        if constexpr (EZERO) X = __builtin_fma(A, ms_, wmh_);
        else X = __builtin_fma(__builtin_fma(A, ms_, wm_), prr, 0.5);
        return add_sat(cvt_sat(__builtin_floor(X)), b_);
    };
    // GELU factor (lut16i) for tables with 0 <= L <= 65536
    // z = x + 2^20 clamped to [-1, 2^21]; index (z >> 10) + 1 = (x >> 10) + 1025 and z & 1023 =
    // x & 1023 (2^20 is a multiple of 1024), so the offset folds into the LDS address
    auto phi = [&](int x) -> int {
        const int xc = min(max(x, -1048577), 1048576);
        const int2 t = sh.lut[(xc >> 10) + 1025];
        return t.x + (__mul24(t.y, xc & 1023) >> 10);
    };
    // floor((y * phi(y) + 2^15) / 2^16) for 0 <= phi <= 65536 (never saturates)
    auto gelu_fast = [&](int y) -> double {
        const double P = __builtin_fma(double(y), double(phi(y)), 32768.0);
        return __builtin_floor(P * (1.0 / 65536.0));
    };
    // the same from y held both as an int and as a double
    auto gelu_fast2 = [&](int yi, double yd) -> double {
        const double P = __builtin_fma(yd, double(phi(yi)), 32768.0);
        return __builtin_floor(P * (1.0 / 65536.0));
    };

    constexpr int NOUT = EPI == EPI_GEGLU ? NS / 2 : NS;
#pragma unroll
    for (int ns = 0; ns < NOUT; ++ns) {
        const int lr = wsub_row<EPI, T>(wn, ns) + 4 * fg;   // table row of this lane's 4 columns
        const int lg = EPI == EPI_GEGLU ? wsub_row<EPI, T>(wn, ns + NS / 2) + 4 * fg : lr;
        // output column of value v: n0 + lr + v (plain); (n0 >> 1) + lr + v (GEGLU, lr < BN/2)
        const int ncol = EPI == EPI_GEGLU ? (n0 >> 1) + lr : n0 + lr;
        const int nlim = EPI == EPI_GEGLU ? (p.Nreal >> 1) : p.Nreal;
        if (ncol >= nlim) continue;
        double c_ms[4], c_wm[4], c_wmh[4], g_ms[4], g_wm[4], g_wmh[4];
        int c_b[4], g_b[4];
        if (fast) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                c_ms[v] = sh.ms[lr + v];
                if constexpr (EZERO) c_wmh[v] = sh.wm[lr + v];
                else c_wm[v] = sh.wm[lr + v];
                if constexpr (!FOLD) c_b[v] = sh.b[lr + v];
                if constexpr (EPI == EPI_GEGLU) {
                    g_ms[v] = sh.ms[lg + v];
                    if constexpr (EZERO) g_wmh[v] = sh.wm[lg + v];
                    else g_wm[v] = sh.wm[lg + v];
                    if constexpr (!FOLD) g_b[v] = sh.b[lg + v];
                }
            }
        }
        const bool full = ncol + 3 < nlim;
        // GroupNorm statistics of this lane's four columns over its rows (EPI_PLAIN_GN)
        constexpr bool gn = EPI == EPI_PLAIN_GN;
        long long gsum[4] = {0, 0, 0, 0};
        int gmn[4] = {INT_MAX, INT_MAX, INT_MAX, INT_MAX}, gmx[4] = {INT_MIN, INT_MIN, INT_MIN, INT_MIN};
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            const int r = rbase + ms * 16 + fr;
            if (r >= p.Mreal) continue;
            int y[4];
            if (FOLD) {
                // y = floor(A*m*2^-s + 1/2 + b): b folded into the constant, nothing saturates
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const double ya = __builtin_floor(__builtin_fma(comb(acc_h[ns][ms][v], acc_l[ns][ms][v]), c_ms[v], c_wmh[v]));
                    if constexpr (EPI == EPI_GEGLU) {
                        const double yg = __builtin_floor(__builtin_fma(comb(acc_h[ns + NS / 2][ms][v], acc_l[ns + NS / 2][ms][v]), g_ms[v], g_wmh[v]));
                        const double ge = gelu_fast2(int(yg), yg);
                        // (a*ge + 2^15) * 2^-16 with a pre-scaled by 2^-16 (exact: a power of two)
                        y[v] = cvt_sat(__builtin_floor(__builtin_fma(ya * (1.0 / 65536.0), ge, 0.5)));
                    } else if constexpr (EPI == EPI_GELU) {
                        y[v] = int(gelu_fast2(int(ya), ya));
                    } else {
                        y[v] = int(ya);
                    }
                }
            } else if (fast) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int ya = epi_fast(comb(acc_h[ns][ms][v], acc_l[ns][ms][v]), c_ms[v], c_wm[v], c_wmh[v], c_b[v], pr[ms]);
                    if constexpr (EPI == EPI_GEGLU) {
                        const int yg = epi_fast(comb(acc_h[ns + NS / 2][ms][v], acc_l[ns + NS / 2][ms][v]), g_ms[v], g_wm[v], g_wmh[v], g_b[v], pr[ms]);
                        const double ge = gelu_fast(yg);
                        const double Q = __builtin_fma(double(ya), ge, 32768.0);
                        y[v] = cvt_sat(__builtin_floor(Q * (1.0 / 65536.0)));
                    } else if constexpr (EPI == EPI_GELU) {
                        y[v] = int(gelu_fast(ya));
                    } else {
                        y[v] = ya;
                    }
                }
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (ncol + v >= nlim) { y[v] = 0; continue; }
                    if constexpr (EPI == EPI_GEGLU) {
                        const int na = 2 * (ncol + v);
                        const int4 ca = p.cst[na], cg = p.cst[na + 1];
                        const int ya = epi1_exact(acc_h[ns][ms][v], acc_l[ns][ms][v], ca.x, ca.y, ca.z, ca.w, er[ms]);
                        const int yg = epi1_exact(acc_h[ns + NS / 2][ms][v], acc_l[ns + NS / 2][ms][v], cg.x, cg.y, cg.z, cg.w, er[ms]);
                        y[v] = geglu_exact(ya, yg, p.Lphi);
                    } else {
                        const int4 c = p.cst[ncol + v];
                        int yy = epi1_exact(acc_h[ns][ms][v], acc_l[ns][ms][v], c.x, c.y, c.z, c.w, er[ms]);
                        if constexpr (EPI == EPI_GELU) yy = gelu_exact(yy, p.Lphi);
                        y[v] = yy;
                    }
                }
            }
            if constexpr (EPI == EPI_SPLIT3) {
                // Cs % 4 == 0: the four columns lie in one part (src/gemm_hl.cu:288-290)
                const int part = ncol >= 2 * p.Cs ? 2 : (ncol >= p.Cs ? 1 : 0);
                int32_t* d = (part == 0 ? p.Y : (part == 1 ? p.Y1 : p.Y2)) + size_t(r) * p.Cs + (ncol - part * p.Cs);
                if (full && p.vec_store) *reinterpret_cast<v4i*>(d) = v4i{y[0], y[1], y[2], y[3]};
                else {
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        if (ncol + v < nlim) d[v] = y[v];
                }
            } else {
                int32_t* d = p.Y + size_t(r) * p.ldy + ncol;
                if constexpr (EPI != EPI_GEGLU) {
                    if (p.R) {
                        const int32_t* rp = p.R + size_t(r) * p.ldy + ncol;
                        if (full && p.vec_store) {
                            const v4i rv = *reinterpret_cast<const v4i*>(rp);
#pragma unroll
                            for (int v = 0; v < 4; ++v) y[v] = add_sat(y[v], rv[v]);
                        } else {
#pragma unroll
                            for (int v = 0; v < 4; ++v)
                                if (ncol + v < nlim) y[v] = add_sat(y[v], rp[v]);
                        }
                    }
                }
                if (full && p.vec_store) *reinterpret_cast<v4i*>(d) = v4i{y[0], y[1], y[2], y[3]};
                else {
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        if (ncol + v < nlim) d[v] = y[v];
                }
                if (p.rowmax) {
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        if (ncol + v < nlim) { ymax[ms] = max(ymax[ms], y[v]); ymin[ms] = min(ymin[ms], y[v]); }
                }
                if constexpr (gn) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        gsum[v] += y[v];
                        gmn[v] = min(gmn[v], y[v]);
                        gmx[v] = max(gmx[v], y[v]);
                    }
                }
            }
        }
        if constexpr (gn) {
            // group of column c: c / (Nreal / 32); region of the lane's rows and four columns: the
            // block's rows and columns start at multiples of its shape, which holds whole regions
            S& shw = const_cast<S&>(sh);
            const int cg = p.Nreal >> 5;
            const int slot = ((rbase % T::BM) / p.gnBM) * 4 + (ncol % T::BN) / p.gnBN;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (ncol + v < nlim) {
                    const int g = (ncol + v) / cg;
                    atomicAdd(reinterpret_cast<unsigned long long*>(&shw.gsum[slot][g]), static_cast<unsigned long long>(gsum[v]));
                    atomicMin(&shw.gmin[slot][g], gmn[v]);
                    atomicMax(&shw.gmax[slot][g], gmx[v]);
                }
            }
        }
    }
    if constexpr (EPI != EPI_SPLIT3) {
        if (p.rowmax) {
            // lanes fr, fr+16, fr+32, fr+48 hold the same row: one atomic per row and wave
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                uint32_t m = max(uint32_t(ymax[ms]), uabs(ymin[ms]));
                m = max(m, uint32_t(__shfl_xor(int(m), 16)));
                m = max(m, uint32_t(__shfl_xor(int(m), 32)));
                const int r = rbase + ms * 16 + fr;
                if (fg == 0 && r < p.Mreal && m) atomicMax(p.rowmax + r, m);
            }
        }
    }
}

template <int EPI, int SRC, class T, class S>
__device__ __forceinline__ void fused_epilogue(const GemmParams& p, const v4i (&acc_h)[T::NS][T::MS], const v4i (&acc_l)[T::NS][T::MS],
                                               int rbase, int n0, int wn, const S& sh, EpiFlags f, const int (&er)[T::MS]) {
    const bool smallK = p.Kp <= 496;   // |256*Chi + Clo| < 2^31
    if (f.fold) {
        if (smallK) fused_epilogue_t<EPI, SRC, T, true, true, true>(p, acc_h, acc_l, rbase, n0, wn, sh, f.fast, er);
        else fused_epilogue_t<EPI, SRC, T, true, false, true>(p, acc_h, acc_l, rbase, n0, wn, sh, f.fast, er);
    } else if (f.ezero) {
        if (smallK) fused_epilogue_t<EPI, SRC, T, true, true, false>(p, acc_h, acc_l, rbase, n0, wn, sh, f.fast, er);
        else fused_epilogue_t<EPI, SRC, T, true, false, false>(p, acc_h, acc_l, rbase, n0, wn, sh, f.fast, er);
    } else {
        if (smallK) fused_epilogue_t<EPI, SRC, T, false, true, false>(p, acc_h, acc_l, rbase, n0, wn, sh, f.fast, er);
        else fused_epilogue_t<EPI, SRC, T, false, false, false>(p, acc_h, acc_l, rbase, n0, wn, sh, f.fast, er);
    }
}

// EPI_QKV (src/gemm_hl.cu:179-241): output columns n = part*C + 64*head + d. Part 2 (v) goes to
// Y2[r][64*head + d] as int32; parts 0 and 1 (q, k) are quantised per row and head to 16 bits with
// e = row_exp(max |y| over the head's 64 columns), split into hi/lo bytes at
// [(b*heads + head)*Tp + t][d] (b = r / T, t = r % T, Tp = TpQ or TpK), with e and the sums of hi,
// lo and q per row and head (the k_quant_heads layout, src/kernels.cu:611-631). Each head lies in
// one wave (64-aligned columns, 4 subtiles); y is the reference's int64 formula. Pad rows t >= T are
// not written (the caller pads them, src/engine.cu:329-330).
template <class T>
__device__ __forceinline__ void qkv_epilogue(const GemmParams& p, const v4i (&acc_h)[T::NS][T::MS], const v4i (&acc_l)[T::NS][T::MS],
                                             int rbase, int n0, int wn, const int (&er)[T::MS]) {
    constexpr int MS = T::MS, NS = T::NS;
    static_assert(NS % 4 == 0, "whole heads per wave");
    const int lane = threadIdx.x & 63, fr = lane & 15, fg = lane >> 4;
    const int cw = n0 + wn * T::WTN;   // first column of the wave (wsub_row is the identity here)
#pragma unroll
    for (int hh = 0; hh < NS / 4; ++hh) {
        const int c0 = cw + hh * 64;
        if (c0 >= p.Nreal) continue;
        const int part = c0 / p.qC, head = (c0 - part * p.qC) >> 6;
        int4 cc[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) cc[j][v] = p.cst[c0 + 16 * j + 4 * fg + v];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            const int r = rbase + ms * 16 + fr;
            const bool rok = r < p.Mreal;
            int y[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    y[j][v] = epi1_exact(acc_h[4 * hh + j][ms][v], acc_l[4 * hh + j][ms][v], cc[j][v].x, cc[j][v].y, cc[j][v].z,
                                         cc[j][v].w, er[ms]);
            if (part == 2) {
                if (rok) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        *reinterpret_cast<v4i*>(p.Y2 + size_t(r) * p.qC + head * 64 + 16 * j + 4 * fg) = v4i{y[j][0], y[j][1], y[j][2], y[j][3]};
                }
                continue;
            }
            // lanes fr, fr + 16, fr + 32, fr + 48 hold the row's 64 values of this head
            uint32_t m = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v) m = max(m, uabs(y[j][v]));
            m = max(m, uint32_t(__shfl_xor(int(m), 16)));
            m = max(m, uint32_t(__shfl_xor(int(m), 32)));
            const int ee = rowexp_u32(m);
            const int b = rok ? r / p.qT : 0, t = r - b * p.qT;
            const size_t gt = size_t(b * p.heads + head) * (part ? p.TpK : p.TpQ) + t;
            int8_t* hp = part ? p.khi : p.qhi;
            int8_t* lp = part ? p.klo : p.qlo;
            int hs = 0, ls = 0, ts = 0;   // |sum of 64 values| < 2^22
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                unsigned hw = 0, lw = 0;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int q = quant16_32(y[j][v], ee);
                    const int h = q >> 8, l = (q & 255) - 128;
                    hw |= unsigned(h & 255) << (8 * v);
                    lw |= unsigned(l & 255) << (8 * v);
                    hs += h;
                    ls += l;
                    ts += q;
                }
                if (rok) {
                    *reinterpret_cast<unsigned*>(hp + gt * 64 + 16 * j + 4 * fg) = hw;
                    *reinterpret_cast<unsigned*>(lp + gt * 64 + 16 * j + 4 * fg) = lw;
                }
            }
            hs += __shfl_xor(hs, 16); hs += __shfl_xor(hs, 32);
            ls += __shfl_xor(ls, 16); ls += __shfl_xor(ls, 32);
            ts += __shfl_xor(ts, 16); ts += __shfl_xor(ts, 32);
            if (rok && fg == 0) {
                (part ? p.ke : p.qe)[gt] = ee;
                (part ? p.khs : p.qhs)[gt] = hs;
                (part ? p.kls : p.qls)[gt] = ls;
                (part ? p.kts : p.qts)[gt] = ts;
            }
        }
    }
}

// int32 partial sums of one K range: ws[(ks*2 + plane) * ws_rows + row][col]
template <class T>
__device__ __forceinline__ void store_partial(const GemmParams& p, const v4i (&acc_h)[T::NS][T::MS], const v4i (&acc_l)[T::NS][T::MS],
                                              int rbase, int cbase, int ks) {
    const int lane = threadIdx.x & 63, fr = lane & 15, fg = lane >> 4;
#pragma unroll
    for (int ns = 0; ns < T::NS; ++ns)
#pragma unroll
        for (int ms = 0; ms < T::MS; ++ms) {
            const int r = rbase + ms * 16 + fr;
            const int n = cbase + ns * 16 + 4 * fg;
            int32_t* dh = p.ws + (size_t(ks * 2) * p.ws_rows + r) * p.ws_ld + n;
            int32_t* dl = dh + size_t(p.ws_rows) * p.ws_ld;
            *reinterpret_cast<v4i*>(dh) = acc_h[ns][ms];
            *reinterpret_cast<v4i*>(dl) = acc_l[ns][ms];
        }
}

// plain int32 output of the single-plane GEMM
template <class T>
__device__ __forceinline__ void store_raw(const GemmParams& p, const v4i (&acc)[T::NS][T::MS], int rbase, int cbase, int bt) {
    const int lane = threadIdx.x & 63, fr = lane & 15, fg = lane >> 4;
    int32_t* C = p.Y + bt * p.sC;
#pragma unroll
    for (int ns = 0; ns < T::NS; ++ns)
#pragma unroll
        for (int ms = 0; ms < T::MS; ++ms) {
            const int r = rbase + ms * 16 + fr;
            const int n = cbase + ns * 16 + 4 * fg;
            if (r >= p.Mreal) continue;
            int32_t* d = C + size_t(r) * p.ldy + n;
            if (p.vec_store && n + 3 < p.Nreal) {
                *reinterpret_cast<v4i*>(d) = acc[ns][ms];
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (n + v < p.Nreal) d[v] = acc[ns][ms][v];
            }
        }
}

// Tile of this block. Blocks are dispatched round-robin over the 8 XCDs; renumber them so that
// each XCD receives a contiguous range of work units, in one of two orders. Row order (K range
// fastest, then column tile, then row tile): an XCD owns whole row stripes and its L2 serves their
// A rows to every column tile, while every XCD reads all of W. Column order (row tile fastest, then
// column tile, then K range): an XCD owns a run of (K range, column tile) groups, so W is read about
// once over the chip and A once per XCD for the K ranges it covers; the blocks resident together
// on an XCD share a few W column tiles. The host picks the order with the smaller estimated fetch.
struct TileIdx {
    int ks, mt, nt;
};
// The kernel arguments, one 64-byte line at a time, in one round of scalar loads at kernel entry:
// the argument block is read cold from memory, and the prologue's own argument loads sit between
// branches, each round waiting for the last; with the lines in the scalar cache they hit.
__device__ __forceinline__ void prefetch_args() {
    static_assert(sizeof(GemmParams) <= 8 * 64, "eight lines of kernel arguments");
    const auto k = (const __attribute__((address_space(4))) int*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" ::"s"(k[0]), "s"(k[16]), "s"(k[32]), "s"(k[48]), "s"(k[64]), "s"(k[80]), "s"(k[96]), "s"(k[112]));
}

__device__ __forceinline__ TileIdx tile_index(const GemmParams& p) {
    const int nblk = gridDim.x, bid = blockIdx.x;
    const int q8 = nblk >> 3, r8 = nblk & 7, xcd = bid & 7, slot = bid >> 3;
    const int lin = (xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8) + slot;
    TileIdx t;
    if (p.colmajor) {
        t.mt = lin % p.mtiles;
        const int g = lin / p.mtiles;
        t.ks = g / p.ntiles;
        t.nt = g - t.ks * p.ntiles;
    } else {
        t.ks = lin % p.ksplit;
        const int tl = lin / p.ksplit;
        t.mt = tl / p.ntiles;
        t.nt = tl - t.mt * p.ntiles;
    }
    return t;
}

// ================================================================ DMA main loop (I8, I16, X32, CONV16, CONV32, RAW)

// LDS stages of the raw int32 image rows: two (48 KB per 64 x 128 block, three blocks per CU)
// measured 116 us on the C3 shape against 153 us with three stages (two blocks per CU)
#ifndef VK_RAW32_STAGES
#define VK_RAW32_STAGES 2
#endif
template <int SRC, int EPI, class T>
struct DmaCfg {
    static constexpr bool TWO = EPI != EPI_RAW;
    static constexpr bool FUSED = EPI != EPI_PARTIAL && EPI != EPI_RAW;
    static constexpr bool NEEDLUT = EPI == EPI_GEGLU || EPI == EPI_GELU;
    static constexpr bool RAW16 = SRC == SRC_I16 || SRC == SRC_CONV16;   // raw int16 rows in LDS
    static constexpr bool RAW32 = SRC == SRC_CONV32 || SRC == SRC_X32;  // raw int32 rows in LDS
    static constexpr int W_BYTES = T::BN * 64;
    static constexpr int A_BYTES = RAW32 ? T::BM * 256 : RAW16 ? T::BM * 128 : (TWO ? 2 : 1) * T::BM * 64;
    static constexpr int STAGE = W_BYTES + A_BYTES;
#ifndef VK_DMA_STAGES
    // LDS stages: three, or two where a GELU table must fit beside them for two blocks per CU (raw
    // int32 rows: VK_RAW32_STAGES)
    static constexpr int NST = RAW32 ? VK_RAW32_STAGES : NEEDLUT && T::BM * T::BN < 128 * 256 ? 2 : 3;
#else
    static constexpr int NST = NEEDLUT && T::BM * T::BN < 128 * 256 ? 2 : VK_DMA_STAGES;
#endif
    static constexpr int W_INS = W_BYTES / 1024 / T::NW;   // DMA instructions per wave per stage: W
    static constexpr int A_INS = A_BYTES / 1024 / T::NW;   //                                     A
    static constexpr int PER_STAGE = W_INS + A_INS;
    static_assert(W_INS >= 1 && A_INS >= 1 && (A_BYTES % (1024 * T::NW)) == 0 && (W_BYTES % (1024 * T::NW)) == 0, "DMA mapping");
};

#ifndef VK_MIN_BLOCKS_SMALL
#define VK_MIN_BLOCKS_SMALL 2
#endif
// waves per SIMD the register allocator must allow (the second __launch_bounds__ argument):
// blocks per CU x waves per block / 4. Two blocks per CU, three for 64 x 128 tiles without a GELU
// table, one for the 128 x 256 tile.
template <class T, int EPI>
constexpr int dma_waves_per_simd() {
    const int blocks = T::BM * T::BN >= 128 * 256 ? 1
                     : (T::BM * T::BN <= 64 * 128 && EPI != EPI_GEGLU && EPI != EPI_GELU ? VK_MIN_BLOCKS_SMALL : 2);
    return blocks * T::NW / 4;
}

template <int SRC, int EPI, class T>
__global__ void __launch_bounds__(T::NT, (dma_waves_per_simd<T, EPI>())) gemm_dma_kernel(const GemmParams p) {
    prefetch_args();
    using D = DmaCfg<SRC, EPI, T>;
    constexpr int BM = T::BM, BN = T::BN, MS = T::MS, NS = T::NS, NST = D::NST;
    constexpr bool TWO = D::TWO, FUSED = D::FUSED;

    __shared__ __attribute__((aligned(16))) unsigned char smem[NST * D::STAGE];
    __shared__ __attribute__((aligned(16))) EpiShared<FUSED ? BN : 1, D::NEEDLUT, EPI == EPI_PLAIN_GN> sh;

    // the wave index in a scalar register (the DMA's LDS addresses must be wave-uniform); waves
    // are WM x WN over the tile, wm the row slot and wn the column slot
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % T::WM, wn = wave / T::WM;
    const TileIdx ti = tile_index(p);
    const int m0 = ti.mt * BM, n0 = ti.nt * BN;
    const int nK = (p.Kp + 63) >> 6;
    const int kb = ti.ks * p.kper, ke = min(nK, kb + p.kper);
    const int bt = blockIdx.y;   // batch index (EPI_RAW)

    const char* a0p = static_cast<const char*>(p.a0) + (EPI == EPI_RAW ? bt * p.sA : 0);
    const int8_t* wp = p.w + (EPI == EPI_RAW ? bt * p.sW : 0);
    const v4i rW = make_rsrc_words(wp, p.w_bytes);   // scalar registers
    const v4i rA0 = make_rsrc_words(a0p, p.a0_bytes);
    const v4i rA1 = make_rsrc_words(SRC == SRC_I8 && TWO ? p.a1 : a0p, SRC == SRC_I8 && TWO ? p.a1_bytes : p.a0_bytes);

    // rows owned by this wave and their shifts (for the epilogue and the image quantisation), and
    // the epilogue's table inputs: all loaded first, so that they are older than every DMA below
    // (loads complete in order: waiting for a K step's DMA then implies these are in too)
    const int rbase = m0 + wm * T::WTM;
    int er[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
        const int r = rbase + ms * 16 + (lane & 15);
        er[ms] = (r < p.Mreal && (FUSED || D::RAW32 || SRC == SRC_CONV16)) ? row_shift<SRC>(p, r) : 0;
    }
    TilePre pre{};
    if constexpr (FUSED) pre = load_tile_pre<EPI, SRC, BM, BN>(p, m0, n0);
    const int L2048 = D::NEEDLUT ? p.Lphi[2048] : 0;
    if constexpr (D::NEEDLUT) {
        // GELU table entries 0..2047 -> LDS (raw), 8 KB: eight 1 KB DMA instructions per block
        const v4i rL = make_rsrc_words(p.Lphi, 2049u * 4u);
        const unsigned lbase = lds_addr(sh.lut) + LUT_RAW_OFF;
        constexpr int LJ = 8 / T::NW;
#pragma unroll
        for (int j = 0; j < LJ; ++j) {
            const unsigned c = unsigned(wave * LJ + j) * 1024u;
            dma16(rL, unsigned(lane) * 16u, c, lbase + c);
        }
    }

    // ---- DMA address state. W: wave instruction j covers LDS rows 16*(wave*W_INS + j) + lane/4,
    // chunk position lane%4 (holding the global chunk that the swizzle puts there). A (raw int16):
    // rows 8*(wave*A_INS + j) + lane/8, chunk position lane%8. A (int8 planes): like W, hi then lo.
    // Per-lane byte offsets are fixed over the K loop; each K step adds a scalar offset, and only
    // the last, partial K step checks columns lane by lane.
    unsigned w_off[D::W_INS];
    int w_k[D::W_INS];
#pragma unroll
    for (int j = 0; j < D::W_INS; ++j) {
        // instruction j fills 128-byte LDS rows 8 (wave * W_INS + j) + lane / 8 (pswz): lane l holds
        // the chunk that the swizzle puts at position l % 8, of W row 2 R + (chunk >> 2)
        const int R = 8 * (wave * D::W_INS + j) + (lane >> 3), lc = (lane & 7) ^ swz16_key(R);
        const int lr = 2 * R + (lc >> 2);
        const int nrow = n0 + (FUSED ? wrow_of_lds<EPI, BN>(lr) : lr);
        w_k[j] = 16 * (lc & 3);
        w_off[j] = nrow < p.Nreal ? unsigned(nrow) * unsigned(p.ldw) + unsigned(w_k[j]) : OOB;
    }
    constexpr int A_ROWS_INS = D::RAW32 ? 4 : D::RAW16 ? 8 : 16;       // rows per DMA instruction
    constexpr int A_INS_PLANE = D::RAW16 || D::RAW32 ? D::A_INS : D::A_INS / (TWO ? 2 : 1);
    unsigned a_off[A_INS_PLANE];
    int a_k[A_INS_PLANE], a_pix[A_INS_PLANE];
    unsigned a_mask[A_INS_PLANE];
    // SRC_CONV16 with C % 64 == 0: a 64-wide K step never straddles a 3x3 tap, so the tap and the
    // channel offset of a step are block-wide scalars and each lane only checks its tap mask
    // (SRC_CONV32 runs here only with C % 64 == 0: the host sends other convolutions to the
    // register-staged kernel)
    const bool conv_fast = (SRC == SRC_CONV16 || SRC == SRC_CONV32) && (p.C & 63) == 0;
    const unsigned cmagic = SRC == SRC_CONV16 ? unsigned((0x100000000ull + unsigned(p.C) - 1) / unsigned(p.C)) : 0u;
#pragma unroll
    for (int j = 0; j < A_INS_PLANE; ++j) {
        // int8 planes (pswz, as W): LDS row R = 8 g + lane / 8 of the plane holds rows 2 R, 2 R + 1
        const int g = wave * A_INS_PLANE + j;
        const int R8 = 8 * g + (lane >> 3), lc8 = (lane & 7) ^ swz16_key(R8);
        const int row = D::RAW32 ? A_ROWS_INS * g + (lane >> 4) : D::RAW16 ? A_ROWS_INS * g + (lane >> 3) : 2 * R8 + (lc8 >> 2);
        const int r = m0 + row;
        const bool rok = r < p.Mreal;
        if constexpr (D::RAW32) a_k[j] = 4 * ((lane & 15) ^ (row & 15));
        else if constexpr (D::RAW16) a_k[j] = 8 * ((lane & 7) ^ swz16_key(row));
        else a_k[j] = 16 * (lc8 & 3);
        if constexpr (SRC == SRC_I16) {
            a_off[j] = rok ? (unsigned(r) * unsigned(p.lda) + unsigned(a_k[j])) * 2u : OOB;
        } else if constexpr (SRC == SRC_X32) {
            a_off[j] = rok ? (unsigned(r) * unsigned(p.lda) + unsigned(a_k[j])) * 4u : OOB;
        } else if constexpr (SRC == SRC_CONV16 || SRC == SRC_CONV32) {
            constexpr int EB = SRC == SRC_CONV32 ? 4 : 2;   // bytes per image value
            const int HoWo = p.Ho * p.Wo;
            const int rr = rok ? r : 0;
            const int b = rr / HoWo, pp = rr - b * HoWo, oy = pp / p.Wo, ox = pp - oy * p.Wo;
            const int iy0 = oy * p.stride - 1, ix0 = ox * p.stride - 1;
            unsigned mask = 0;
#pragma unroll
            for (int t = 0; t < 9; ++t) {
                const int iy = iy0 + t / 3, ix = ix0 + t % 3;
                mask |= unsigned(rok && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W) << t;
            }
            a_mask[j] = mask;
            // byte offset of channel a_k of pixel (iy0, ix0); negative at the border, but only taps
            // inside the image are ever added to it
            a_pix[j] = (((b * p.H + iy0) * p.W + ix0) * p.C + a_k[j]) * EB;
            a_off[j] = unsigned(a_pix[j]);
        } else {
            a_off[j] = rok ? unsigned(r) * unsigned(p.lda) + unsigned(a_k[j]) : OOB;
        }
    }

    // implicit im2col position of the next K step to issue, (tap, channel): the steps are issued in
    // order kb, kb + 1, ..., so it advances by 64 channels per call instead of dividing each time
    int nx_tap = 0, nx_c0 = 0;
    if constexpr (SRC == SRC_CONV16 || SRC == SRC_CONV32) {
        if (conv_fast) {
            nx_tap = (kb * 64) / p.C;
            nx_c0 = kb * 64 - nx_tap * p.C;
        }
    }
    auto issue = [&](int kt, int stage) {
        const unsigned sbase = lds_addr(smem) + stage * D::STAGE;
        const int kbase = kt * 64;
        // the K step lies wholly inside K (uniform): no per-lane range test
        if (kbase + 64 <= p.Kp) {
#pragma unroll
            for (int j = 0; j < D::W_INS; ++j) dma16(rW, w_off[j], unsigned(kbase), sbase + (wave * D::W_INS + j) * 1024);
        } else {
#pragma unroll
            for (int j = 0; j < D::W_INS; ++j) {
                const unsigned off = kbase + w_k[j] >= p.Kp ? OOB : w_off[j];
                dma16(rW, off, unsigned(kbase), sbase + (wave * D::W_INS + j) * 1024);
            }
        }
        const unsigned sA = sbase + D::W_BYTES;
        if constexpr (SRC == SRC_I16) {
            if (kbase + 64 <= p.K) {
#pragma unroll
                for (int j = 0; j < A_INS_PLANE; ++j) dma16(rA0, a_off[j], unsigned(kbase) * 2u, sA + (wave * A_INS_PLANE + j) * 1024);
            } else {
#pragma unroll
                for (int j = 0; j < A_INS_PLANE; ++j) {
                    const unsigned off = kbase + a_k[j] >= p.K ? OOB : a_off[j];
                    dma16(rA0, off, unsigned(kbase) * 2u, sA + (wave * A_INS_PLANE + j) * 1024);
                }
            }
        } else if constexpr (SRC == SRC_X32) {
            // int32 rows, K % 4 == 0 (the host's condition), so each 16-byte piece is all in or all out
            const bool atail = kbase + 64 > p.K;
#pragma unroll
            for (int j = 0; j < A_INS_PLANE; ++j) {
                const unsigned off = (atail && kbase + a_k[j] >= p.K) ? OOB : a_off[j];
                dma16(rA0, off, unsigned(kbase) * 4u, sA + (wave * A_INS_PLANE + j) * 1024);
            }
        } else if constexpr (SRC == SRC_CONV32) {
            // implicit 3x3 im2col of the int32 image (conv_fast shapes only)
            const int tap = nx_tap, c0 = nx_c0;
            nx_c0 += 64;
            if (nx_c0 >= p.C) { nx_c0 -= p.C; ++nx_tap; }
            const int ky = (tap * 11) >> 5, kx = tap - 3 * ky;
            const int soff = ((ky * p.W + kx) * p.C + c0) * 4;
#pragma unroll
            for (int j = 0; j < A_INS_PLANE; ++j) {
                const bool ok = tap < 9 && ((a_mask[j] >> tap) & 1u);
                dma16(rA0, ok ? unsigned(a_pix[j] + soff) : OOB, 0u, sA + (wave * A_INS_PLANE + j) * 1024);
            }
        } else if constexpr (SRC == SRC_CONV16) {
            if (conv_fast) {
                // implicit 3x3 im2col, tap-major K: k = tap*C + c (src/gemm_hl.cu:104-114)
                const int tap = nx_tap, c0 = nx_c0;
                nx_c0 += 64;
                if (nx_c0 >= p.C) { nx_c0 -= p.C; ++nx_tap; }
                const int ky = (tap * 11) >> 5, kx = tap - 3 * ky;   // tap / 3, tap % 3 for tap < 9
                const int soff = ((ky * p.W + kx) * p.C + c0) * 2;
#pragma unroll
                for (int j = 0; j < A_INS_PLANE; ++j) {
                    const bool ok = tap < 9 && ((a_mask[j] >> tap) & 1u);
                    dma16(rA0, ok ? unsigned(a_pix[j] + soff) : OOB, 0u, sA + (wave * A_INS_PLANE + j) * 1024);
                }
            } else {
#pragma unroll
                for (int j = 0; j < A_INS_PLANE; ++j) {
                    const int k = kbase + a_k[j];
                    const int tap = int(__umulhi(unsigned(k), cmagic));
                    const int ch = k - tap * p.C;
                    const int ky = (tap * 11) >> 5, kx = tap - 3 * ky;
                    const bool ok = k < p.K && ((a_mask[j] >> tap) & 1u);
                    const int off = a_pix[j] - a_k[j] * 2 + ((ky * p.W + kx) * p.C + ch) * 2;
                    dma16(rA0, ok ? unsigned(off) : OOB, 0u, sA + (wave * A_INS_PLANE + j) * 1024);
                }
            }
        } else {
            const bool atail = kbase + 64 > p.Kp;
#pragma unroll
            for (int j = 0; j < A_INS_PLANE; ++j) {
                const unsigned off = (atail && kbase + a_k[j] >= p.Kp) ? OOB : a_off[j];
                dma16(rA0, off, unsigned(kbase), sA + (wave * A_INS_PLANE + j) * 1024);
                if constexpr (TWO) dma16(rA1, off, unsigned(kbase), sA + BM * 64 + (wave * A_INS_PLANE + j) * 1024);
            }
        }
    };

    // the first stages load while the block prologue runs
    const int n = ke - kb;
    PrioBands pb;
    pb.init(n, p.prio_bands);
#pragma unroll
    for (int s = 0; s < NST - 1; ++s)
        if (s < n) issue(kb + s, s);

    // image rows of this wave all have e == 0 (the usual case): a clamp is the whole quantisation.
    // Decided per wave, so that the compiler branches instead of evaluating both forms.
    bool e_any = false;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) e_any |= er[ms] != 0;
    const bool wave_e0 = SRC == SRC_CONV16 || D::RAW32 ? __builtin_amdgcn_ballot_w64(e_any) == 0 : true;
    // raw int32 rows: every row of the wave with e <= 16 (the three-instruction quantisation)
    bool e_big = false;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) e_big |= er[ms] > 16;
    const bool wave_e16 = D::RAW32 ? __builtin_amdgcn_ballot_w64(e_big) == 0 : true;

    v4i acc_h[NS][MS], acc_l[TWO ? NS : 1][TWO ? MS : 1];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            acc_h[ns][ms] = v4i{0, 0, 0, 0};
            if constexpr (TWO) acc_l[ns][ms] = v4i{0, 0, 0, 0};
        }

    auto compute = [&](int stage) {
        const unsigned char* sW = smem + stage * D::STAGE;
        const unsigned char* sA = sW + D::W_BYTES;
        const int fr = lane & 15, fg = lane >> 4;
        v4i hf[MS], lf[TWO ? MS : 1];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            const int row = wm * T::WTM + ms * 16 + fr;
            if constexpr (D::RAW32) {
                // the lane's 16 K values (four 16-byte chunks), quantised to int16 and split
                v4i x[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) x[q] = *reinterpret_cast<const v4i*>(sA + swz32(row, 4 * fg + q));
                unsigned d[8];
                if (wave_e0) clamp_pack16(x, d);
                else if (wave_e16) quant_pack16_e16(x, er[ms], d);
                else quant_pack16(x, er[ms], d);
                split16x16(d, hf[ms], lf[ms]);
            } else if constexpr (D::RAW16) {
                const v4i x0 = *reinterpret_cast<const v4i*>(sA + swz16(row, 2 * fg));
                const v4i x1 = *reinterpret_cast<const v4i*>(sA + swz16(row, 2 * fg + 1));
                unsigned d[8] = {unsigned(x0[0]), unsigned(x0[1]), unsigned(x0[2]), unsigned(x0[3]),
                                 unsigned(x1[0]), unsigned(x1[1]), unsigned(x1[2]), unsigned(x1[3])};
                if constexpr (SRC == SRC_CONV16) {
                    if (wave_e0) clamp16_pairs(d);
                    else quant16_pairs(d, er[ms]);
                }
                split16x16(d, hf[ms], lf[ms]);
            } else {
                hf[ms] = *reinterpret_cast<const v4i*>(sA + pswz(row, fg));
                if constexpr (TWO) lf[ms] = *reinterpret_cast<const v4i*>(sA + BM * 64 + pswz(row, fg));
            }
        }
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
            const int row = (FUSED ? wsub_row<EPI, T>(wn, ns) : (wn * NS + ns) * 16) + fr;
            const v4i wf = *reinterpret_cast<const v4i*>(sW + pswz(row, fg));
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                acc_h[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, hf[ms], acc_h[ns][ms], 0, 0, 0);
                if constexpr (TWO) acc_l[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, lf[ms], acc_l[ns][ms], 0, 0, 0);
            }
        }
    };

    // ---- main loop: NST-stage LDS ring, loads NST-1 steps ahead of the MFMAs, unrolled by NST so
    // that every LDS address is an immediate offset. The ordinary loads above are first used after
    // the loop (or, for image rows, by the ballot above), so no compiler wait lands inside it.
    for (int s0 = 0; s0 < n; s0 += NST) {
#pragma unroll
        for (int u = 0; u < NST; ++u) {
            const int s = s0 + u;
            if (s < n) {
                pb.step(s);
                // this stage's DMA done (the later stages' may still be in flight), then publish it
                if (NST >= 4 && s + 2 < n) vm_wait<(NST >= 4 ? 2 : 0) * D::PER_STAGE>();
                else if (NST >= 3 && s + 1 < n) vm_wait<D::PER_STAGE>();
                else vm_wait<0>();
                block_barrier();
                if (s + NST - 1 < n) issue(kb + s + NST - 1, (u + NST - 1) % NST);
                compute(u);
            }
        }
    }

    if constexpr (EPI == EPI_PARTIAL) {
        store_partial<T>(p, acc_h, acc_l, rbase, n0 + wn * T::WTN, ti.ks);
    } else if constexpr (EPI == EPI_RAW) {
        // split K: each K range's sums go to its own plane of the workspace (p.Y, stride p.sC)
        store_raw<T>(p, acc_h, rbase, n0 + wn * T::WTN, p.ksplit > 1 ? ti.ks : bt);
    } else if constexpr (EPI == EPI_QKV) {
        qkv_epilogue<T>(p, acc_h, acc_l, rbase, n0, wn, er);
    } else {
        const EpiFlags fl = epi_setup<EPI, SRC, BM, BN, T::NT>(p, pre, L2048, sh);
        fused_epilogue<EPI, SRC, T>(p, acc_h, acc_l, rbase, n0, wn, sh, fl, er);
        if constexpr (EPI == EPI_PLAIN_GN) gn_flush(p, sh);
    }
}

// ================================================================ register-staged main loop (X32, CONV32)

template <int SRC, int EPI, class T>
__global__ void __launch_bounds__(256) gemm_hl_kernel(const GemmParams p) {
    prefetch_args();
    constexpr int BM = T::BM, BN = T::BN, MS = T::MS, NS = T::NS;
    constexpr bool FUSED = EPI != EPI_PARTIAL;
    constexpr bool NEEDLUT = EPI == EPI_GEGLU || EPI == EPI_GELU;
    constexpr int AREG = 4;   // 16-byte loads per 16-value int32 chunk
    constexpr bool CONV = SRC == SRC_CONV32;
    static_assert(SRC == SRC_X32 || SRC == SRC_CONV32, "register path serves the int32 sources");

    __shared__ __attribute__((aligned(16))) unsigned char smem[2 * T::STAGE];
    __shared__ __attribute__((aligned(16))) EpiShared<FUSED ? BN : 1, NEEDLUT, EPI == EPI_PLAIN_GN> sh;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % T::WM, wn = wave / T::WM;
    const TileIdx ti = tile_index(p);
    const int m0 = ti.mt * BM, n0 = ti.nt * BN;
    const int nK = (p.Kp + 63) >> 6;
    const int kb = ti.ks * p.kper, ke = min(nK, kb + p.kper);

    const __amdgpu_buffer_rsrc_t rW = make_rsrc(p.w, p.w_bytes);
    const __amdgpu_buffer_rsrc_t rA0 = make_rsrc(p.a0, p.a0_bytes);

    EpiFlags fl{true, true, false};
    if constexpr (FUSED) fl = block_prologue<EPI, SRC, BM, BN>(p, m0, n0, sh);

    const int rbase = m0 + wm * T::WTM;
    int er[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
        const int r = rbase + ms * 16 + (lane & 15);
        er[ms] = 0;
        if (r < p.Mreal) er[ms] = row_shift<SRC>(p, r);
    }

    // ---- per-thread load tasks (fixed over the K loop)
    int a_row[T::AT], a_kc[T::AT], a_e[T::AT];
    int a_base[T::AT], a_iy0[T::AT], a_ix0[T::AT], a_tap[T::AT], a_c0[T::AT];
    bool a_ok[T::AT];
#pragma unroll
    for (int i = 0; i < T::AT; ++i) {
        const int c = tid + i * 256;
        a_row[i] = c >> 2;
        a_kc[i] = c & 3;
        const int r = m0 + a_row[i];
        a_ok[i] = r < p.Mreal;
        a_e[i] = 0;
        if constexpr (SRC == SRC_X32) a_e[i] = a_ok[i] ? row_shift<SRC>(p, r) : 0;
        if constexpr (CONV) {
            a_e[i] = a_ok[i] ? row_shift<SRC>(p, r) : 0;
            const int HoWo = p.Ho * p.Wo;
            const int rr = a_ok[i] ? r : 0;
            const int b = rr / HoWo, pp = rr - b * HoWo, oy = pp / p.Wo, ox = pp - oy * p.Wo;
            a_base[i] = b * p.H;
            a_iy0[i] = oy * p.stride - 1;
            a_ix0[i] = ox * p.stride - 1;
            const int k = kb * 64 + a_kc[i] * 16;
            a_tap[i] = k / p.C;
            a_c0[i] = k - a_tap[i] * p.C;
        }
    }

    v4i wreg[T::WT];
    v4i areg[T::AT][AREG];

    auto gload = [&](int kt) {
        const int kbase = kt * 64;
#pragma unroll
        for (int i = 0; i < T::WT; ++i) {
            const int c = tid + i * 256, row = c >> 2, kc = c & 3;
            const int n = n0 + (FUSED ? wrow_of_lds<EPI, BN>(row) : row), k = kbase + kc * 16;
            const unsigned off = (n < p.Nreal && k < p.Kp) ? unsigned(n) * unsigned(p.ldw) + unsigned(k) : OOB;
            wreg[i] = bload16(rW, off);
        }
#pragma unroll
        for (int i = 0; i < T::AT; ++i) {
            const int r = m0 + a_row[i], k = kbase + a_kc[i] * 16;
            if constexpr (SRC == SRC_X32) {
                const unsigned base = (unsigned(r) * unsigned(p.lda) + unsigned(k)) * 4u;
#pragma unroll
                for (int j = 0; j < 4; ++j) areg[i][j] = bload16(rA0, (a_ok[i] && k + 4 * j < p.K) ? base + 16u * j : OOB);
            } else {
                // implicit 3x3 im2col, tap-major K: k = tap*C + c (src/gemm_hl.cu:104-114)
                const int tap = a_tap[i], c0 = a_c0[i];
                const int ky = (tap * 11) >> 5, kx = tap - 3 * ky;
                const int iy = a_iy0[i] + ky, ix = a_ix0[i] + kx;
                const bool ok = a_ok[i] && tap < 9 && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W;
                const unsigned base = ((unsigned(a_base[i] + iy) * unsigned(p.W) + unsigned(ix)) * unsigned(p.C) + unsigned(c0)) * 4u;
#pragma unroll
                for (int j = 0; j < AREG; ++j) areg[i][j] = bload16(rA0, ok ? base + 16u * j : OOB);
                int nc = c0 + 64, ntap = tap;
                while (nc >= p.C) { nc -= p.C; ++ntap; }
                a_c0[i] = nc;
                a_tap[i] = ntap;
            }
        }
    };

    // the W tile is stored row-for-row here (gload already picked the permuted global rows)
    auto lstore = [&](int buf) {
        unsigned char* sW = smem + buf * T::STAGE;
        unsigned char* sAh = sW + BN * 64;
        unsigned char* sAl = sAh + BM * 64;
#pragma unroll
        for (int i = 0; i < T::WT; ++i) {
            const int c = tid + i * 256, row = c >> 2, kc = c & 3;
            *reinterpret_cast<v4i*>(sW + swz(row, kc)) = wreg[i];
        }
#pragma unroll
        for (int i = 0; i < T::AT; ++i) {
            v4i h, l;
            unsigned d[8];
            quant_pack16(areg[i], a_e[i], d);
            split16x16(d, h, l);
            const int off = swz(a_row[i], a_kc[i]);
            *reinterpret_cast<v4i*>(sAh + off) = h;
            *reinterpret_cast<v4i*>(sAl + off) = l;
        }
    };

    v4i acc_h[NS][MS], acc_l[NS][MS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            acc_h[ns][ms] = v4i{0, 0, 0, 0};
            acc_l[ns][ms] = v4i{0, 0, 0, 0};
        }

    auto compute = [&](int buf) {
        const unsigned char* sW = smem + buf * T::STAGE;
        const unsigned char* sAh = sW + BN * 64;
        const unsigned char* sAl = sAh + BM * 64;
        const int fr = lane & 15, fc = lane >> 4;
        v4i wf[NS], hf[MS], lf[MS];
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
            const int row = (FUSED ? wsub_row<EPI, T>(wn, ns) : (wn * NS + ns) * 16) + fr;
            wf[ns] = *reinterpret_cast<const v4i*>(sW + swz(row, fc));
        }
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            const int row = wm * T::WTM + ms * 16 + fr;
            hf[ms] = *reinterpret_cast<const v4i*>(sAh + swz(row, fc));
            lf[ms] = *reinterpret_cast<const v4i*>(sAl + swz(row, fc));
        }
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                acc_h[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ns], hf[ms], acc_h[ns][ms], 0, 0, 0);
                acc_l[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ns], lf[ms], acc_l[ns][ms], 0, 0, 0);
            }
    };

    // ---- main loop: global loads for step k+1 are in flight while step k runs on the MFMAs
    if (kb < ke) {
        gload(kb);
        lstore(0);
        __syncthreads();
        for (int kt = kb; kt < ke; ++kt) {
            const int cur = (kt - kb) & 1;
            const bool more = kt + 1 < ke;
            if (more) gload(kt + 1);
            compute(cur);
            if (more) lstore(cur ^ 1);
            __syncthreads();
        }
    }

    if constexpr (EPI == EPI_PARTIAL) {
        // columns in natural order: W rows were not permuted for partials
        store_partial<T>(p, acc_h, acc_l, rbase, n0 + wn * T::WTN, ti.ks);
    } else if constexpr (EPI == EPI_QKV) {
        qkv_epilogue<T>(p, acc_h, acc_l, rbase, n0, wn, er);
    } else {
        fused_epilogue<EPI, SRC, T>(p, acc_h, acc_l, rbase, n0, wn, sh, fl, er);
        if constexpr (EPI == EPI_PLAIN_GN) gn_flush(p, sh);
    }
}

// Split-K reduction and epilogue: one thread per (row, group of four output columns), numbered row by
// row over a flat grid so that every thread has work whatever the column count; sums the int32
// partials of all K ranges and applies the exact int64 epilogue.
template <int EPI>
__global__ void __launch_bounds__(256) splitk_epilogue_kernel(const GemmParams p) {
    prefetch_args();
    const int nout = EPI == EPI_GEGLU ? (p.Nreal >> 1) : p.Nreal;
    const int tpr = (nout + 3) >> 2;   // threads per row
    const unsigned total = unsigned(p.Mreal) * unsigned(tpr);
    const size_t plane = size_t(p.ws_rows) * p.ws_ld;
    for (unsigned idx = blockIdx.x * 256u + threadIdx.x; idx - threadIdx.x < total; idx += gridDim.x * 256u) {
        const bool live = idx < total;
        const int r = live ? int(idx / unsigned(tpr)) : 0;
        const int c0 = live ? int(idx - unsigned(r) * unsigned(tpr)) * 4 : 0;
        const bool full = c0 + 3 < nout;
        uint32_t mx = 0;
        if (live) {
            const int er = p.xrowmax ? rowexp_u32(p.xrowmax[r]) : (p.pm ? conv_window_shift(p, r) : (p.e ? p.e[r] : 0));
            // plane sums of ws columns [wc, wc + 4) over the K splits (16-byte loads: ws_ld % 4 == 0)
            auto sum4 = [&](int wc, v4i& h, v4i& l) {
                h = v4i{0, 0, 0, 0};
                l = v4i{0, 0, 0, 0};
#pragma unroll 4
                for (int s = 0; s < p.ksplit; ++s) {
                    const int32_t* b = p.ws + (size_t(s * 2) * p.ws_rows + r) * p.ws_ld + wc;
                    h += *reinterpret_cast<const v4i*>(b);
                    l += *reinterpret_cast<const v4i*>(b + plane);
                }
            };
            int y[4] = {0, 0, 0, 0};
            // the column constants of the thread's columns, loaded together ahead of the sums (columns
            // past the output read zeros and are not stored)
            constexpr int NC = EPI == EPI_GEGLU ? 8 : 4;
            int4 cs[NC];
            {
                const __amdgpu_buffer_rsrc_t rC = make_rsrc(p.cst, unsigned(p.Nreal) * 16u);
                const int cb0 = EPI == EPI_GEGLU ? 2 * c0 : c0;
#pragma unroll
                for (int j = 0; j < NC; ++j) {
                    const v4i t = bload16(rC, cb0 + j < p.Nreal ? unsigned(cb0 + j) * 16u : OOB);
                    cs[j] = make_int4(t[0], t[1], t[2], t[3]);
                }
            }
            if constexpr (EPI == EPI_GEGLU) {
                v4i h0, l0, h1, l1;
                sum4(2 * c0, h0, l0);       // columns a0 g0 a1 g1
                sum4(2 * c0 + 4, h1, l1);   // columns a2 g2 a3 g3
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int ah = v < 2 ? h0[2 * v] : h1[2 * v - 4], al = v < 2 ? l0[2 * v] : l1[2 * v - 4];
                    const int gh = v < 2 ? h0[2 * v + 1] : h1[2 * v - 3], gl = v < 2 ? l0[2 * v + 1] : l1[2 * v - 3];
                    const int4 ca = cs[2 * v], cg = cs[2 * v + 1];
                    y[v] = geglu_exact(epi1_exact(ah, al, ca.x, ca.y, ca.z, ca.w, er), epi1_exact(gh, gl, cg.x, cg.y, cg.z, cg.w, er), p.Lphi);
                }
            } else {
                v4i h, l;
                sum4(c0, h, l);
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int4 cc = cs[v];
                    int yy = epi1_exact(h[v], l[v], cc.x, cc.y, cc.z, cc.w, er);
                    if constexpr (EPI == EPI_GELU) yy = gelu_exact(yy, p.Lphi);
                    y[v] = yy;
                }
            }
            if constexpr (EPI == EPI_SPLIT3) {
                // Cs % 4 == 0: the four columns lie in one part
                const int part = c0 >= 2 * p.Cs ? 2 : (c0 >= p.Cs ? 1 : 0);
                int32_t* d = (part == 0 ? p.Y : (part == 1 ? p.Y1 : p.Y2)) + size_t(r) * p.Cs + (c0 - part * p.Cs);
                if (full && p.vec_store) *reinterpret_cast<v4i*>(d) = v4i{y[0], y[1], y[2], y[3]};
                else
                    for (int v = 0; v < 4 && c0 + v < nout; ++v) d[v] = y[v];
            } else {
                int32_t* d = p.Y + size_t(r) * p.ldy + c0;
                if constexpr (EPI != EPI_GEGLU) {
                    if (p.R) {
                        const int32_t* rp = p.R + size_t(r) * p.ldy + c0;
                        if (full && p.vec_store) {
                            const v4i rv = *reinterpret_cast<const v4i*>(rp);
#pragma unroll
                            for (int v = 0; v < 4; ++v) y[v] = add_sat(y[v], rv[v]);
                        } else {
                            for (int v = 0; v < 4 && c0 + v < nout; ++v) y[v] = add_sat(y[v], rp[v]);
                        }
                    }
                }
                if (full && p.vec_store) *reinterpret_cast<v4i*>(d) = v4i{y[0], y[1], y[2], y[3]};
                else
                    for (int v = 0; v < 4 && c0 + v < nout; ++v) d[v] = y[v];
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (c0 + v < nout) mx = max(mx, uabs(y[v]));
            }
        }
        if (EPI != EPI_SPLIT3 && p.rowmax) {
            // one atomic per wave when the wave's lanes share a row, else one per lane
            const int r0 = __shfl(r, 0), r63 = __shfl(r, 63);
            if (r0 == r63) {
#pragma unroll
                for (int o = 32; o; o >>= 1) mx = max(mx, uint32_t(__shfl_xor(int(mx), o)));
                if ((threadIdx.x & 63) == 0 && mx) atomicMax(p.rowmax + r, mx);
            } else if (live && mx) {
                atomicMax(p.rowmax + r, mx);
            }
        }
    }
}

// ---------------------------------------------------------------- host-side launches

template <int SRC, int EPI, class T>
hipError_t launch_dma_t(const GemmParams& p, int batch, hipStream_t st) {
    dim3 grid(unsigned(p.mtiles * p.ntiles * p.ksplit), unsigned(batch));
    hipLaunchKernelGGL((gemm_dma_kernel<SRC, EPI, T>), grid, dim3(T::NT), 0, st, p);
    return hipGetLastError();
}

template <int SRC, int EPI, class T>
hipError_t launch_reg_t(const GemmParams& p, int batch, hipStream_t st) {
    dim3 grid(unsigned(p.mtiles * p.ntiles * p.ksplit), unsigned(batch));
    hipLaunchKernelGGL((gemm_hl_kernel<SRC, EPI, T>), grid, dim3(256), 0, st, p);
    return hipGetLastError();
}

template <int SRC, class T, bool DMA>
hipError_t launch_gemm_epi(int epi, const GemmParams& p, int batch, hipStream_t st) {
#define VK_LAUNCH(E)                                       \
    [&]() {                                                \
        if constexpr (DMA) return launch_dma_t<SRC, E, T>(p, batch, st); \
        else return launch_reg_t<SRC, E, T>(p, batch, st); \
    }()
    switch (epi) {
    case EPI_PLAIN: return VK_LAUNCH(EPI_PLAIN);
    case EPI_PLAIN_GN: return VK_LAUNCH(EPI_PLAIN_GN);
    case EPI_SPLIT3: return VK_LAUNCH(EPI_SPLIT3);
    case EPI_GEGLU: return VK_LAUNCH(EPI_GEGLU);
    case EPI_GELU: return VK_LAUNCH(EPI_GELU);
    case EPI_PARTIAL: return VK_LAUNCH(EPI_PARTIAL);
    case EPI_QKV:
        // whole heads per wave: the 128 x 128 tiles only (the host selects variant 0)
        if constexpr (std::is_same<T, TileD0>::value || std::is_same<T, TileV0>::value) return VK_LAUNCH(EPI_QKV);
        else return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
#undef VK_LAUNCH
}

// variant -> tile: 0 = 128x128, 1 = 64x128, 2 = 128x64 (rows x columns)
template <int SRC>
hipError_t launch_gemm_src(int variant, int epi, const GemmParams& p, int batch, hipStream_t st) {
    constexpr bool DMA = SRC == SRC_I8 || SRC == SRC_I16 || SRC == SRC_CONV16;
    if constexpr (DMA) {
        switch (variant) {
        case 1: return launch_gemm_epi<SRC, TileD1, true>(epi, p, batch, st);
        case 2: return launch_gemm_epi<SRC, TileD2, true>(epi, p, batch, st);
        case 3: return launch_gemm_epi<SRC, TileD3, true>(epi, p, batch, st);
        default: return launch_gemm_epi<SRC, TileD0, true>(epi, p, batch, st);
        }
    } else {
        // int32 images with C % 64 == 0 and int32 rows with K % 4 == 0: 64 x 128 tiles on the DMA
        // kernel (raw int32 rows in LDS)
        if constexpr (SRC == SRC_CONV32)
            if (variant == 1 && (p.C & 63) == 0) return launch_gemm_epi<SRC, TileD1, true>(epi, p, batch, st);
        if constexpr (SRC == SRC_X32)
            if (variant == 1 && (p.K & 3) == 0) return launch_gemm_epi<SRC, TileD1, true>(epi, p, batch, st);
        switch (variant) {
        case 1: return launch_gemm_epi<SRC, TileV1, false>(epi, p, batch, st);
        case 2: return launch_gemm_epi<SRC, TileV2, false>(epi, p, batch, st);
        default: return launch_gemm_epi<SRC, TileV0, false>(epi, p, batch, st);
        }
    }
}

hipError_t launch_gemm_i8(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_x32(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_conv32(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_i16(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_conv16(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_raw(int variant, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_raw_reduce(const int32_t* ws, int splits, long long plane, int ldw, int M, int N, int32_t* C, int ldc, hipStream_t st);
hipError_t launch_splitk_epilogue(int epi, const GemmParams& p, hipStream_t st);

}  // namespace vk

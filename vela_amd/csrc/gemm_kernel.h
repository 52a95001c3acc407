// The W8A16 hi/lo-split GEMM kernel for gfx950 (CDNA4), templated on the A source, the epilogue
// and the tile shape. Each source file gemm_src_*.hip instantiates it for one source.
//
// Block = 256 threads = 4 wave64s, each wave owning a (BM/WM) x (BN/WN) output sub-tile. Per 64-wide
// K step every thread loads its share of the W tile and of the A tile from HBM with buffer loads
// (out-of-range offsets read as zero: pad rows/columns and the image border of the implicit im2col
// cost no branches), splits int16 activations into a signed hi byte and an offset lo byte
// (lo - 128 = (q & 255) ^ 0x80) with byte permutes, and stores the three int8 planes (W, hi, lo)
// to an XOR-swizzled, double-buffered LDS stage. The MFMA v_mfma_i32_16x16x64_i8 takes W as its A
// operand and the activations as its B operand, so each lane ends up holding four consecutive output
// columns of one output row; one W fragment feeds both activation planes.
//
// Epilogue: acc = 256*Chi + Clo + 128*wsum, y = sat32(rshr(acc*m, s-e) + b) (src/gemm_hl.cu:40-52).
// When the block's columns satisfy Kp*|m| < 2^30 (so |acc*m| < 2^52) and every shift s-e lies in
// [1, 52], the epilogue runs in FP64, where it is exact: acc*m*2^-(s-e) + 1/2 is a dyadic rational
// with a numerator below 2^53, one FMA produces it without rounding, and floor() then gives the
// rounding shift. Otherwise it runs the reference's int64 formula element by element.
#pragma once
#include <climits>

#include "vk_common.h"

namespace vk {

template <int BM_, int BN_, int WM_, int WN_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
    static constexpr int WTM = BM / WM, WTN = BN / WN;   // wave sub-tile (rows x columns)
    static constexpr int MS = WTM / 16, NS = WTN / 16;   // 16x16 MFMA tiles per wave
    static constexpr int WT = BN * 4 / 256;              // 16-byte W chunks per thread per K step
    static constexpr int AT = BM * 4 / 256;              // 16-value A chunks per thread per K step
    static constexpr int STAGE = (BN + 2 * BM) * 64;     // LDS bytes per stage: W, hi, lo planes
    static_assert(WM * WN == 4, "four waves");
    static_assert(MS >= 1 && NS >= 2 && (NS % 2) == 0, "wave tile");
    static_assert(WT >= 1 && AT >= 1 && (BN * 4) % 256 == 0 && (BM * 4) % 256 == 0, "loader mapping");
};

typedef Tile<128, 128, 2, 2> TileV0;   // 128 rows x 128 columns
typedef Tile<64, 128, 1, 4> TileV1;    //  64 rows x 128 columns
typedef Tile<128, 64, 2, 2> TileV2;    // 128 rows x  64 columns

// byte offset of 16-byte chunk `chunk` (0..3) of LDS row `row` (64 bytes per row); the XOR keeps
// the 16 rows read by one MFMA fragment load on 16 distinct bank groups
__device__ __forceinline__ int swz(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4); }

// LDS row of W-tile row `row`. For GEGLU the a-columns (even) go to the first half and the
// g-columns (odd) to the second half, so a wave's a- and g-subtiles hold matching columns.
template <int EPI, int BN>
__device__ __forceinline__ int wrow_lds(int row) {
    if constexpr (EPI == EPI_GEGLU) return (row & 1) ? (BN / 2 + (row >> 1)) : (row >> 1);
    else return row;
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

// 16 int32 values quantised with shift e (quant16_32), packed to int16 pairs
__device__ __forceinline__ void quant_pack16(const v4i* x, int e, unsigned* d) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q0 = quant16_32(x[j >> 1][(2 * j) & 3], e);
        const int q1 = quant16_32(x[j >> 1][(2 * j + 1) & 3], e);
        d[j] = __builtin_amdgcn_perm(unsigned(q1), unsigned(q0), 0x05040100u);
    }
}

// 16 int16 values of an image quantised with shift e, packed back to int16 pairs
__device__ __forceinline__ void quant16_pairs(const v4i* x, int e, unsigned* d) {
    if (e == 0) {
        // quant16_32(v, 0) = max(v, -32767) for int16 v
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // copy the vector element to a scalar first: this compiler folds __builtin_bit_cast of
            // an ext-vector subscript to element 0 of the vector
            const int w = x[j >> 2][j & 3];
            s2 v = __builtin_bit_cast(s2, w);
            v = __builtin_elementwise_max(v, s2{-32767, -32767});
            d[j] = __builtin_bit_cast(unsigned, v);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int w = x[j >> 2][j & 3];
            const int q0 = quant16_32(int(short(w & 0xffff)), e);
            const int q1 = quant16_32(w >> 16, e);
            d[j] = __builtin_amdgcn_perm(unsigned(q1), unsigned(q0), 0x05040100u);
        }
    }
}

template <int SRC, int EPI, class T>
__global__ void __launch_bounds__(256) gemm_hl_kernel(const GemmParams p) {
    constexpr int BM = T::BM, BN = T::BN, MS = T::MS, NS = T::NS;
    constexpr bool TWO = EPI != EPI_RAW;                            // two activation planes
    constexpr bool FUSED = EPI != EPI_PARTIAL && EPI != EPI_RAW;     // requantising epilogue here
    constexpr bool NEEDLUT = EPI == EPI_GEGLU || EPI == EPI_GELU;
    constexpr int AREG = (SRC == SRC_X32 || SRC == SRC_CONV32) ? 4 : 2;   // 16-byte loads per A chunk
    constexpr bool CONV = SRC == SRC_CONV32 || SRC == SRC_CONV16;

    __shared__ __attribute__((aligned(16))) unsigned char smem[2 * T::STAGE];
    __shared__ __attribute__((aligned(16))) double s_ms[FUSED ? BN : 1];
    __shared__ __attribute__((aligned(16))) double s_wm[FUSED ? BN : 1];
    __shared__ __attribute__((aligned(16))) double s_wmh[FUSED ? BN : 1];
    __shared__ __attribute__((aligned(16))) int s_b[FUSED ? BN : 1];
    __shared__ int2 s_lut[NEEDLUT ? 2050 : 1];
    __shared__ int s_flag[6];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % T::WM, wn = wave / T::WM;

    // ---- tile of this block. Blocks are dispatched round-robin over the 8 XCDs; renumber them so
    // that each XCD receives a contiguous range of tiles (neighbouring column tiles of one row
    // stripe share the A stripe in that XCD's L2).
    const int nblk = gridDim.x, bid = blockIdx.x;
    const int q8 = nblk >> 3, r8 = nblk & 7, xcd = bid & 7, slot = bid >> 3;
    const int lin = (xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8) + slot;
    const int ks = lin % p.ksplit, tl = lin / p.ksplit;
    const int mt = tl / p.ntiles, nt = tl - mt * p.ntiles;
    const int m0 = mt * BM, n0 = nt * BN;
    const int nK = (p.Kp + 63) >> 6;
    const int kb = ks * p.kper, ke = min(nK, kb + p.kper);

    const int bt = blockIdx.y;   // batch index (EPI_RAW)
    const char* a0p = static_cast<const char*>(p.a0) + (EPI == EPI_RAW ? bt * p.sA : 0);
    const int8_t* wp = p.w + (EPI == EPI_RAW ? bt * p.sW : 0);
    const __amdgpu_buffer_rsrc_t rW = make_rsrc(wp, p.w_bytes);
    const __amdgpu_buffer_rsrc_t rA0 = make_rsrc(a0p, p.a0_bytes);
    const __amdgpu_buffer_rsrc_t rA1 = make_rsrc(SRC == SRC_I8 && TWO ? p.a1 : a0p, SRC == SRC_I8 && TWO ? p.a1_bytes : p.a0_bytes);

    // ---- block prologue: epilogue constants, GELU table, and the exactness conditions of the
    // FP64 epilogue over this block's rows and columns
    bool fast = true, ezero = true;
    if constexpr (FUSED) {
        if (tid == 0) {
            s_flag[0] = INT_MAX; s_flag[1] = INT_MIN; s_flag[2] = INT_MAX; s_flag[3] = INT_MIN;
            s_flag[4] = 0; s_flag[5] = 0;
        }
        __syncthreads();
        if (tid < BM) {
            const int r = m0 + tid;
            if (r < p.Mreal) {
                const int er = SRC == SRC_X32 ? rowexp_u32(p.xrowmax[r]) : (p.e ? p.e[r] : 0);
                atomicMin(&s_flag[0], er);
                atomicMax(&s_flag[1], er);
            }
        }
        if (tid < BN) {
            const int j = tid;
            const int n = EPI == EPI_GEGLU ? n0 + (j < BN / 2 ? 2 * j : 2 * (j - BN / 2) + 1) : n0 + j;
            double ms = 0.0, wmv = 0.0, wmh = 0.5;
            int bb = 0;
            if (n < p.Nreal) {
                const int4 c = p.cst[n];
                const i64 mag = (c.x < 0 ? -i64(c.x) : i64(c.x)) * i64(p.Kp);
                if (mag >= (1LL << 30)) atomicOr(&s_flag[4], 1);
                atomicMin(&s_flag[2], c.y);
                atomicMax(&s_flag[3], c.y);
                if (c.y >= -1000 && c.y <= 1000) {
                    ms = ldexp(double(c.x), -c.y);
                    wmv = ldexp(128.0 * (double(c.w) * double(c.x)), -c.y);
                    wmh = wmv + 0.5;
                }
                bb = c.z;
            }
            s_ms[j] = ms; s_wm[j] = wmv; s_wmh[j] = wmh; s_b[j] = bb;
        }
        if constexpr (NEEDLUT) {
            // s_lut[i + 1] = (L[i], L[i+1] - L[i]) for i in [0, 2048); s_lut[0] serves arguments
            // below the table (value 0) and s_lut[2049] arguments at or above its end (65536)
            for (int i = tid; i < 2050; i += 256) {
                int2 v;
                if (i == 0) v = make_int2(0, 0);
                else if (i == 2049) v = make_int2(65536, 0);
                else {
                    const int a = p.Lphi[i - 1], nx = p.Lphi[i];
                    v = make_int2(a, nx - a);
                    if (a < 0 || a > 65536 || nx < 0 || nx > 65536) atomicOr(&s_flag[5], 1);
                }
                s_lut[i] = v;
            }
        }
        __syncthreads();
        const i64 emin = s_flag[0], emax = s_flag[1], smin = s_flag[2], smax = s_flag[3];
        fast = !s_flag[4] && (smin - emax >= 1) && (smax - emin <= 52);
        if (NEEDLUT && s_flag[5]) fast = false;
        ezero = emin > emax || (emin == 0 && emax == 0);
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
        if constexpr (SRC == SRC_X32) a_e[i] = a_ok[i] ? rowexp_u32(p.xrowmax[r]) : 0;
        if constexpr (CONV) {
            a_e[i] = (a_ok[i] && p.e) ? p.e[r] : 0;
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
            const int n = n0 + row, k = kbase + kc * 16;
            const unsigned off = (n < p.Nreal && k < p.Kp) ? unsigned(n) * unsigned(p.ldw) + unsigned(k) : OOB;
            wreg[i] = bload16(rW, off);
        }
#pragma unroll
        for (int i = 0; i < T::AT; ++i) {
            const int r = m0 + a_row[i], k = kbase + a_kc[i] * 16;
            if constexpr (SRC == SRC_I8) {
                const unsigned off = (a_ok[i] && k < p.Kp) ? unsigned(r) * unsigned(p.lda) + unsigned(k) : OOB;
                areg[i][0] = bload16(rA0, off);
                if constexpr (TWO) areg[i][1] = bload16(rA1, off);
            } else if constexpr (SRC == SRC_I16) {
                const unsigned base = (unsigned(r) * unsigned(p.lda) + unsigned(k)) * 2u;
                areg[i][0] = bload16(rA0, (a_ok[i] && k < p.K) ? base : OOB);
                areg[i][1] = bload16(rA0, (a_ok[i] && k + 8 < p.K) ? base + 16u : OOB);
            } else if constexpr (SRC == SRC_X32) {
                const unsigned base = (unsigned(r) * unsigned(p.lda) + unsigned(k)) * 4u;
#pragma unroll
                for (int j = 0; j < 4; ++j) areg[i][j] = bload16(rA0, (a_ok[i] && k + 4 * j < p.K) ? base + 16u * j : OOB);
            } else {
                // implicit 3x3 im2col, tap-major K: k = tap*C + c (src/gemm_hl.cu:104-114)
                const int tap = a_tap[i], c0 = a_c0[i];
                const int ky = (tap * 11) >> 5, kx = tap - 3 * ky;   // tap / 3, tap % 3 for tap < 9
                const int iy = a_iy0[i] + ky, ix = a_ix0[i] + kx;
                const bool ok = a_ok[i] && tap < 9 && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W;
                constexpr unsigned ES = SRC == SRC_CONV32 ? 4u : 2u;
                const unsigned base = ((unsigned(a_base[i] + iy) * unsigned(p.W) + unsigned(ix)) * unsigned(p.C) + unsigned(c0)) * ES;
#pragma unroll
                for (int j = 0; j < AREG; ++j) areg[i][j] = bload16(rA0, ok ? base + 16u * j : OOB);
                int nc = c0 + 64, ntap = tap;
                while (nc >= p.C) { nc -= p.C; ++ntap; }
                a_c0[i] = nc;
                a_tap[i] = ntap;
            }
        }
    };

    auto lstore = [&](int buf) {
        unsigned char* sW = smem + buf * T::STAGE;
        unsigned char* sAh = sW + BN * 64;
        unsigned char* sAl = sAh + BM * 64;
#pragma unroll
        for (int i = 0; i < T::WT; ++i) {
            const int c = tid + i * 256, row = c >> 2, kc = c & 3;
            const int lr = FUSED ? wrow_lds<EPI, BN>(row) : row;
            *reinterpret_cast<v4i*>(sW + swz(lr, kc)) = wreg[i];
        }
#pragma unroll
        for (int i = 0; i < T::AT; ++i) {
            v4i h, l;
            if constexpr (SRC == SRC_I8) {
                h = areg[i][0];
                if constexpr (TWO) l = areg[i][1];
            } else {
                unsigned d[8];
                if constexpr (SRC == SRC_I16) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) d[j] = unsigned(areg[i][j >> 2][j & 3]);
                } else if constexpr (SRC == SRC_CONV16) {
                    quant16_pairs(areg[i], a_e[i], d);
                } else {
                    quant_pack16(areg[i], a_e[i], d);
                }
                split16x16(d, h, l);
            }
            const int off = swz(a_row[i], a_kc[i]);
            *reinterpret_cast<v4i*>(sAh + off) = h;
            if constexpr (TWO) *reinterpret_cast<v4i*>(sAl + off) = l;
        }
    };

    v4i acc_h[NS][MS], acc_l[TWO ? NS : 1][TWO ? MS : 1];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            acc_h[ns][ms] = v4i{0, 0, 0, 0};
            if constexpr (TWO) acc_l[ns][ms] = v4i{0, 0, 0, 0};
        }

    auto compute = [&](int buf) {
        const unsigned char* sW = smem + buf * T::STAGE;
        const unsigned char* sAh = sW + BN * 64;
        const unsigned char* sAl = sAh + BM * 64;
        const int fr = lane & 15, fc = lane >> 4;
        v4i wf[NS], hf[MS], lf[TWO ? MS : 1];
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
            const int row = (FUSED ? wsub_row<EPI, T>(wn, ns) : (wn * NS + ns) * 16) + fr;
            wf[ns] = *reinterpret_cast<const v4i*>(sW + swz(row, fc));
        }
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            const int row = wm * T::WTM + ms * 16 + fr;
            hf[ms] = *reinterpret_cast<const v4i*>(sAh + swz(row, fc));
            if constexpr (TWO) lf[ms] = *reinterpret_cast<const v4i*>(sAl + swz(row, fc));
        }
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                acc_h[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ns], hf[ms], acc_h[ns][ms], 0, 0, 0);
                if constexpr (TWO) acc_l[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ns], lf[ms], acc_l[ns][ms], 0, 0, 0);
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

    // ---- epilogues
    const int fr = lane & 15, fg = lane >> 4;
    if constexpr (EPI == EPI_PARTIAL) {
        // int32 partial sums of this K range: ws[(ks*2 + plane) * ws_rows + row][col]
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                const int r = m0 + wm * T::WTM + ms * 16 + fr;
                const int n = n0 + (wn * NS + ns) * 16 + 4 * fg;
                int32_t* dh = p.ws + (size_t(ks * 2) * p.ws_rows + r) * p.ws_ld + n;
                int32_t* dl = dh + size_t(p.ws_rows) * p.ws_ld;
                *reinterpret_cast<v4i*>(dh) = acc_h[ns][ms];
                *reinterpret_cast<v4i*>(dl) = acc_l[ns][ms];
            }
        return;
    } else if constexpr (EPI == EPI_RAW) {
        int32_t* C = p.Y + bt * p.sC;
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                const int r = m0 + wm * T::WTM + ms * 16 + fr;
                const int n = n0 + (wn * NS + ns) * 16 + 4 * fg;
                if (r >= p.Mreal) continue;
                int32_t* d = C + size_t(r) * p.ldy + n;
                if (p.vec_store && n + 3 < p.Nreal) {
                    *reinterpret_cast<v4i*>(d) = acc_h[ns][ms];
                } else {
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        if (n + v < p.Nreal) d[v] = acc_h[ns][ms][v];
                }
            }
        return;
    } else {
        // per-lane row shifts
        int er[MS];
        double pr[MS];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            const int r = m0 + wm * T::WTM + ms * 16 + fr;
            er[ms] = 0;
            if (r < p.Mreal) er[ms] = SRC == SRC_X32 ? rowexp_u32(p.xrowmax[r]) : (p.e ? p.e[r] : 0);
            pr[ms] = ldexp(1.0, er[ms] > 1000 ? 1000 : (er[ms] < -1000 ? -1000 : er[ms]));
        }
        const bool smallK = p.Kp <= 496;   // |256*Chi + Clo| < 2^31
        uint32_t mx[MS];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) mx[ms] = 0;

        // A = 256*Chi + Clo as an exact double
        auto comb = [&](int h, int l) -> double {
            if (smallK) return double((h << 8) + l);
            return __builtin_fma(double(h), 256.0, double(l));
        };
        // floor(acc*m*2^-(s-e) + 1/2) saturated, + b saturated: exact under the block conditions
        auto epi_fast = [&](double A, double ms_, double wm_, double wmh_, int b_, double prr) -> int {
            const double X = ezero ? __builtin_fma(A, ms_, wmh_) : __builtin_fma(__builtin_fma(A, ms_, wm_), prr, 0.5);
            return add_sat(cvt_sat(__builtin_floor(X)), b_);
        };
        // GELU factor table lookup (lut16i) for 0 <= L <= 65536
        auto phi = [&](int x) -> int {
            const int z = min(max(x, -1048577), 1048576) + 1048576;   // [-1, 2^21]
            const int2 t = s_lut[(z >> 10) + 1];
            return t.x + (__mul24(t.y, z & 1023) >> 10);
        };
        // sat32(rshr(y * phi(y), 16)) for 0 <= phi <= 65536: never saturates
        auto gelu_fast = [&](int y) -> double {
            const double P = __builtin_fma(double(y), double(phi(y)), 32768.0);
            return __builtin_floor(P * (1.0 / 65536.0));
        };

        constexpr int NOUT = EPI == EPI_GEGLU ? NS / 2 : NS;
#pragma unroll
        for (int ns = 0; ns < NOUT; ++ns) {
            const int lr = wsub_row<EPI, T>(wn, ns) + 4 * fg;   // table row of this lane's 4 columns
            const int lg = EPI == EPI_GEGLU ? wsub_row<EPI, T>(wn, ns + NS / 2) + 4 * fg : lr;
            double c_ms[4], c_wm[4], c_wmh[4], g_ms[4], g_wm[4], g_wmh[4];
            int c_b[4], g_b[4];
            if (fast) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    c_ms[v] = s_ms[lr + v]; c_wm[v] = s_wm[lr + v]; c_wmh[v] = s_wmh[lr + v]; c_b[v] = s_b[lr + v];
                    if constexpr (EPI == EPI_GEGLU) { g_ms[v] = s_ms[lg + v]; g_wm[v] = s_wm[lg + v]; g_wmh[v] = s_wmh[lg + v]; g_b[v] = s_b[lg + v]; }
                }
            }
            // output column of value v: n0 + lr + v (plain); (n0 >> 1) + lr + v (GEGLU, lr < BN/2)
            const int ncol = EPI == EPI_GEGLU ? (n0 >> 1) + lr : n0 + lr;
            const int nlim = EPI == EPI_GEGLU ? (p.Nreal >> 1) : p.Nreal;
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                const int r = m0 + wm * T::WTM + ms * 16 + fr;
                if (r >= p.Mreal || ncol >= nlim) continue;
                int y[4];
                if (fast) {
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
                const bool full = ncol + 3 < nlim;
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
                            if (ncol + v < nlim) mx[ms] = max(mx[ms], uabs(y[v]));
                    }
                }
            }
        }
        if constexpr (EPI != EPI_SPLIT3) {
            if (p.rowmax) {
                // lanes fr, fr+16, fr+32, fr+48 hold the same row: one atomic per row and wave
#pragma unroll
                for (int ms = 0; ms < MS; ++ms) {
                    uint32_t m = mx[ms];
                    m = max(m, uint32_t(__shfl_xor(int(m), 16)));
                    m = max(m, uint32_t(__shfl_xor(int(m), 32)));
                    const int r = m0 + wm * T::WTM + ms * 16 + fr;
                    if (fg == 0 && r < p.Mreal && m) atomicMax(p.rowmax + r, m);
                }
            }
        }
    }
}

// Split-K reduction and epilogue: one thread per row and group of four output columns; sums the
// int32 partials of all K ranges and applies the exact int64 epilogue.
template <int EPI>
__global__ void __launch_bounds__(256) splitk_epilogue_kernel(const GemmParams p) {
    const int nout = EPI == EPI_GEGLU ? (p.Nreal >> 1) : p.Nreal;
    const int groups = (nout + 3) >> 2;
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const int r = int(idx / groups), g = int(idx - (long long)r * groups);
    if (r >= p.Mreal) return;
    const int er = p.xrowmax ? rowexp_u32(p.xrowmax[r]) : (p.e ? p.e[r] : 0);
    const size_t plane = size_t(p.ws_rows) * p.ws_ld;
    auto sum = [&](int col, int& h, int& l) {
        int sh = 0, sl = 0;
        for (int s = 0; s < p.ksplit; ++s) {
            const int32_t* b = p.ws + (size_t(s * 2) * p.ws_rows + r) * p.ws_ld + col;
            sh += b[0];
            sl += b[plane];
        }
        h = sh; l = sl;
    };
    uint32_t mx = 0;
    for (int v = 0; v < 4; ++v) {
        const int c = g * 4 + v;
        if (c >= nout) break;
        int y;
        if constexpr (EPI == EPI_GEGLU) {
            int ah, al, gh, gl;
            sum(2 * c, ah, al);
            sum(2 * c + 1, gh, gl);
            const int4 ca = p.cst[2 * c], cg = p.cst[2 * c + 1];
            y = geglu_exact(epi1_exact(ah, al, ca.x, ca.y, ca.z, ca.w, er), epi1_exact(gh, gl, cg.x, cg.y, cg.z, cg.w, er), p.Lphi);
            p.Y[size_t(r) * p.ldy + c] = y;
        } else {
            int h, l;
            sum(c, h, l);
            const int4 cc = p.cst[c];
            y = epi1_exact(h, l, cc.x, cc.y, cc.z, cc.w, er);
            if constexpr (EPI == EPI_GELU) y = gelu_exact(y, p.Lphi);
            if constexpr (EPI == EPI_SPLIT3) {
                const int part = c >= 2 * p.Cs ? 2 : (c >= p.Cs ? 1 : 0);
                int32_t* d = part == 0 ? p.Y : (part == 1 ? p.Y1 : p.Y2);
                d[size_t(r) * p.Cs + (c - part * p.Cs)] = y;
                continue;
            } else {
                if (p.R) y = add_sat(y, p.R[size_t(r) * p.ldy + c]);
                p.Y[size_t(r) * p.ldy + c] = y;
            }
        }
        mx = max(mx, uabs(y));
    }
    if (EPI != EPI_SPLIT3 && p.rowmax && mx) atomicMax(p.rowmax + r, mx);
}

// host-side launch of one instantiation
template <int SRC, int EPI, class T>
hipError_t launch_gemm_t(const GemmParams& p, int batch, hipStream_t st) {
    dim3 grid(unsigned(p.mtiles * p.ntiles * p.ksplit), unsigned(batch));
    hipLaunchKernelGGL((gemm_hl_kernel<SRC, EPI, T>), grid, dim3(256), 0, st, p);
    return hipGetLastError();
}

template <int SRC, class T>
hipError_t launch_gemm_epi(int epi, const GemmParams& p, int batch, hipStream_t st) {
    switch (epi) {
    case EPI_PLAIN: return launch_gemm_t<SRC, EPI_PLAIN, T>(p, batch, st);
    case EPI_SPLIT3: return launch_gemm_t<SRC, EPI_SPLIT3, T>(p, batch, st);
    case EPI_GEGLU: return launch_gemm_t<SRC, EPI_GEGLU, T>(p, batch, st);
    case EPI_GELU: return launch_gemm_t<SRC, EPI_GELU, T>(p, batch, st);
    case EPI_PARTIAL: return launch_gemm_t<SRC, EPI_PARTIAL, T>(p, batch, st);
    default: return hipErrorInvalidValue;
    }
}

template <int SRC>
hipError_t launch_gemm_src(int variant, int epi, const GemmParams& p, int batch, hipStream_t st) {
    switch (variant) {
    case 1: return launch_gemm_epi<SRC, TileV1>(epi, p, batch, st);
    case 2: return launch_gemm_epi<SRC, TileV2>(epi, p, batch, st);
    default: return launch_gemm_epi<SRC, TileV0>(epi, p, batch, st);
    }
}

// declared here, defined in the per-source translation units
hipError_t launch_gemm_i8(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_x32(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_conv32(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_i16(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_conv16(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_raw(int variant, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_splitk_epilogue(int epi, const GemmParams& p, hipStream_t st);

}  // namespace vk

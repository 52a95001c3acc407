// Row-stationary ("stripe") hi/lo GEMM for shallow K (Kp <= 320) with int16 rows (SRC_I16) or int8
// planes (SRC_I8), epilogues PLAIN (+ residual), GEGLU and GELU, with or without the row maximum.
//
// A block owns 128 activation rows (32 per wave) and a range of W rows (output columns). Each wave
// loads its rows once, splits them into hi/lo MFMA fragments and keeps those in registers for the
// whole block; W streams through LDS in chunks of 64 rows (a 2-stage ring filled by buffer-load
// DMA), and each chunk is multiplied and requantised before the next. So an activation row is read
// and split once per block, the GELU table and the per-column constants are set up once per block,
// and the row maximum needs one atomic per row and wave at the end.
//
// MFMA: v_mfma_i32_32x32x32_i8 with the activations as the A operand and W as the B operand, so lane
// l holds output column l % 32 of a 32-column subtile for rows 8g + 4(l / 32) + v (g, v = 0..3): the
// per-column constants of a lane are one LDS read per chunk, and each output store instruction
// writes two 128-byte row segments.
//
// Epilogue (src/gemm_hl.cu:40-52, 279-302), two exact forms chosen per block:
//  * integer: every row has e == 0, every shift s lies in [0, 31] and no element can saturate
//    (checked from max |m| 2^-s and max |b|). Then y = (A m + C) >> s with A = 256 Chi + Clo
//    (int32, Kp <= 496) and C = 128 wsum m + 2^(s-1) + b 2^s, one v_mad_i64_i32 and one funnel
//    shift; for GELU/GEGLU, whose epilogue is VALU-bound, 2 |m| < 2^s as well (the reference's
//    multipliers lie in [2^14, 2^15), its shifts at 16 and above), and y is the high word of one
//    v_mad_i64_i32 of A, m 2^(32-s) and C 2^(32-s) (the table holds both pre-shifted); GELU/GEGLU take phi(g) from the table as (1024 L[i] + (L[i+1] - L[i]) f) >> 10, then
//    ge = (g phi + 2^15) >> 16 (never saturates, phi <= 65536) and y = sat32((a ge + 2^15) >> 16).
//  * otherwise the reference's int64 formula element by element (one element per loop iteration,
//    so that this rarely used form adds few registers to the kernel). The host sends calls with
//    per-row shifts to the tile kernels, whose FP64 form covers them at speed.
//
// Chunk loop of the integer form (calls without a residual): software-pipelined. Chunk c's MFMAs run
// in two halves (one 32-column subtile each), interleaved instruction by instruction with the
// requantising epilogue of chunk c - 1, whose plane sums were folded into one int32 per element
// (256 Chi + Clo) when its MFMAs finished; the epilogue has no branch (a saturating GEGLU product is
// clamped per element), so each half is one scheduling region ordered as one MFMA, a few VALU
// instructions and one LDS read, repeated. The int64 form and residual calls keep the plain loop:
// a chunk's MFMAs, then its epilogue.
//
// Set-up order: the column constants, the GELU table DMA and chunk cb's W DMA are issued before the
// activation rows, a fixed number of loads per lane, so that the set-up (table expansion, bounds
// checks, column table) waits for its own data and runs while the rows are in flight.
//
// Memory ordering: the W DMA of chunk c + 1 is issued right after the barrier of chunk c, and the
// only vector-memory instructions after it in chunk c are that chunk's output stores, a fixed
// number per lane (every lane stores unconditionally; rows and columns outside the output go to
// an out-of-range buffer offset, which the hardware drops). So waiting for at most that many
// outstanding operations completes the DMA. Residual loads (integer form) are consumed before the
// chunk's last stores, so they do not change that count; blocks of the int64 form, whose epilogue
// loads from memory element by element, wait for all operations instead.
#pragma once
#include <type_traits>

#include "gemm_kernel.h"

namespace vk {

typedef int v16i __attribute__((ext_vector_type(16)));

struct StripeCfg {
    static constexpr int BM = 128;                  // rows per block: four waves of 32
    static constexpr int NKS = 10;                  // 32-deep K substeps held in registers (Kp <= 320)
    static constexpr int CH = 64;                   // W rows per chunk
    static constexpr int NSUB = CH / 32;            // 32-column MFMA subtiles per chunk
    static constexpr int KSTEP = CH * 64;           // LDS bytes of one 64-deep K step of a chunk
    static constexpr int STAGE = (NKS / 2) * KSTEP; // LDS bytes of one chunk
    static constexpr int NCOLS = 1280;              // W rows (table columns) per block, at most
    static constexpr int CPT = NCOLS / 256;         // table columns per thread
    static constexpr int DMA_INS = STAGE / 1024 / 4;// DMA instructions per wave per chunk
    static constexpr int EB_GEGLU = 4;              // GEGLU outputs computed together (8: spills)
    static_assert(STAGE % 4096 == 0, "stripe geometry");
};

template <bool LUT>
struct StripeShared {
    unsigned char w[2][StripeCfg::STAGE];
    int4 tab[StripeCfg::NCOLS];   // per column {m, C lo, C hi, s} of the integer form (GELU/GEGLU: m and C times 2^(32-s))
    // lut[i + 1] = (1024 L[i] - d 1024 (i - 1024) mod 2^32, d = L[i+1] - L[i]); lut[0] below, lut[2049]
    // above the table: 1024 phi(x) = lut[j].x + lut[j].y x (mod 2^32) for x in entry j's range
    int2 lut[LUT ? 2050 : 1];
    int erow[StripeCfg::BM];    // per-row shifts of the block (int64 form)
    int wflag[8];               // per wave of the set-up: bit 0 the integer form cannot hold, bit 1 a table entry lies outside [0, 65536]
};

// byte offset inside sh.lut of the raw table as the DMA delivers it (entries 0..2047)
constexpr unsigned STRIPE_LUT_RAW = 8192;

enum { FORM_INT = 0, FORM_EXACT = 1 };

// ---- block set-up shared by the row-stationary kernels (NT threads per block, at least BM)

// column constants cst[n] of the block's chunks [cb, cb + ncols / CH): thread column j = tid + NT q.
// Issued first, so that their latency passes under the row loads rather than in the set-up.
template <int EPI, int NT>
__device__ __forceinline__ void stripe_load_cols(const GemmParams& p, int tid, int cb, int ncols, v4i* craw) {
    constexpr int CH = StripeCfg::CH, CPT = (StripeCfg::NCOLS + NT - 1) / NT;
    const __amdgpu_buffer_rsrc_t rC = make_rsrc(p.cst, unsigned(p.Nreal) * 16u);
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
        const int j = tid + NT * q;
        const int n = cb * CH + (j / CH) * CH + wrow_of_lds<EPI, CH>(j % CH);
        craw[q] = bload16(rC, j < ncols && n < p.Nreal ? unsigned(n) * 16u : OOB);
    }
}

// the row shift of row m0 + tid (0 without per-row shifts: a null buffer reads zeros)
__device__ __forceinline__ int stripe_load_erow(const GemmParams& p, int tid, int m0) {
    const __amdgpu_buffer_rsrc_t rE = make_rsrc(p.e, p.e ? unsigned(p.Mreal) * 4u : 0u);
    const bool ok = tid < StripeCfg::BM && m0 + tid < p.Mreal;
    return int(__builtin_amdgcn_raw_buffer_load_b32(rE, int(ok ? unsigned(m0 + tid) * 4u : OOB), 0, 0));
}

// DMA of the raw GELU table (entries 0..2047, 8 KB) into sh.lut + STRIPE_LUT_RAW by waves 0..3
template <bool LUT>
__device__ __forceinline__ void stripe_lut_dma(const GemmParams& p, StripeShared<LUT>& sh, int wave, int lane) {
    const v4i rL = make_rsrc_words(p.Lphi, 2049u * 4u);
    const unsigned lbase = lds_addr(sh.lut) + STRIPE_LUT_RAW;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const unsigned c = unsigned(wave * 2 + j) * 1024u;
        dma16(rL, unsigned(lane) * 16u, c, lbase + c);
    }
}

// Once the column constants, the raw table and the row shifts are in: the expanded GELU table, the
// integer form's column table and the block's epilogue form (uniform), which is the integer form
// when every row has e = 0 and every column satisfies, with 32-bit tests: 0 <= s <= 31 (GELU/GEGLU:
// 2 |m| < 2^s), |m| Kp < 2^30, |wsum| <= 128 Kp, |b| < 2^30 and 2^22 Kp |m| 2^-s < 2^30 (so that no element saturates:
// |y| <= 2^22 Kp |m| 2^-s + 1 + |b| < 2^31, as |acc| <= 32768 * 128 * Kp), and the table lies in
// [0, 65536]. Each thread tests its own columns, rows and table entries; a ballot per wave and one
// LDS word per wave carry the result through the barrier that the table expansion needs anyway.
// lut_ok: the table lies in [0, 65536] (the expanded table in LDS is then valid). Ends with a
// block-wide barrier after the tables are written.
template <int EPI, int NT>
__device__ __forceinline__ int stripe_setup(const GemmParams& p, StripeShared<EPI == EPI_GEGLU || EPI == EPI_GELU>& sh, int tid,
                                            int m0, int cb, int ncols, const v4i* craw, int erv, int L2048, bool& lut_ok) {
    constexpr bool NEEDLUT = EPI == EPI_GEGLU || EPI == EPI_GELU;
    constexpr int CH = StripeCfg::CH, BM = StripeCfg::BM, CPT = (StripeCfg::NCOLS + NT - 1) / NT;
    constexpr int LPT = NEEDLUT ? (2050 + NT - 1) / NT : 1;
    static_assert(NT / 64 <= 8, "one set-up word per wave");
    int2 lv[LPT];
    bool lbad = false;
    if constexpr (NEEDLUT) {
        const int* raw = reinterpret_cast<const int*>(reinterpret_cast<const char*>(sh.lut) + STRIPE_LUT_RAW);
#pragma unroll
        for (int q = 0; q < LPT; ++q) {
            const int i = tid + NT * q;
            int2 v = make_int2(0, 0);
            if (i == 2049) v = make_int2(65536 << 10, 0);
            else if (i >= 1 && i < 2049) {
                const int a = raw[i - 1], nx = i - 1 == 2047 ? L2048 : raw[i];
                lbad |= unsigned(a) > 65536u || unsigned(nx) > 65536u;
                // the entry's offset taken at x = 0 instead of at its first x, 1024 (i - 1025)
                v = make_int2(int((unsigned(a) << 10) - unsigned(nx - a) * unsigned(1024 * (i - 1025))), nx - a);
            }
            lv[q] = v;
        }
    }
    const unsigned mlim = (1u << 30) / unsigned(p.Kp);   // |m| < mlim  <=>  |m| Kp < 2^30
    int4 cc[CPT];
    bool bad = false;
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
        const int j = tid + NT * q;
        const int n = cb * CH + (j / CH) * CH + wrow_of_lds<EPI, CH>(j % CH);
        const bool live = j < ncols && n < p.Nreal;
        const int4 c = live ? make_int4(craw[q][0], craw[q][1], craw[q][2], craw[q][3]) : make_int4(0, 0, 0, 0);
        cc[q] = c;
        const unsigned am = uabs(c.x);
        const bool sok = unsigned(c.y) <= 31u;
        // 2^22 Kp |m| 2^-s < 2^30  <=>  Kp |m| < 2^(8 + s), with Kp |m| < 2^30
        // (for s >= 23 the shift by 31 holds too, as Kp |m| < 2^30)
        const bool umok = am < mlim && ((am * unsigned(p.Kp)) >> (sok ? min(8 + c.y, 31) : 0)) == 0u;
        // GELU/GEGLU: 2 |m| < 2^s, so that m 2^(32-s) fits in int32: the table then holds the
        // multiplier and the constant pre-shifted by 32 - s and the result is the high word of the
        // product (s = 0 passes with m = 0 only, as in the unused slots)
        const bool hiok = !NEEDLUT || (sok && (u64(am) << 1) < (u64(1) << c.y));
        bad |= !(sok && umok && hiok && uabs(c.w) <= 128u * unsigned(p.Kp) && uabs(c.z) < (1u << 30));
    }
    if (tid < BM) {
        sh.erow[tid] = erv;
        bad |= m0 + tid < p.Mreal && erv != 0;
    }
    const bool anybad = __builtin_amdgcn_ballot_w64(bad) != 0, anylbad = __builtin_amdgcn_ballot_w64(lbad) != 0;
    if ((tid & 63) == 0) sh.wflag[tid >> 6] = (anybad ? 1 : 0) | (anylbad ? 2 : 0);
    __syncthreads();   // raw table read by everyone, every wave's word in
    int f = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) f |= sh.wflag[w];
    lut_ok = !NEEDLUT || !(f & 2);
    if constexpr (NEEDLUT) {
#pragma unroll
        for (int q = 0; q < LPT; ++q) {
            const int i = tid + NT * q;
            if (i < 2050) sh.lut[i] = lv[q];
        }
    }
    const int form = __builtin_amdgcn_readfirstlane(f == 0 ? FORM_INT : FORM_EXACT);
    if (form == FORM_INT) {
#pragma unroll
        for (int q = 0; q < CPT; ++q) {
            const int j = tid + NT * q;
            if (j < ncols) {
                const int4 c = cc[q];
                // C = 128 wsum m + 2^(s-1) + b 2^s (|C| < 2^63: |wsum| <= 128 Kp, s <= 31); GELU/GEGLU:
                // the multiplier and C times 2^(32-s) (C's product wraps modulo 2^64; m = 0 when s = 0)
                const i64 C = 128LL * i64(c.w) * i64(c.x) + (c.y ? (1LL << (c.y - 1)) : 0) + i64(c.z) * (1LL << c.y);
                const int sh32 = NEEDLUT ? 32 - c.y : 0;
                const u64 Cs = u64(C) << sh32;
                const unsigned ms = sh32 < 32 ? unsigned(c.x) << sh32 : 0u;
                sh.tab[j] = make_int4(int(ms), int(unsigned(Cs)), int(unsigned(Cs >> 32)), c.y);
            }
        }
    }
    __syncthreads();
    return form;
}

// W chunk DMA of the row-stationary kernels: waves 0..3 fill a chunk (64 W rows x Kp) of the LDS
// ring, five 1 KB instructions each. W rows of a K step sit in pairs in 128-byte LDS rows (pswz).
// Instruction j of wave w fills K step ks = q / 4, LDS rows 8 rg .. 8 rg + 7 (rg = q % 4, the W rows
// 16 rg .. 16 rg + 15) of a chunk, q = 5 w + j; lane l holds the 16-byte piece that swz16 puts at
// position l % 8 of LDS row R = 8 rg + l / 8: piece pc = (l % 8) ^ (l / 8) ^ (rg % 2) (the swz16 key
// of R), which is K chunk pc % 4 of W row 16 rg + x, x = 2 (l / 8) + pc / 4. So wrow(16 rg + x) =
// wrow(x) + a constant of rg, and three per-lane values cover every instruction.
template <int EPI>
struct StripeDma {
    static constexpr int RG = StripeCfg::CH / 16;
    static_assert(RG == 4 && StripeCfg::DMA_INS * 4 == (StripeCfg::NKS / 2) * RG, "DMA mapping");
    v4i rW;
    int wb, wk0, wk1;
    unsigned wlane;
    __device__ __forceinline__ void init(const GemmParams& p, int lane) {
        rW = make_rsrc_words(p.w, p.w_bytes);
        const int pce = (lane & 7) ^ (lane >> 3);                 // piece, rg even
        const int lx = 2 * (lane >> 3) + (pce >> 2);
        wb = EPI == EPI_GEGLU ? 2 * lx : lx;                      // wrow(x)
        wk0 = 16 * (pce & 3);                                     // K offset, rg even
        wk1 = 16 * ((pce ^ 1) & 3);                               // K offset, rg odd
        wlane = unsigned(wb) * unsigned(p.ldw);
    }
    // chunk c into ring stage `stage` (the instructions of wave `wave` < 4)
    template <bool LUT>
    __device__ __forceinline__ void issue(const GemmParams& p, StripeShared<LUT>& sh, int wave, int c, int stage) const {
        constexpr int CH = StripeCfg::CH;
        const int n0 = c * CH;
        const unsigned sbase = lds_addr(sh.w[stage]);
        const bool rows_in = n0 + CH <= p.Nreal;   // the whole chunk lies inside W (uniform)
#pragma unroll
        for (int j = 0; j < StripeCfg::DMA_INS; ++j) {
            const int q = wave * StripeCfg::DMA_INS + j, ks = q / RG, rg = q - ks * RG;
            // wrow(16 rg + l4) - wrow(l4): GEGLU rows 2 lr (lr < 32) and 2 (lr - 32) + 1
            const int rgo = EPI == EPI_GEGLU ? (rg < 2 ? 32 * rg : 32 * (rg - 2) + 1) : 16 * rg;
            const int wk = ks * 64 + ((rg & 1) ? wk1 : wk0);
            unsigned off = wlane + unsigned(wk) + unsigned(rgo) * unsigned(p.ldw);
            if (ks * 64 + 64 > p.Kp && wk >= p.Kp) off = OOB;
            if (!rows_in && n0 + wb + rgo >= p.Nreal) off = OOB;
            dma16(rW, off, unsigned(n0) * unsigned(p.ldw), sbase + unsigned(ks * StripeCfg::KSTEP + rg * 1024));
        }
    }
};

// ---- integer epilogue pieces shared by the row-stationary kernels

// phi(x) for tables with 0 <= L <= 65536 (lut: the expanded table in LDS): x clamped to
// [-2^20 - 1, 2^20], entry (x >> 10) + 1025, (1024 L[i] + d (x - 1024 (i - 1025))) >> 10 as one 24-bit
// multiply-add mod 2^32: the exact value lies in [0, 2^26] and |d| <= 65536, |xc| <= 2^20 + 1 fit the
// 24-bit operands
__device__ __forceinline__ int stripe_phi(const int2* lut, int x) {
    const int xc = min(max(x, -1048577), 1048576);
    const int2 t = lut[(xc >> 10) + 1025];
    return int(unsigned(t.x) + unsigned(__mul24(t.y, xc))) >> 10;
}
// (a b + 2^15) >> 16 as a 64-bit product: the high word and the 32-bit result
__device__ __forceinline__ int stripe_mulsh16(int a, int b, unsigned& hi) {
    const i64 t = i64(a) * i64(b) + 32768;
    hi = unsigned(u64(t) >> 32);
    return int(__builtin_amdgcn_alignbit(hi, unsigned(u64(t)), 16));
}
// the same with 2^47 added to the rounding constant: returns y ^ 2^31 (y biased to unsigned order)
// and hi = (high word of a b + 2^15) + 2^15, which is <= 65535 exactly when y fits in int32
__device__ __forceinline__ unsigned stripe_mulsh16b(int a, int b, unsigned& hi) {
    const i64 t = i64(a) * i64(b) + (32768 + (1LL << 47));
    hi = unsigned(u64(t) >> 32);
    return __builtin_amdgcn_alignbit(hi, unsigned(u64(t)), 16);
}
// the integer requantisation (A m + C) >> s of an element, exact when it fits in int32. HI (the
// GELU/GEGLU tables): table entry k = {m 2^(32-s), C 2^(32-s) lo, hi, s} with 2 |m| < 2^s, whose
// product's high word is the result (bits s..s+31 of A m + C are bits 32..63 of (A m + C) 2^(32-s),
// also modulo 2^64); otherwise k = {m, C lo, hi, s} and a funnel shift by s
template <bool HI>
__device__ __forceinline__ int stripe_req(int A, const int4& k) {
    const i64 t = i64(A) * i64(k.x) + i64((u64(unsigned(k.z)) << 32) | unsigned(k.y));
    if constexpr (HI) return int(unsigned(u64(t) >> 32));
    return int(__builtin_amdgcn_alignbit(unsigned(u64(t) >> 32), unsigned(u64(t)), unsigned(k.w)));
}
// the first three words of a HI table entry (all that the high-word form reads)
struct StripeK3 { int m, lo, hi; };
__device__ __forceinline__ StripeK3 stripe_tab3(const int4* tab, int j) {
    const int3 v = *reinterpret_cast<const int3*>(tab + j);
    return {v.x, v.y, v.z};
}
__device__ __forceinline__ int stripe_req_hi(int A, const StripeK3& k) {
    const i64 t = i64(A) * i64(k.m) + i64((u64(unsigned(k.hi)) << 32) | unsigned(k.lo));
    return int(unsigned(u64(t) >> 32));
}

// RES: the PLAIN instantiation for calls with a residual (its own kernel, so that the residual
// loads do not shape the code of the others). VIEW: the int16-view instantiation (no Y; see the
// view loop below).
template <int SRC, int EPI, bool RES = false, bool VIEW = false>
__global__ void __launch_bounds__(256, 2) stripe_kernel(const GemmParams p) {
    prefetch_args();
    using S = StripeCfg;
    constexpr int CH = S::CH, NKS = S::NKS, BM = S::BM;
    constexpr bool NEEDLUT = EPI == EPI_GEGLU || EPI == EPI_GELU;
    constexpr bool GEGLU = EPI == EPI_GEGLU;
    constexpr int NOUT = GEGLU ? 1 : S::NSUB;  // output subtiles per chunk
    constexpr int STORES = NOUT * 16;          // output stores per lane per chunk
    constexpr int EB = GEGLU ? S::EB_GEGLU : 16;  // epilogue elements computed together
    static_assert(SRC == SRC_I16 || SRC == SRC_I8, "stripe sources");
    static_assert(EPI == EPI_PLAIN || EPI == EPI_GEGLU || EPI == EPI_GELU, "stripe epilogues");
    static_assert(!RES || EPI == EPI_PLAIN, "residual: PLAIN only");
    static_assert(!(RES && VIEW), "the int16 view takes no residual");

    __shared__ __attribute__((aligned(16))) StripeShared<NEEDLUT> sh;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lc = lane & 31, lh = lane >> 5;   // MFMA column / row group of this lane
    const TileIdx ti = tile_index(p);
    const int m0 = ti.mt * BM;
    const int nch = (p.Nreal + CH - 1) / CH;
    const int cb = ti.nt * p.kper, ce = min(nch, cb + p.kper);   // this block's chunks
    // a block dispatched second to its CU runs its first prio_chunks chunks at raised priority
    const bool young = !p.prio_bands && p.young0 && p.prio_chunks > 0 && int(blockIdx.x) >= p.young0;
    if (young) __builtin_amdgcn_s_setprio(1);
    PrioBands pb;
    pb.init(ce - cb, p.prio_bands);
    auto prio_step = [&](int c) __attribute__((always_inline)) {
        if (young && c - cb == p.prio_chunks) __builtin_amdgcn_s_setprio(0);
        pb.step(c - cb);
    };
    const int rbase = m0 + wave * 32;
    const int nlim = GEGLU ? (p.Nreal >> 1) : p.Nreal;
    if (cb >= ce) return;   // (the host sizes the grid so that every block has a chunk)


    // ---- the block's column constants, the row shift of row m0 + tid, the GELU table (DMA)
    const int ncols = (ce - cb) * CH;
    v4i craw[S::CPT];
    stripe_load_cols<EPI, 256>(p, tid, cb, ncols, craw);
    const int erv = stripe_load_erow(p, tid, m0);
    if constexpr (NEEDLUT) stripe_lut_dma(p, sh, wave, lane);
    const int L2048 = NEEDLUT ? p.Lphi[2048] : 0;
    StripeDma<EPI> dma;
    dma.init(p, lane);
    auto issue = [&](int c, int stage) { dma.issue(p, sh, wave, c, stage); };
    issue(cb, 0);

    // ---- the wave's activation rows (A operand: lane row lc, K bytes [32t + 16lh, +16) of substep t).
    // Issued after every DMA above and unconditionally (substeps past K read out of range, as zeros),
    // so that exactly AL row loads follow the data the block set-up needs: the set-up then waits for
    // that data alone and runs while the rows are still in flight.
    constexpr int AL = 2 * NKS;
    v4i hf[NKS], lf[NKS];
    v4i raw[NKS][SRC == SRC_I16 ? 2 : 1];
    {
        const __amdgpu_buffer_rsrc_t rA0 = make_rsrc(p.a0, p.a0_bytes);
        const __amdgpu_buffer_rsrc_t rA1 = make_rsrc(SRC == SRC_I8 ? p.a1 : p.a0, SRC == SRC_I8 ? p.a1_bytes : p.a0_bytes);
        const int r = rbase + lc;
        const bool rok = r < p.Mreal;
#pragma unroll
        for (int t = 0; t < NKS; ++t) {
            const int k0 = t * 32 + 16 * lh;
            if constexpr (SRC == SRC_I16) {
                // 16 int16 values = two 16-byte pieces; K % 8 == 0, so each piece is all in or all out
                const unsigned off = (unsigned(r) * unsigned(p.lda) + unsigned(k0)) * 2u;
                raw[t][0] = bload16(rA0, rok && k0 < p.K ? off : OOB);
                raw[t][1] = bload16(rA0, rok && k0 + 8 < p.K ? off + 16u : OOB);
            } else {
                const unsigned off = unsigned(r) * unsigned(p.lda) + unsigned(k0);
                const bool ok = rok && k0 < p.Kp;
                hf[t] = bload16(rA0, ok ? off : OOB);
                lf[t] = bload16(rA1, ok ? off : OOB);
            }
        }
    }

    // ---- block set-up: column constants of chunks [cb, ce), the expanded GELU table, flags
    vm_wait<AL>();   // the column constants, the table and chunk cb's W (older than the row loads)
    block_barrier();
    bool lut_ok;
    const int form = stripe_setup<EPI, 256>(p, sh, tid, m0, cb, ncols, craw, erv, L2048, lut_ok);

    // ---- the rows' hi/lo split (int16 rows), once they have arrived
    if constexpr (SRC == SRC_I16) {
#pragma unroll
        for (int t = 0; t < NKS; ++t) {
            const v4i x0 = raw[t][0], x1 = raw[t][1];
            const unsigned d[8] = {unsigned(x0[0]), unsigned(x0[1]), unsigned(x0[2]), unsigned(x0[3]),
                                   unsigned(x1[0]), unsigned(x1[1]), unsigned(x1[2]), unsigned(x1[3])};
            split16x16(d, hf[t], lf[t]);
        }
    }

    const __amdgpu_buffer_rsrc_t rY = make_rsrc(p.Y, p.y_bytes);
    const __amdgpu_buffer_rsrc_t rR = make_rsrc(p.R ? p.R : p.Y, p.y_bytes);
    const unsigned ldy4 = unsigned(p.ldy) * 4u;
    // this lane's rows are rbase + 4 lh + 8g + v
    const unsigned rowoff = unsigned(rbase + 4 * lh) * ldy4;
    // running max of |y| for the lane's 16 rows (max(y, -y) is |y| as an unsigned value, also for INT_MIN)
    v16i yabs;
#pragma unroll
    for (int i = 0; i < 16; ++i) yabs[i] = 0;
    // the integer form's epilogue issues a fixed number of stores per chunk, and residual loads that
    // it consumes before the chunk's last stores
    const bool lean = form == FORM_INT && (RES || !p.R);
    const bool lut_lds = NEEDLUT && lut_ok;  // the expanded table in LDS is valid (0 <= L <= 65536)

    auto phi = [&](int x) -> int { return stripe_phi(sh.lut, x); };
    auto mulsh16 = [&](int a, int b, unsigned& hi) -> int { return stripe_mulsh16(a, b, hi); };
    auto mulsh16b = [&](int a, int b, unsigned& hi) -> unsigned { return stripe_mulsh16b(a, b, hi); };
    auto req = [&](int A, const int4& k) -> int { return stripe_req<NEEDLUT>(A, k); };

    bool pipelined = false;
    if constexpr (!RES && !VIEW) {
        if (form == FORM_INT) {
            pipelined = true;
            // ---- software-pipelined chunk loop (integer form). The MFMAs of chunk c run interleaved
            // with the requantising epilogue of chunk c - 1, so that the matrix core and the VALU work
            // at the same time inside each wave. When a chunk's MFMAs finish, its two plane sums are
            // folded into one int32 per element, X = 256 Chi + Clo (exact: Kp <= 320), which frees the
            // accumulators for the next chunk; the epilogue has no branch (GEGLU products that
            // saturate are clamped per element), so the whole chunk body is one scheduling region.
            int X[2][16];
            v16i acc_h[S::NSUB], acc_l[S::NSUB];
            const v16i vzero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
            // the MFMAs of K step t of the chunk in LDS stage `stage`
            auto mfma_step = [&](const unsigned char* sW, int t) __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < S::NSUB; ++u) {
                    const v4i wf = *reinterpret_cast<const v4i*>(sW + (t >> 1) * S::KSTEP + pswz(32 * u + lc, 2 * (t & 1) + lh));
                    acc_h[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(hf[t], wf, t ? acc_h[u] : vzero, 0, 0, 0);
                    acc_l[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(lf[t], wf, t ? acc_l[u] : vzero, 0, 0, 0);
                }
            };
            auto mfma_chunk = [&](int stage) __attribute__((always_inline)) {
#pragma unroll
                for (int t = 0; t < NKS; ++t) mfma_step(sh.w[stage], t);
            };
            auto fold = [&]() __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < S::NSUB; ++u)
#pragma unroll
                    for (int i = 0; i < 16; ++i) X[u][i] = (acc_h[u][i] << 8) + acc_l[u][i];
            };
            // per-chunk constants of the epilogue of the chunk held in X: table entries of the lane's
            // column(s) and the byte offset of its first output (OOB past the output's columns)
            struct EpiC { int4 ka[NOUT], kg; unsigned vbase[NOUT]; };
            auto epi_consts = [&](int tb, int ocol0) __attribute__((always_inline)) {
                EpiC k;
#pragma unroll
                for (int u = 0; u < NOUT; ++u) {
                    const int ncol = ocol0 + 32 * u + lc;
                    k.vbase[u] = ncol < nlim ? rowoff + unsigned(ncol) * 4u : OOB;
                    k.ka[u] = sh.tab[tb + 32 * u + lc];
                }
                k.kg = GEGLU ? sh.tab[tb + 32 + lc] : k.ka[0];
                return k;
            };
            // output o = 16 u + i of the chunk held in X: requantise, store, row maximum
            auto epi_one = [&](const EpiC& k, int o, auto rmax, auto full) __attribute__((always_inline)) {
                constexpr bool RMAX = decltype(rmax)::value, FULL = decltype(full)::value;
                const int u = o >> 4, i = o & 15;
                int y;
                if constexpr (GEGLU) {
                    const int yg = req(X[1][i], k.kg);
                    unsigned h0;
                    const int ge = mulsh16(yg, phi(yg), h0);
                    // (ya ge + 2^15) >> 16 with 2^47 added: hb is the high word + 2^15, at most 65535
                    // exactly when y fits in int32; otherwise y saturates to the product's sign
                    unsigned hb;
                    const unsigned yb = mulsh16b(req(X[0][i], k.ka[0]), ge, hb);
                    asm("" : "+v"(hb));   // keep the tests on the 32-bit high word
                    const int sat = (int(hb) >> 31) ^ 0x7fffffff;
                    y = hb > 65535u ? sat : int(yb ^ 0x80000000u);
                } else if constexpr (EPI == EPI_GELU) {
                    const int ya = req(X[u][i], k.ka[u]);
                    unsigned h0;
                    y = mulsh16(ya, phi(ya), h0);
                } else {
                    y = req(X[u][i], k.ka[u]);
                }
                const unsigned soff = unsigned(8 * (i >> 2) + (i & 3)) * ldy4;
                __builtin_amdgcn_raw_buffer_store_b32(y, rY, int(FULL ? k.vbase[u] : k.vbase[u] + soff), FULL ? int(soff) : 0, 0);
                if constexpr (RMAX) yabs[i] = int(max(unsigned(yabs[i]), unsigned(max(y, int(0u - unsigned(y))))));
            };
            auto epilogue = [&](int tb, int ocol0, auto rmax, auto full) __attribute__((always_inline)) {
                const EpiC k = epi_consts(tb, ocol0);
#pragma unroll
                for (int o = 0; o < NOUT * 16; ++o) epi_one(k, o, rmax, full);
            };
            // One chunk body in two halves, one per 32-column MFMA subtile u: K step t's two MFMAs of
            // subtile u, then the previous chunk's outputs assigned to that step, each step ordered
            // as one MFMA, VPM VALU instructions and one LDS read, twice. Half u takes the previous
            // chunk's outputs that are done with X[.][i] for the elements whose registers the fold
            // of subtile u then reuses (GEGLU: outputs 8u..8u+7, which read X[0][i] and X[1][i];
            // otherwise: the 16 outputs of subtile u), so only one subtile's accumulators are live.
            // W fragments are read PFB steps ahead of their MFMAs.
            constexpr int NO = NOUT * 16, NOH = NO / 2;
            constexpr int VPM = GEGLU ? 8 : (EPI == EPI_GELU ? 7 : 4);
            constexpr int PFB = 2;
            auto wfrag = [&](const unsigned char* sW, int t, int u) __attribute__((always_inline)) {
                return *reinterpret_cast<const v4i*>(sW + (t >> 1) * S::KSTEP + pswz(32 * u + lc, 2 * (t & 1) + lh));
            };
            auto body = [&](int stage, int tbp, int ocp, auto rmax, auto full) __attribute__((always_inline)) {
                const unsigned char* sW = sh.w[stage];
                const EpiC k = epi_consts(tbp, ocp);
                int Xn[S::NSUB][16];
#pragma unroll
                for (int u = 0; u < S::NSUB; ++u) {
                    v4i wq[PFB];
#pragma unroll
                    for (int t = 0; t < PFB; ++t) wq[t] = wfrag(sW, t, u);
                    v16i ah, al;
#pragma unroll
                    for (int t = 0; t < NKS; ++t) {
                        const v4i wf = wq[t % PFB];
                        if (t + PFB < NKS) wq[t % PFB] = wfrag(sW, t + PFB, u);
                        ah = __builtin_amdgcn_mfma_i32_32x32x32_i8(hf[t], wf, t ? ah : vzero, 0, 0, 0);
                        al = __builtin_amdgcn_mfma_i32_32x32x32_i8(lf[t], wf, t ? al : vzero, 0, 0, 0);
#pragma unroll
                        for (int o = u * NOH + t * NOH / NKS; o < u * NOH + (t + 1) * NOH / NKS; ++o) {
                            // GEGLU output o reads X[0][o], X[1][o]; the others X[o >> 4][o & 15]
                            epi_one(k, o, rmax, full);
                        }
#pragma unroll
                        for (int q = 0; q < 2; ++q) {
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                            __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
                            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        }
                    }
#pragma unroll
                    for (int i = 0; i < 16; ++i) Xn[u][i] = (ah[i] << 8) + al[i];
                }
#pragma unroll
                for (int u = 0; u < S::NSUB; ++u)
#pragma unroll
                    for (int i = 0; i < 16; ++i) X[u][i] = Xn[u][i];
            };
            auto run = [&](auto rmax, auto full) __attribute__((always_inline)) {
                // the first chunk: MFMAs alone
                vm_wait<0>();
                block_barrier();
                if (cb + 1 < ce) issue(cb + 1, 1);
                mfma_chunk(0);
                fold();
                for (int c = cb + 1; c < ce; ++c) {
                    prio_step(c);
                    const int stage = (c - cb) & 1;
                    // chunk c's DMA is done once at most the previous chunk body's stores are outstanding
                    if (c == cb + 1) vm_wait<0>();
                    else vm_wait<STORES>();
                    block_barrier();
                    if (c + 1 < ce) issue(c + 1, stage ^ 1);
                    body(stage, (c - 1 - cb) * CH, GEGLU ? (c - 1) * (CH / 2) : (c - 1) * CH, rmax, full);
                }
                epilogue((ce - 1 - cb) * CH, GEGLU ? (ce - 1) * (CH / 2) : (ce - 1) * CH, rmax, full);
            };
            const bool full = m0 + BM <= p.Mreal;
            if (p.rowmax) {
                if (full) run(std::true_type{}, std::true_type{});
                else run(std::true_type{}, std::false_type{});
            } else {
                if (full) run(std::false_type{}, std::true_type{});
                else run(std::false_type{}, std::false_type{});
            }
        }
    }
    if constexpr (VIEW) {
        // ---- int16 view (quant_row_out semantics, src/kernels.cu:317-331, on this GEMM's outputs).
        // The MFMAs take W as the A operand and the activations as the B operand, so that the
        // accumulators are transposed: lane l holds activation row rbase + lc and, of each 32-row W
        // subtile u, the W rows 8g + 4 lh + v (element i = 4g + v). A chunk's outputs of one row then
        // sit in two lanes (lh = 0, 1), and its row maximum is the lane's own maximum and one
        // exchange. The row exponent is not known until every chunk of the row is done, so each chunk
        // is quantised at the running exponent e_c = row_exp(max |y| over the row's chunks so far in
        // this block), which the final e can only exceed. Per element the bit d = (y >> e_c) - q (0
        // or -1; q is the clamped rounding quotient) is kept, so that y >> e_c = q + d can be
        // recovered; since floor shifts compose, y >> (e - 1) = (y >> e_c) >> (e - 1 - e_c) for any
        // e > e_c, and the final value (that + 1) >> 1 (clamped) follows exactly. Per (row, 32-column
        // group) the chunk's e_c and the 32 bits go to the workspace, the row maximum to vmax; the
        // fix-up pass (producers.hip) rewrites the groups whose e_c fell short of the row's e.
        constexpr int NU = GEGLU ? 1 : S::NSUB;       // 32-output groups per chunk
        constexpr int NOV = 16 * NU;                  // outputs of a lane per chunk
        constexpr int VST = NU * 6;                   // stores per lane per chunk: 4 plane pieces, a mask, an exponent
        const __amdgpu_buffer_rsrc_t rH = make_rsrc(p.vhi, p.v_bytes), rLo = make_rsrc(p.vlo, p.v_bytes);
        const unsigned gbytes = unsigned(p.Mreal) * unsigned(p.vgroups);
        const __amdgpu_buffer_rsrc_t rM = make_rsrc(p.vmask, gbytes * 4u), rE = make_rsrc(p.vexp, gbytes);
        const int r = rbase + lc;
        const bool rok = r < p.Mreal;
        const int erl = sh.erow[wave * 32 + lc];     // the exact form's shift of the lane's row
        unsigned mrun = 0;                           // running max |y| of the lane's row
        const bool lean_v = form == FORM_INT;
        for (int c = cb; c < ce; ++c) {
            prio_step(c);
            const int stage = (c - cb) & 1;
            // chunk c's DMA is done once at most the previous chunk's stores are outstanding (every
            // lane issues exactly VST stores per chunk: rows, columns and lanes without output store
            // to an out-of-range offset); the exact form also loads, so it waits for everything
            if (c > cb && lean_v) vm_wait<VST>();
            else vm_wait<0>();
            block_barrier();
            if (c + 1 < ce) issue(c + 1, stage ^ 1);

            v16i acc_h[S::NSUB], acc_l[S::NSUB];
#pragma unroll
            for (int u = 0; u < S::NSUB; ++u)
#pragma unroll
                for (int i = 0; i < 16; ++i) { acc_h[u][i] = 0; acc_l[u][i] = 0; }
            const unsigned char* sW = sh.w[stage];
            auto wfrag = [&](int t, int u) -> v4i {
                return *reinterpret_cast<const v4i*>(sW + (t >> 1) * S::KSTEP + pswz(32 * u + lc, 2 * (t & 1) + lh));
            };
            constexpr int PF = 2;
            v4i wq[PF][S::NSUB];
#pragma unroll
            for (int t = 0; t < PF; ++t)
#pragma unroll
                for (int u = 0; u < S::NSUB; ++u) wq[t][u] = wfrag(t, u);
#pragma unroll
            for (int t = 0; t < NKS; ++t) {
                v4i wf[S::NSUB];
#pragma unroll
                for (int u = 0; u < S::NSUB; ++u) {
                    wf[u] = wq[t % PF][u];
                    if (t + PF < NKS) wq[t % PF][u] = wfrag(t + PF, u);
                }
#pragma unroll
                for (int u = 0; u < S::NSUB; ++u) {
                    acc_h[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[u], hf[t], acc_h[u], 0, 0, 0);
                    acc_l[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[u], lf[t], acc_l[u], 0, 0, 0);
                }
                if (t + PF < NKS) __builtin_amdgcn_sched_group_barrier(0x100, S::NSUB, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 2 * S::NSUB, 0);
            }

            // ---- the lane's outputs of chunk c: o = 16 u + i is W row 32 u + j of the chunk, j = 8 (i >> 2) + 4 lh + (i & 3)
            // (GEGLU: a row j, g row 32 + j, output j). Columns past the output come out 0: their table
            // entries and W rows are zero (integer form), and the int64 form is masked.
            const int tb = (c - cb) * CH;
            const int oc0 = GEGLU ? c * (CH / 2) : c * CH;   // first output column of the chunk
            int y[NOV];
            if (form == FORM_INT) {
#pragma unroll
                for (int o = 0; o < NOV; ++o) {
                    const int u = o >> 4, i = o & 15;
                    const int j = 32 * u + 8 * (i >> 2) + 4 * lh + (i & 3);
                    const int4 ka = sh.tab[tb + j];
                    if constexpr (GEGLU) {
                        const int4 kg = sh.tab[tb + 32 + j];
                        const int yg = req((acc_h[1][i] << 8) + acc_l[1][i], kg);
                        unsigned h0, hb;
                        const int ge = mulsh16(yg, phi(yg), h0);
                        const unsigned yb = mulsh16b(req((acc_h[0][i] << 8) + acc_l[0][i], ka), ge, hb);
                        asm("" : "+v"(hb));
                        const int sat = (int(hb) >> 31) ^ 0x7fffffff;
                        y[o] = hb > 65535u ? sat : int(yb ^ 0x80000000u);
                    } else if constexpr (EPI == EPI_GELU) {
                        const int ya = req((acc_h[u][i] << 8) + acc_l[u][i], ka);
                        unsigned h0;
                        y[o] = mulsh16(ya, phi(ya), h0);
                    } else {
                        y[o] = req((acc_h[u][i] << 8) + acc_l[u][i], ka);
                    }
                }
            } else {
#pragma unroll 1
                for (int o = 0; o < NOV; ++o) {
                    const int u = o >> 4, i = o & 15;
                    const int j = 32 * u + 8 * (i >> 2) + 4 * lh + (i & 3);
                    const int col = oc0 + j;
                    const int cc = col < nlim ? col : 0;
                    const int4 ca = p.cst[GEGLU ? 2 * cc : cc];
                    const int ya = epi1_exact(acc_h[u][i], acc_l[u][i], ca.x, ca.y, ca.z, ca.w, erl);
                    int v;
                    if constexpr (GEGLU) {
                        const int4 cg = p.cst[2 * cc + 1];
                        const int yg = epi1_exact(acc_h[1][i], acc_l[1][i], cg.x, cg.y, cg.z, cg.w, erl);
                        const i64 pg = lut_lds ? phi(yg) : lut16i(yg, p.Lphi);
                        const i64 ge = sat32(rshr(i64(yg) * pg, 16));
                        v = int(sat32(rshr(i64(ya) * ge, 16)));
                    } else if constexpr (EPI == EPI_GELU) {
                        const i64 pa = lut_lds ? phi(ya) : lut16i(ya, p.Lphi);
                        v = int(sat32(rshr(i64(ya) * pa, 16)));
                    } else {
                        v = ya;
                    }
                    y[o] = col < nlim ? v : 0;
                }
            }
            // running row maximum of |y| (from the signed maximum and minimum) and exponent
            int mx = 0, mn = 0;
#pragma unroll
            for (int o = 0; o < NOV; ++o) { mx = max(mx, y[o]); mn = min(mn, y[o]); }
            unsigned m = max(mrun, max(unsigned(mx), 0u - unsigned(mn)));
            m = max(m, unsigned(__shfl_xor(int(m), 32)));
            mrun = m;
            const int ec = rowexp_u32(m);
            // quantise at ec: t = y >> (ec - 1) (y << 1 for ec = 0), floor y >> ec = t >> 1, rounded
            // q = clamp((t + 1) >> 1), correction d = (y >> ec) - q in {0, -1}
            const int sl = ec == 0 ? 1 : 0, sr = ec == 0 ? 0 : ec - 1;
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                unsigned bits = 0;   // bit 8g + v (this lane's half; shifted to 8g + 4 lh + v below)
                unsigned hw[4], lw[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    int q[4];
#pragma unroll
                    for (int vv = 0; vv < 4; ++vv) {
                        const int t = (y[16 * u + 4 * g + vv] << sl) >> sr;
                        q[vv] = min(max((t + 1) >> 1, -32767), 32767);
                        bits |= unsigned((t >> 1) - q[vv]) & (1u << (8 * g + vv));
                    }
                    // bytes 1 (hi) and 0 (lo, biased by 128) of the four values (columns 8g + 4 lh + v)
                    hw[g] = __builtin_amdgcn_perm(unsigned(q[1]), unsigned(q[0]), 0x0c0c0501u) |
                            __builtin_amdgcn_perm(unsigned(q[3]), unsigned(q[2]), 0x05010c0cu);
                    lw[g] = (__builtin_amdgcn_perm(unsigned(q[1]), unsigned(q[0]), 0x0c0c0400u) |
                             __builtin_amdgcn_perm(unsigned(q[3]), unsigned(q[2]), 0x04000c0cu)) ^ 0x80808080u;
                }
                // the two lanes of a row swap halves: lane lh = 0 gathers the 32 hi bytes of the group,
                // lane lh = 1 the 32 lo bytes, so that each plane's row segment goes out as whole 16-byte
                // pieces (full 32-byte sectors per row and plane, no partial-sector writes)
                unsigned wv[8];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const unsigned recv = unsigned(__shfl_xor(int(lh ? hw[g] : lw[g]), 32));
                    wv[2 * g] = lh ? recv : hw[g];
                    wv[2 * g + 1] = lh ? lw[g] : recv;
                }
                const v4i s0 = {int(wv[0]), int(wv[1]), int(wv[2]), int(wv[3])}, s1 = {int(wv[4]), int(wv[5]), int(wv[6]), int(wv[7])};
                const int col = oc0 + 32 * u;
                const unsigned rb = unsigned(r) * unsigned(p.vld) + unsigned(col);
                // columns [nlim, 16-column boundary) get y = 0, i.e. the pad value (0, -128)
                const unsigned o0 = rok && col < nlim ? rb : OOB, o1 = rok && col + 16 < nlim ? rb + 16u : OOB;
                __builtin_amdgcn_raw_buffer_store_b128(s0, rH, int(lh ? OOB : o0), 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(s1, rH, int(lh ? OOB : o1), 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(s0, rLo, int(lh ? o0 : OOB), 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(s1, rLo, int(lh ? o1 : OOB), 0, 0);
                bits <<= 4 * lh;
                bits |= unsigned(__shfl_xor(int(bits), 32));
                // group-major: the rows of a group are consecutive, so these stores are contiguous
                const int grp = (oc0 >> 5) + u;
                const bool gok = rok && lh == 0 && grp < p.vgroups;
                const unsigned gi = unsigned(grp) * unsigned(p.Mreal) + unsigned(r);
                __builtin_amdgcn_raw_buffer_store_b32(int(bits), rM, int(gok ? gi * 4u : OOB), 0, 0);
                __builtin_amdgcn_raw_buffer_store_b8((unsigned char)ec, rE, int(gok ? gi : OOB), 0, 0);
            }
        }
        if (rok && lh == 0 && mrun) atomicMax(p.vmax + r, mrun);
    } else {
    if (!pipelined) {
        for (int c = cb; c < ce; ++c) {
            prio_step(c);
            const int stage = (c - cb) & 1;
            // chunk c's DMA is done once at most the previous chunk's stores are outstanding
            if (c > cb && lean) vm_wait<STORES>();
            else vm_wait<0>();
            block_barrier();
            if (c + 1 < ce) issue(c + 1, stage ^ 1);

            v16i acc_h[S::NSUB], acc_l[S::NSUB];
    #pragma unroll
            for (int u = 0; u < S::NSUB; ++u)
    #pragma unroll
                for (int i = 0; i < 16; ++i) { acc_h[u][i] = 0; acc_l[u][i] = 0; }
            const unsigned char* sW = sh.w[stage];
            // all ten K steps: past Kp both operands hold zeros (A registers cleared, W bytes out of range).
            // The W fragments of step t + 2 are read from LDS before the MFMAs of step t, so that their
            // latency hides behind four MFMAs of this wave.
            auto wfrag = [&](int t, int u) -> v4i {
                return *reinterpret_cast<const v4i*>(sW + (t >> 1) * S::KSTEP + pswz(32 * u + lc, 2 * (t & 1) + lh));
            };
            constexpr int PF = 2;
            v4i wq[PF][S::NSUB];
    #pragma unroll
            for (int t = 0; t < PF; ++t)
    #pragma unroll
                for (int u = 0; u < S::NSUB; ++u) wq[t][u] = wfrag(t, u);
            __builtin_amdgcn_sched_group_barrier(0x100, PF * S::NSUB, 0);
    #pragma unroll
            for (int t = 0; t < NKS; ++t) {
                v4i wf[S::NSUB];
    #pragma unroll
                for (int u = 0; u < S::NSUB; ++u) {
                    wf[u] = wq[t % PF][u];
                    if (t + PF < NKS) wq[t % PF][u] = wfrag(t + PF, u);
                }
    #pragma unroll
                for (int u = 0; u < S::NSUB; ++u) {
                    acc_h[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(hf[t], wf[u], acc_h[u], 0, 0, 0);
                    acc_l[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(lf[t], wf[u], acc_l[u], 0, 0, 0);
                }
                // keep that order in the schedule: the reads of step t + 2, then the MFMAs of step t
                if (t + PF < NKS) __builtin_amdgcn_sched_group_barrier(0x100, S::NSUB, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 2 * S::NSUB, 0);
            }

            // ---- epilogue of chunk c: output subtile u is table rows tb + 32u + lc (GEGLU: a columns,
            // g columns 32 further), output column ocol0 + 32u + lc
            const int tb = (c - cb) * CH;
            const int ocol0 = GEGLU ? c * (CH / 2) : c * CH;
    #pragma unroll
            for (int u = 0; u < NOUT; ++u) {
                const int ncol = ocol0 + 32 * u + lc;
                const bool cok = ncol < nlim;
                // byte offset of the lane's row rbase + 4 lh and column; + slot rows below. Rows at or past
                // Mreal land at or past the end of the Y buffer and columns past the output at OOB, so the
                // hardware drops those stores (and residual loads read zeros there)
                const unsigned vbase = cok ? rowoff + unsigned(ncol) * 4u : OOB;
                if (form == FORM_INT) {
                    const int4 ka = sh.tab[tb + 32 * u + lc];
                    const int4 kg = sh.tab[tb + (GEGLU ? 32 : 32 * u) + lc];
                    // GEGLU of element i, biased (y ^ 2^31); hi = the high word of a ge + 2^15, plus 2^15
                    auto geglu = [&](int i, unsigned& hi) -> unsigned {
                        const int ya = req((acc_h[0][i] << 8) + acc_l[0][i], ka);
                        const int yg = req((acc_h[1][i] << 8) + acc_l[1][i], kg);
                        unsigned h0;
                        const int ge = mulsh16(yg, phi(yg), h0);
                        return mulsh16b(ya, ge, hi);
                    };
                    // FULL: every row of the block is below Mreal. Then a store's row offset (uniform)
                    // goes in the instruction's scalar offset and its vector offset is the lane's base:
                    // in range exactly when the column is (OOB otherwise), whether or not the hardware
                    // range check counts the scalar offset. Otherwise each element's full offset is in
                    // the vector offset, so that rows at or past Mreal fall outside the buffer.
                    auto run = [&](auto hasr, auto rmax, auto full) {
                        constexpr bool HASR = decltype(hasr)::value, RMAX = decltype(rmax)::value;
                        constexpr bool FULL = decltype(full)::value;
                        // EB elements at a time: their values first, with no branch between them, so
                        // that their dependency chains (64-bit products, table lookups) interleave; then
                        // their stores
    #pragma unroll
                        for (int i0 = 0; i0 < 16; i0 += EB) {
                            int yv[EB];        // GEGLU: biased, y ^ 2^31
                            int rv[HASR ? EB : 1];
                            if constexpr (HASR) {
                                // the batch's residuals first, so that their latency hides behind its arithmetic
    #pragma unroll
                                for (int j = 0; j < EB; ++j) {
                                    const int i = i0 + j;
                                    const unsigned soff = unsigned(8 * (i >> 2) + (i & 3)) * ldy4;
                                    rv[j] = int(__builtin_amdgcn_raw_buffer_load_b32(rR, int(FULL ? vbase : vbase + soff), FULL ? int(soff) : 0, 0));
                                }
                            }
                            unsigned hv[GEGLU ? EB : 1];
                            unsigned ov = 0;   // OR of the biased high words: > 65535 iff one overflows
    #pragma unroll
                            for (int j = 0; j < EB; ++j) {
                                const int i = i0 + j;
                                if constexpr (GEGLU) {
                                    yv[j] = int(geglu(i, hv[j]));
                                    // opaque to the compiler, so that the tests below stay on the 32-bit
                                    // high word (not on a 64-bit product kept alive for them)
                                    asm volatile("" : "+v"(hv[j]));
                                    ov |= hv[j];
                                } else if constexpr (EPI == EPI_GELU) {
                                    const int ya = req((acc_h[u][i] << 8) + acc_l[u][i], ka);
                                    unsigned h0;
                                    yv[j] = mulsh16(ya, phi(ya), h0);
                                } else {
                                    yv[j] = req((acc_h[u][i] << 8) + acc_l[u][i], ka);
                                }
                            }
                            if constexpr (GEGLU) {
                                // |a ge| >= 2^47 for an element of the wave: that result saturates. Rarely
                                // taken; the overflowing elements are replaced.
                                if (__builtin_amdgcn_ballot_w64(ov > 65535u)) {
                                    asm volatile("; saturating GEGLU product");
                                    // the sign of the product is the sign bit of the biased high word;
                                    // the biased saturated value is ~0 (INT_MAX) or 0 (INT_MIN)
    #pragma unroll
                                    for (int j = 0; j < EB; ++j)
                                        if (hv[j] > 65535u) yv[j] = ~(int(hv[j]) >> 31);
                                }
                            }
    #pragma unroll
                            for (int j = 0; j < EB; ++j) {
                                const int i = i0 + j;
                                const unsigned soff = unsigned(8 * (i >> 2) + (i & 3)) * ldy4;
                                const unsigned voff = FULL ? vbase : vbase + soff;
                                const int sgo = FULL ? int(soff) : 0;
                                int y = GEGLU ? int(unsigned(yv[j]) ^ 0x80000000u) : yv[j];
                                if constexpr (HASR) y = add_sat(y, rv[j]);
                                __builtin_amdgcn_raw_buffer_store_b32(y, rY, int(voff), sgo, 0);
                                // Columns past the output have m = s = C = 0 in the table and zero W rows,
                                // so their y is 0.
                                if constexpr (RMAX) {
                                    unsigned ay;
                                    if constexpr (GEGLU) {
                                        // |y| = |(y ^ 2^31) - 2^31| as an unsigned difference, also for INT_MIN
                                        asm("v_sad_u32 %0, %1, %2, 0" : "=v"(ay) : "v"(yv[j]), "s"(0x80000000u));
                                    } else {
                                        // max(y, -y) is |y| as an unsigned value, also for INT_MIN
                                        ay = unsigned(max(y, int(0u - unsigned(y))));
                                    }
                                    yabs[i] = int(max(unsigned(yabs[i]), ay));
                                }
                            }
                            __builtin_amdgcn_sched_barrier(0);   // batches do not mix (register pressure)
                        }
                    };
                    auto run_rows = [&](auto hasr, auto rmax) {
                        if (m0 + BM <= p.Mreal) run(hasr, rmax, std::true_type{});
                        else run(hasr, rmax, std::false_type{});
                    };
                    if constexpr (RES) {
                        if (p.rowmax) run_rows(std::true_type{}, std::true_type{});
                        else run_rows(std::true_type{}, std::false_type{});
                    } else {
                        if (p.rowmax) run_rows(std::false_type{}, std::true_type{});
                        else run_rows(std::false_type{}, std::false_type{});
                    }
                } else {
                    // the reference's int64 formula, one element per iteration (its row maximum goes
                    // straight to memory)
                    const int col = cok ? ncol : 0;
                    const int4 ca = p.cst[GEGLU ? 2 * col : col];
                    const int4 cg = GEGLU ? p.cst[2 * col + 1] : ca;
    #pragma unroll 1
                    for (int i = 0; i < 16; ++i) {
                        const int slot = 8 * (i >> 2) + (i & 3);
                        const unsigned voff = vbase + unsigned(slot) * ldy4;
                        const int er = sh.erow[wave * 32 + 4 * lh + slot];
                        const int ya = epi1_exact(acc_h[u][i], acc_l[u][i], ca.x, ca.y, ca.z, ca.w, er);
                        int y;
                        if constexpr (GEGLU) {
                            const int yg = epi1_exact(acc_h[1][i], acc_l[1][i], cg.x, cg.y, cg.z, cg.w, er);
                            const i64 pg = lut_lds ? phi(yg) : lut16i(yg, p.Lphi);
                            const i64 ge = sat32(rshr(i64(yg) * pg, 16));
                            y = int(sat32(rshr(i64(ya) * ge, 16)));
                        } else if constexpr (EPI == EPI_GELU) {
                            const i64 pa = lut_lds ? phi(ya) : lut16i(ya, p.Lphi);
                            y = int(sat32(rshr(i64(ya) * pa, 16)));
                        } else {
                            y = ya;
                        }
                        if (EPI == EPI_PLAIN && p.R) y = add_sat(y, int(__builtin_amdgcn_raw_buffer_load_b32(rR, int(voff), 0, 0)));
                        __builtin_amdgcn_raw_buffer_store_b32(y, rY, int(voff), 0, 0);
                        const int r = rbase + 4 * lh + slot;
                        if (p.rowmax && cok && r < p.Mreal && y) atomicMax(p.rowmax + r, uabs(y));
                    }
                }
            }
        }
    }

    }   // !VIEW

    if (!VIEW && p.rowmax) {
        // lanes with the same lh hold the same 16 rows: reduce over the 32 columns, one atomic per row
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            uint32_t m = uint32_t(yabs[i]);
#pragma unroll
            for (int o = 1; o < 32; o <<= 1) m = max(m, uint32_t(__shfl_xor(int(m), o)));
            const int r = rbase + 4 * lh + 8 * (i >> 2) + (i & 3);
            if (lc == 0 && r < p.Mreal && m) atomicMax(p.rowmax + r, m);
        }
    }
}

template <int SRC>
hipError_t launch_stripe_t(int epi, const GemmParams& p, hipStream_t st) {
    const dim3 grid(unsigned(p.mtiles * p.ntiles));
    switch (epi) {
    case EPI_PLAIN:
        if (p.R) hipLaunchKernelGGL((stripe_kernel<SRC, EPI_PLAIN, true>), grid, dim3(256), 0, st, p);
        else hipLaunchKernelGGL((stripe_kernel<SRC, EPI_PLAIN>), grid, dim3(256), 0, st, p);
        break;
    case EPI_GEGLU: hipLaunchKernelGGL((stripe_kernel<SRC, EPI_GEGLU>), grid, dim3(256), 0, st, p); break;
    case EPI_GELU: hipLaunchKernelGGL((stripe_kernel<SRC, EPI_GELU>), grid, dim3(256), 0, st, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int SRC>
hipError_t launch_stripe_view_t(int epi, const GemmParams& p, hipStream_t st) {
    const dim3 grid(unsigned(p.mtiles * p.ntiles));
    switch (epi) {
    case EPI_PLAIN: hipLaunchKernelGGL((stripe_kernel<SRC, EPI_PLAIN, false, true>), grid, dim3(256), 0, st, p); break;
    case EPI_GEGLU: hipLaunchKernelGGL((stripe_kernel<SRC, EPI_GEGLU, false, true>), grid, dim3(256), 0, st, p); break;
    case EPI_GELU: hipLaunchKernelGGL((stripe_kernel<SRC, EPI_GELU, false, true>), grid, dim3(256), 0, st, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_stripe(int src, int epi, const GemmParams& p, hipStream_t st);
hipError_t launch_stripe_view(int src, int epi, const GemmParams& p, hipStream_t st);

}  // namespace vk

// Row-stationary hi/lo GEMM with sixteen rows per wave ("stripe16"), for shallow K (Kp <= 320): int16
// rows (SRC_I16) or int8 planes (SRC_I8), epilogues PLAIN (no residual), GEGLU and GELU, with or
// without the row maximum; the same results as stripe_kernel, bit for bit.
//
// Geometry. A block of eight waves owns 128 activation rows, sixteen per wave, and a range of W rows
// (output columns) streamed through LDS in 64-row chunks, exactly as stripe_kernel does (same DMA,
// LDS ring, column table and set-up). The difference is the MFMA: v_mfma_i32_16x16x64_i8 (the same
// rate per cycle as the 32x32x32 form on gfx950) with the activations as the A operand, so that a
// wave's sixteen rows take 40 registers of hi/lo fragments instead of 80, its accumulators 4 per
// 16-column subtile, and its row maxima 4. That fits a wave in 128 registers: two blocks per CU
// give four waves per SIMD (stripe_kernel: two), and the requantising epilogue, whose cost is each
// output's dependency chain (two 64-bit products, the table lookup, the saturation test), has twice
// as many independent waves to hide behind.
//
// Lane layout of a 16x16 subtile: lane l holds output column l % 16 for rows 4 (l / 16) + v
// (v = 0..3). A chunk has four subtiles: GEGLU pairs subtile u (a columns 16 u .. 16 u + 15) with
// subtile u + 2 (the g columns), two output subtiles; PLAIN and GELU have four.
//
// Chunk loop of the integer form. A block's waves pass one barrier per chunk (the W ring has two
// stages), so they move in step; the two waves of a block on one SIMD (waves w and w + 4) take
// opposite phases instead of the in-wave software pipeline of stripe_kernel, which would need two
// chunks of sums in registers: waves 0..3 run a chunk's MFMAs (four subtiles x five K steps x two
// planes) and then its requantising epilogue, waves 4..7 the previous chunk's epilogue and then the
// chunk's MFMAs, the plane sums folded into one int32 per element (256 Chi + Clo, exact for
// Kp <= 320) across the barrier. The int64 form (per-row shifts, columns whose constants fail the
// integer form's bounds, tables outside [0, 65536]) runs a plain loop, a chunk's MFMAs then its
// outputs element by element.
#pragma once
#include "stripe_kernel.h"

namespace vk {

struct Stripe16Cfg {
    static constexpr int NW = 8;                                   // waves per block
    static constexpr int NT = 64 * NW;                             // threads per block
    static constexpr int WR = StripeCfg::BM / NW;                  // rows per wave
    static constexpr int NKS = 5;                                  // 64-deep K steps (Kp <= 320)
    static constexpr int NSUB = StripeCfg::CH / 16;                // 16-column subtiles per chunk
    static constexpr int CPT = (StripeCfg::NCOLS + NT - 1) / NT;   // table columns per thread
    static_assert(WR == 16 && NKS * 64 == 32 * StripeCfg::NKS, "stripe16 geometry");
};

template <int SRC, int EPI>
__global__ void __launch_bounds__(512, 4) stripe16_kernel(const GemmParams p) {
    using S = StripeCfg;
    using G = Stripe16Cfg;
    constexpr int CH = S::CH, BM = S::BM, NKS = G::NKS, NT = G::NT, NSUB = G::NSUB;
    constexpr bool NEEDLUT = EPI == EPI_GEGLU || EPI == EPI_GELU;
    constexpr bool GEGLU = EPI == EPI_GEGLU;
    constexpr int NOUT = GEGLU ? NSUB / 2 : NSUB;   // output subtiles per chunk
    constexpr int NO = NOUT * 4;                    // outputs per lane per chunk
    constexpr int STORES = NO;                      // output stores per lane per chunk
    static_assert(SRC == SRC_I16 || SRC == SRC_I8, "stripe sources");
    static_assert(EPI == EPI_PLAIN || EPI == EPI_GEGLU || EPI == EPI_GELU, "stripe epilogues");

    __shared__ __attribute__((aligned(16))) StripeShared<NEEDLUT> sh;

    prefetch_args();
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 15, fg = lane >> 4;   // MFMA column / row group of this lane
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
    const int rbase = m0 + wave * G::WR;
    const int nlim = GEGLU ? (p.Nreal >> 1) : p.Nreal;
    if (cb >= ce) return;   // (the host sizes the grid so that every block has a chunk)
    const bool dma_wave = wave < 4;   // waves 0..3 issue the W and table DMA

    // ---- the block's column constants, the row shift of row m0 + tid, the GELU table (DMA), chunk cb
    const int ncols = (ce - cb) * CH;
    v4i craw[G::CPT];
    stripe_load_cols<EPI, NT>(p, tid, cb, ncols, craw);
    const int erv = stripe_load_erow(p, tid, m0);
    if constexpr (NEEDLUT) {
        if (dma_wave) stripe_lut_dma(p, sh, wave, lane);
    }
    const int L2048 = NEEDLUT ? p.Lphi[2048] : 0;
    StripeDma<EPI> dma;
    dma.init(p, lane);
    auto issue = [&](int c, int stage) __attribute__((always_inline)) {
        if (dma_wave) dma.issue(p, sh, wave, c, stage);
    };
    issue(cb, 0);

    // ---- the wave's activation rows (A operand: lane row fr, K bytes [64 t + 16 fg, +16) of step t),
    // issued last and unconditionally (steps past K read out of range, as zeros), so that the set-up
    // waits for its own data alone and runs while the rows are in flight
    constexpr int AL = 2 * NKS;
    v4i hf[NKS], lf[NKS];
    v4i raw[NKS][SRC == SRC_I16 ? 2 : 1];
    {
        const __amdgpu_buffer_rsrc_t rA0 = make_rsrc(p.a0, p.a0_bytes);
        const __amdgpu_buffer_rsrc_t rA1 = make_rsrc(SRC == SRC_I8 ? p.a1 : p.a0, SRC == SRC_I8 ? p.a1_bytes : p.a0_bytes);
        const int r = rbase + fr;
        const bool rok = r < p.Mreal;
#pragma unroll
        for (int t = 0; t < NKS; ++t) {
            const int k0 = t * 64 + 16 * fg;
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

    // ---- block set-up (column table, expanded GELU table, flags, form)
    vm_wait<AL>();   // the column constants, the table and chunk cb's W (older than the row loads)
    block_barrier();
    bool lut_ok;
    const int form = stripe_setup<EPI, NT>(p, sh, tid, m0, cb, ncols, craw, erv, L2048, lut_ok);

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
    const unsigned ldy4 = unsigned(p.ldy) * 4u;
    // this lane's rows are rbase + 4 fg + v
    const unsigned rowoff = unsigned(rbase + 4 * fg) * ldy4;
    unsigned yabs[4] = {0u, 0u, 0u, 0u};   // running max |y| of the lane's four rows
    int ymx[4] = {0, 0, 0, 0}, ymn[4] = {0, 0, 0, 0};   // GEGLU: running max and min of y (0 included)
    const bool lut_lds = NEEDLUT && lut_ok;
    const v4i vzero = {0, 0, 0, 0};
    // W fragment of K step t, subtile u of the chunk in LDS stage sW (B operand: lane column fr)
    auto wfrag = [&](const unsigned char* sW, int t, int u) __attribute__((always_inline)) {
        return *reinterpret_cast<const v4i*>(sW + t * S::KSTEP + pswz(16 * u + fr, fg));
    };

    if (form == FORM_INT) {
        // ---- chunk loop of the integer form
        int X[NSUB][4];   // a chunk's folded sums 256 Chi + Clo
        struct EpiC { int4 ka[NOUT], kg[NOUT]; unsigned vbase[NOUT]; };
        // per-chunk constants of the epilogue of the chunk held in X: table entries of the lane's
        // columns and the byte offset of its first output (OOB past the output's columns)
        auto epi_consts = [&](int tb, int ocol0) __attribute__((always_inline)) {
            EpiC k;
#pragma unroll
            for (int u = 0; u < NOUT; ++u) {
                const int ncol = ocol0 + 16 * u + fr;
                k.vbase[u] = ncol < nlim ? rowoff + unsigned(ncol) * 4u : OOB;
                k.ka[u] = sh.tab[tb + 16 * u + fr];
                k.kg[u] = GEGLU ? sh.tab[tb + CH / 2 + 16 * u + fr] : k.ka[u];
            }
            return k;
        };
        // output o = 4 u + v of the chunk held in X (PLAIN, GELU): requantise, store, row maximum
        auto epi_one = [&](const EpiC& k, int o, auto rmax, auto full) __attribute__((always_inline)) {
            constexpr bool RMAX = decltype(rmax)::value, FULL = decltype(full)::value;
            const int u = o >> 2, v = o & 3;
            int y;
            unsigned ay;
            if constexpr (EPI == EPI_GELU) {
                const int ya = stripe_req<NEEDLUT>(X[u][v], k.ka[u]);
                unsigned h0;
                y = stripe_mulsh16(ya, stripe_phi(sh.lut, ya), h0);
                ay = unsigned(max(y, int(0u - unsigned(y))));
            } else {
                y = stripe_req<NEEDLUT>(X[u][v], k.ka[u]);
                ay = unsigned(max(y, int(0u - unsigned(y))));
            }
            const unsigned soff = unsigned(v) * ldy4;
            __builtin_amdgcn_raw_buffer_store_b32(y, rY, int(FULL ? k.vbase[u] : k.vbase[u] + soff), FULL ? int(soff) : 0, 0);
            if constexpr (RMAX) yabs[v] = max(yabs[v], ay);
        };
        // GEGLU: the chunk's outputs computed and stored without the saturation test: y is the low
        // word of (ya ge + 2^15) >> 16, exact when the product's high word lies in [-2^15, 2^15).
        // One test per four outputs (the high words' max and min, a ballot) sends the rare group with
        // a product outside that range to a second pass that stores the saturated values again
        // (a lane's stores to one address stay in order). The row maximum then follows from each
        // row's max and min of y.
        auto epilogue_geglu = [&](int tb, int ocol0, auto rmax, auto full) __attribute__((always_inline)) {
            constexpr bool RMAX = decltype(rmax)::value, FULL = decltype(full)::value;
            int yv[NO];
#pragma unroll
            for (int u = 0; u < NOUT; ++u) {
                // the lane's a and g table entries and output offset for this subtile pair
                const StripeK3 ka = stripe_tab3(sh.tab, tb + 16 * u + fr), kg = stripe_tab3(sh.tab, tb + CH / 2 + 16 * u + fr);
                const int ncol = ocol0 + 16 * u + fr;
                const unsigned vbase = ncol < nlim ? rowoff + unsigned(ncol) * 4u : OOB;
                auto store = [&](int y, int v) __attribute__((always_inline)) {
                    const unsigned soff = unsigned(v) * ldy4;
                    __builtin_amdgcn_raw_buffer_store_b32(y, rY, int(FULL ? vbase : vbase + soff), FULL ? int(soff) : 0, 0);
                };
                int hv[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int yg = stripe_req_hi(X[u + NSUB / 2][v], kg);
                    unsigned h0, hi;
                    const int ge = stripe_mulsh16(yg, stripe_phi(sh.lut, yg), h0);
                    yv[4 * u + v] = stripe_mulsh16(stripe_req_hi(X[u][v], ka), ge, hi);
                    hv[v] = int(hi);
                    store(yv[4 * u + v], v);
                }
                const int hmx = max(max(hv[0], hv[1]), max(hv[2], hv[3]));
                const int hmn = min(min(hv[0], hv[1]), min(hv[2], hv[3]));
                if (__builtin_amdgcn_ballot_w64(hmx > 32767 || hmn < -32768)) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        if (hv[v] > 32767 || hv[v] < -32768) {
                            yv[4 * u + v] = (hv[v] >> 31) ^ 0x7fffffff;   // INT_MAX or INT_MIN, the product's sign
                            store(yv[4 * u + v], v);
                        }
                    }
                }
            }
            if constexpr (RMAX) {
#pragma unroll
                for (int o = 0; o < NO; ++o) {
                    ymx[o & 3] = max(ymx[o & 3], yv[o]);
                    ymn[o & 3] = min(ymn[o & 3], yv[o]);
                }
            }
        };
        auto epilogue = [&](int tb, int ocol0, auto rmax, auto full) __attribute__((always_inline)) {
            if constexpr (GEGLU) {
                epilogue_geglu(tb, ocol0, rmax, full);
            } else {
                const EpiC k = epi_consts(tb, ocol0);
#pragma unroll
                for (int o = 0; o < NO; ++o) epi_one(k, o, rmax, full);
            }
        };
        // the MFMAs of the chunk in LDS stage `stage`, two subtiles at a time (four independent
        // accumulator chains per K step; all four subtiles at once would not fit in the registers),
        // folded into X
        auto mfma_chunk = [&](int stage) __attribute__((always_inline)) {
            const unsigned char* sW = sh.w[stage];
            static_assert(NSUB % 2 == 0, "subtile pairs");
#pragma unroll
            for (int h = 0; h < NSUB; h += 2) {
                v4i ah[2] = {vzero, vzero}, al[2] = {vzero, vzero};
#pragma unroll
                for (int t = 0; t < NKS; ++t) {
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const v4i wf = wfrag(sW, t, h + j);
                        ah[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(hf[t], wf, ah[j], 0, 0, 0);
                        al[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(lf[t], wf, al[j], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int v = 0; v < 4; ++v) X[h + j][v] = (ah[j][v] << 8) + al[j][v];
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        // The two waves of a block on one SIMD take opposite phases: waves 0..3 run a chunk's MFMAs
        // and then its epilogue, waves 4..7 the previous chunk's epilogue and then the chunk's MFMAs
        // (their sums wait in X across the barrier), so that while one keeps the matrix core busy
        // the other works the VALU.
        const bool lagging = wave >= 4;
        auto run = [&](auto rmax, auto full) __attribute__((always_inline)) {
            for (int c = cb; c < ce; ++c) {
                prio_step(c);
                const int stage = (c - cb) & 1;
                // chunk c's DMA is done once at most the previous chunk's stores are outstanding.
                // Chunk cb needs neither wait nor barrier: every wave's W DMA of chunk cb was
                // complete before the set-up, which ends with a barrier, and the wave's own rows are
                // in (split above), so each wave starts as soon as its rows are.
                if (c > cb) {
                    vm_wait<STORES>();
                    block_barrier();
                }
                if (c + 1 < ce) issue(c + 1, stage ^ 1);
                if (lagging && c > cb) epilogue((c - 1 - cb) * CH, GEGLU ? (c - 1) * (CH / 2) : (c - 1) * CH, rmax, full);
                mfma_chunk(stage);
                if (!lagging) epilogue((c - cb) * CH, GEGLU ? c * (CH / 2) : c * CH, rmax, full);
            }
            if (lagging) epilogue((ce - 1 - cb) * CH, GEGLU ? (ce - 1) * (CH / 2) : (ce - 1) * CH, rmax, full);
        };
        const bool full = m0 + BM <= p.Mreal;
        if (p.rowmax) {
            if (full) run(std::true_type{}, std::true_type{});
            else run(std::true_type{}, std::false_type{});
        } else {
            if (full) run(std::false_type{}, std::true_type{});
            else run(std::false_type{}, std::false_type{});
        }
        if (p.rowmax) {
            // lanes with the same fg hold the same four rows: reduce over the 16 columns, one atomic per row
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                // GEGLU: |y| max from the max and min (0 - INT_MIN is 2^31 as unsigned)
                unsigned m = GEGLU ? max(unsigned(ymx[v]), 0u - unsigned(ymn[v])) : yabs[v];
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) m = max(m, unsigned(__shfl_xor(int(m), o)));
                const int r = rbase + 4 * fg + v;
                if (fr == 0 && r < p.Mreal && m) atomicMax(p.rowmax + r, m);
            }
        }
    } else {
        // ---- the reference's int64 formula (src/gemm_hl.cu:40-52, 279-302), a chunk's MFMAs then its
        // outputs one by one (the row maximum goes straight to memory)
        for (int c = cb; c < ce; ++c) {
            prio_step(c);
            const int stage = (c - cb) & 1;
            vm_wait<0>();
            block_barrier();
            if (c + 1 < ce) issue(c + 1, stage ^ 1);
            const unsigned char* sW = sh.w[stage];
            v4i ah[NSUB], al[NSUB];
#pragma unroll
            for (int u = 0; u < NSUB; ++u) {
                ah[u] = vzero;
                al[u] = vzero;
#pragma unroll
                for (int t = 0; t < NKS; ++t) {
                    const v4i wf = wfrag(sW, t, u);
                    ah[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(hf[t], wf, ah[u], 0, 0, 0);
                    al[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(lf[t], wf, al[u], 0, 0, 0);
                }
            }
            const int ocol0 = GEGLU ? c * (CH / 2) : c * CH;
#pragma unroll
            for (int u = 0; u < NOUT; ++u) {
                const int ncol = ocol0 + 16 * u + fr;
                const bool cok = ncol < nlim;
                const int col = cok ? ncol : 0;
                const int4 ca = p.cst[GEGLU ? 2 * col : col];
                const int4 cg = GEGLU ? p.cst[2 * col + 1] : ca;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int r = rbase + 4 * fg + v;
                    const int er = sh.erow[wave * G::WR + 4 * fg + v];
                    const int ya = epi1_exact(ah[u][v], al[u][v], ca.x, ca.y, ca.z, ca.w, er);
                    int y;
                    if constexpr (GEGLU) {
                        const int yg = epi1_exact(ah[u + NSUB / 2][v], al[u + NSUB / 2][v], cg.x, cg.y, cg.z, cg.w, er);
                        const i64 pg = lut_lds ? stripe_phi(sh.lut, yg) : lut16i(yg, p.Lphi);
                        const i64 ge = sat32(rshr(i64(yg) * pg, 16));
                        y = int(sat32(rshr(i64(ya) * ge, 16)));
                    } else if constexpr (EPI == EPI_GELU) {
                        const i64 pa = lut_lds ? stripe_phi(sh.lut, ya) : lut16i(ya, p.Lphi);
                        y = int(sat32(rshr(i64(ya) * pa, 16)));
                    } else {
                        y = ya;
                    }
                    // rows at or past Mreal land at or past the end of Y, columns past the output at OOB
                    const unsigned voff = cok ? rowoff + unsigned(v) * ldy4 + unsigned(ncol) * 4u : OOB;
                    __builtin_amdgcn_raw_buffer_store_b32(y, rY, int(voff), 0, 0);
                    if (p.rowmax && cok && r < p.Mreal && y) atomicMax(p.rowmax + r, uabs(y));
                }
            }
        }
    }
}

template <int SRC>
hipError_t launch_stripe16_t(int epi, const GemmParams& p, hipStream_t st) {
    const dim3 grid(unsigned(p.mtiles * p.ntiles));
    switch (epi) {
    case EPI_PLAIN: hipLaunchKernelGGL((stripe16_kernel<SRC, EPI_PLAIN>), grid, dim3(Stripe16Cfg::NT), 0, st, p); break;
    case EPI_GEGLU: hipLaunchKernelGGL((stripe16_kernel<SRC, EPI_GEGLU>), grid, dim3(Stripe16Cfg::NT), 0, st, p); break;
    case EPI_GELU: hipLaunchKernelGGL((stripe16_kernel<SRC, EPI_GELU>), grid, dim3(Stripe16Cfg::NT), 0, st, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_stripe16(int src, int epi, const GemmParams& p, hipStream_t st);

}  // namespace vk

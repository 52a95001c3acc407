// The hi/lo GEMM for shapes with few output tiles and deep K (cross-attention K/V projections,
// convolutions of the smallest images, batch-1 linears): the tiled kernels give such shapes fewer
// blocks than CUs, and each block then walks its K steps one LDS round trip at a time, so their time
// is set by the length of that chain, not by data or MFMA work.
//
// Here a block owns a 64 x 64 output tile and its four waves split the K steps among themselves
// (wave w takes steps w, w + 4, ...), each computing the whole tile over its steps with operands
// loaded straight from global memory into registers -- two steps' loads in flight while a step's
// 32 MFMAs run -- so a block has four independent chains a quarter as long. The four
// partial sums then meet in LDS in a reduce-scatter that leaves wave w with rows 16 w .. 16 w + 15
// of the tile, and the shared requantising epilogue (fused_epilogue) runs on that 64 x 64 tile as a
// Tile<64, 64, 4, 1>. Sources SRC_I16, SRC_I8 and SRC_CONV16 (C % 64 == 0: every K step lies in
// one 3x3 tap); epilogues PLAIN, SPLIT3, GEGLU and GELU.
#pragma once
#include "gemm_kernel.h"

namespace vk {

using TileKW = Tile<64, 64, 4, 1>;   // the epilogue's view: wave w owns rows 16 w .. 16 w + 15, all 64 columns

// PL planes of partial sums exchanged at once: both for the one-block-per-CU int16 sources, one at a
// time for int8 planes (two blocks per CU share the LDS)
template <int EPI, int PL>
struct KwShared {
    v4i red[PL][4][3][4][64];   // [plane][owner wave][other wave][column subtile][lane]: partial sums
    EpiShared<64, EPI == EPI_GEGLU || EPI == EPI_GELU, false> sh;
};

// the A operand of one K step over the tile's 64 rows: raw int16 (8 dwords per subtile) or the
// two int8 planes
template <int SRC>
struct KwA {
    unsigned d[4][SRC == SRC_I8 ? 4 : 8];
    v4i l[SRC == SRC_I8 ? 4 : 1];
};

// two blocks per CU (256 registers per wave) for int8 planes; the int16 sources' raw operand sets
// need the whole register file of one block per CU
template <int SRC, int EPI>
__global__ void __launch_bounds__(256, SRC == SRC_I8 ? 2 : 1) kwave_kernel(const GemmParams p) {
    prefetch_args();
    constexpr int NS = 4, MS = 4;
    constexpr bool NEEDLUT = EPI == EPI_GEGLU || EPI == EPI_GELU;
    constexpr int PL = SRC == SRC_I8 ? 1 : 2;
    __shared__ __attribute__((aligned(16))) KwShared<EPI, PL> s;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 15, fg = lane >> 4;
    const TileIdx ti = tile_index(p);
    const int m0 = ti.mt * 64, n0 = ti.nt * 64;
    const int nK = (p.Kp + 63) >> 6;

    const __amdgpu_buffer_rsrc_t rW = make_rsrc(p.w, p.w_bytes);
    const __amdgpu_buffer_rsrc_t rA0 = make_rsrc(p.a0, p.a0_bytes);
    const __amdgpu_buffer_rsrc_t rA1 = make_rsrc(SRC == SRC_I8 ? p.a1 : p.a0, SRC == SRC_I8 ? p.a1_bytes : p.a0_bytes);

    // row shifts of the tile's rows this lane reads (all four subtiles) and the epilogue's inputs
    int er4[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
        const int r = m0 + ms * 16 + fr;
        er4[ms] = r < p.Mreal ? row_shift<SRC>(p, r) : 0;
    }
    const TilePre pre = load_tile_pre<EPI, SRC, 64, 64>(p, m0, n0);
    const int L2048 = NEEDLUT ? p.Lphi[2048] : 0;
    if constexpr (NEEDLUT) {
        // GELU table entries 0..2047 -> LDS (raw), 8 KB: two 1 KB DMA instructions per wave
        const v4i rL = make_rsrc_words(p.Lphi, 2049u * 4u);
        const unsigned lbase = lds_addr(s.sh.lut) + LUT_RAW_OFF;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const unsigned c = unsigned(wave * 2 + j) * 1024u;
            dma16(rL, unsigned(lane) * 16u, c, lbase + c);
        }
    }

    // ---- per-lane operand addresses, fixed over the K loop. W: subtile ns, row fr, K chunk fg.
    unsigned w_off[NS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
        const int n = n0 + wrow_of_lds<EPI, 64>(wsub_row<EPI, TileKW>(0, ns) + fr);
        w_off[ns] = n < p.Nreal ? unsigned(n) * unsigned(p.ldw) + unsigned(16 * fg) : OOB;
    }
    // A: subtile ms, row fr, K chunk fg (16 values)
    unsigned a_off[MS];
    int a_pix[MS];
    unsigned a_mask[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
        const int r = m0 + ms * 16 + fr;
        const bool rok = r < p.Mreal;
        if constexpr (SRC == SRC_CONV16) {
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
            a_mask[ms] = mask;
            // byte offset of channel 16 fg of pixel (iy0, ix0); only taps inside the image are added to it
            a_pix[ms] = (((b * p.H + iy0) * p.W + ix0) * p.C + 16 * fg) * 2;
            a_off[ms] = 0;
        } else if constexpr (SRC == SRC_I16) {
            a_off[ms] = rok ? (unsigned(r) * unsigned(p.lda) + unsigned(16 * fg)) * 2u : OOB;
        } else {
            a_off[ms] = rok ? unsigned(r) * unsigned(p.lda) + unsigned(16 * fg) : OOB;
        }
    }

    auto load_w = [&](int kt, v4i (&wf)[NS]) {
        const unsigned kbase = unsigned(kt) * 64u;
        const bool ktail = kbase + 16u * unsigned(fg) >= unsigned(p.Kp);
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) wf[ns] = bload16(rW, ktail ? OOB : w_off[ns] + kbase);
    };
    auto load_a = [&](int kt, KwA<SRC>& a) {
        const int kbase = kt * 64;
        if constexpr (SRC == SRC_I16) {
            // two 8-value halves, each wholly inside or outside K (K % 8 == 0)
            const bool t0 = kbase + 16 * fg >= p.K, t1 = kbase + 16 * fg + 8 >= p.K;
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                const v4i x0 = bload16(rA0, t0 ? OOB : a_off[ms] + unsigned(kbase) * 2u);
                const v4i x1 = bload16(rA0, t1 ? OOB : a_off[ms] + unsigned(kbase) * 2u + 16u);
#pragma unroll
                for (int q = 0; q < 4; ++q) { a.d[ms][q] = unsigned(x0[q]); a.d[ms][4 + q] = unsigned(x1[q]); }
            }
        } else if constexpr (SRC == SRC_CONV16) {
            // implicit 3x3 im2col, tap-major K: k = tap*C + c (src/gemm_hl.cu:104-114); C % 64 == 0
            const int tap = kbase / p.C, c0 = kbase - tap * p.C;
            const int ky = (tap * 11) >> 5, kx = tap - 3 * ky;   // tap / 3, tap % 3 for tap < 9
            const int soff = ((ky * p.W + kx) * p.C + c0) * 2;
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                const bool ok = tap < 9 && ((a_mask[ms] >> tap) & 1u);
                const unsigned off = ok ? unsigned(a_pix[ms] + soff) : OOB;
                const v4i x0 = bload16(rA0, off);
                const v4i x1 = bload16(rA0, ok ? off + 16u : OOB);
#pragma unroll
                for (int q = 0; q < 4; ++q) { a.d[ms][q] = unsigned(x0[q]); a.d[ms][4 + q] = unsigned(x1[q]); }
            }
        } else {
            const bool t = unsigned(kbase) + 16u * unsigned(fg) >= unsigned(p.Kp);
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                const v4i h = bload16(rA0, t ? OOB : a_off[ms] + unsigned(kbase));
                a.l[ms] = bload16(rA1, t ? OOB : a_off[ms] + unsigned(kbase));
#pragma unroll
                for (int q = 0; q < 4; ++q) a.d[ms][q] = unsigned(h[q]);
            }
        }
    };

    // image rows of this block all have e == 0 (the usual case): a clamp is the whole quantisation
    bool e_any = false;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) e_any |= er4[ms] != 0;
    const bool wave_e0 = SRC == SRC_CONV16 ? __builtin_amdgcn_ballot_w64(e_any) == 0 : true;

    v4i acc_h[NS][MS], acc_l[NS][MS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) { acc_h[ns][ms] = v4i{0, 0, 0, 0}; acc_l[ns][ms] = v4i{0, 0, 0, 0}; }

    auto compute = [&](const v4i (&wf)[NS], KwA<SRC>& a) {
        v4i hf[MS], lf[MS];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            if constexpr (SRC == SRC_I8) {
                hf[ms] = v4i{int(a.d[ms][0]), int(a.d[ms][1]), int(a.d[ms][2]), int(a.d[ms][3])};
                lf[ms] = a.l[ms];
            } else {
                if constexpr (SRC == SRC_CONV16) {
                    if (wave_e0) clamp16_pairs(a.d[ms]);
                    else quant16_pairs(a.d[ms], er4[ms]);
                }
                split16x16(a.d[ms], hf[ms], lf[ms]);
            }
        }
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                acc_h[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ns], hf[ms], acc_h[ns][ms], 0, 0, 0);
                acc_l[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ns], lf[ms], acc_l[ns][ms], 0, 0, 0);
            }
    };

    // ---- K loop over this wave's steps kt = wave, wave + 4, ...: two operand sets in flight
    // (ping-pong buffers, no register copies, so each step waits only for its own loads). For the
    // int16 sources (one block per CU, registers to spare) the epilogue's set-up (its column and row
    // tests, the expanded table) runs after the first step's MFMAs, while the later steps' operands
    // are in flight: the first step's loads were issued after the table DMA and the set-up's own
    // inputs, and loads complete in order, so those are in by then. The int8 planes' kernel (two
    // blocks per CU) runs it after the K loop.
    constexpr bool EARLY = SRC != SRC_I8;
    EpiFlags fl;
    {
        v4i wa[NS], wb[NS];
        KwA<SRC> aa, ab;
        if (wave < nK) { load_w(wave, wa); load_a(wave, aa); }
        if (wave + 4 < nK) { load_w(wave + 4, wb); load_a(wave + 4, ab); }
        if (EARLY) {
            if (wave < nK) {
                compute(wa, aa);
                if (wave + 8 < nK) { load_w(wave + 8, wa); load_a(wave + 8, aa); }
            }
            // the set-up's first phase reads the whole raw table, a quarter of it DMA'd by each wave:
            // each wave waits for its own DMA, older than every K-step load issued since (twelve per
            // step: four W, eight A; those of steps wave + 4 and wave + 8 stay in flight), then the
            // barrier makes all four parts visible (the other epilogues have no table)
            if constexpr (NEEDLUT) {
                if (wave + 8 < nK) vm_wait<24>();
                else if (wave + 4 < nK) vm_wait<12>();
                else vm_wait<0>();
                block_barrier();
            } else {
                if (wave >= nK) vm_wait<0>();
            }
            fl = epi_setup<EPI, SRC, 64, 64, 256>(p, pre, L2048, s.sh);
        }
        for (int kt = wave; kt < nK; kt += 8) {
            if (!EARLY || kt > wave) {
                compute(wa, aa);
                if (kt + 8 < nK) { load_w(kt + 8, wa); load_a(kt + 8, aa); }
            }
            if (kt + 4 < nK) {
                compute(wb, ab);
                if (kt + 12 < nK) { load_w(kt + 12, wb); load_a(kt + 12, ab); }
            }
        }
    }

    // ---- reduce-scatter (both planes at once, or one at a time): wave w ends with the sums of
    // column subtiles ns and row subtile w
    v4i fin_h[NS][1], fin_l[NS][1];
    auto scatter = [&](v4i (&acc)[NS][MS], v4i (&fin)[NS][1], int pl) {
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
            if (ms != wave) {
                const int slot = wave - (wave > ms ? 1 : 0);
#pragma unroll
                for (int ns = 0; ns < NS; ++ns) s.red[pl][ms][slot][ns][lane] = acc[ns][ms];
            }
    };
    auto gather = [&](v4i (&acc)[NS][MS], v4i (&fin)[NS][1], int pl) {
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
            if (ms == wave)
#pragma unroll
                for (int ns = 0; ns < NS; ++ns) {
                    v4i t = acc[ns][ms];
#pragma unroll
                    for (int o = 0; o < 3; ++o) t += s.red[pl][ms][o][ns][lane];
                    fin[ns][0] = t;
                }
    };
    if constexpr (PL == 2) {
        scatter(acc_h, fin_h, 0);
        scatter(acc_l, fin_l, 1);
        __syncthreads();
        gather(acc_h, fin_h, 0);
        gather(acc_l, fin_l, 1);
    } else {
        scatter(acc_h, fin_h, 0);
        __syncthreads();
        gather(acc_h, fin_h, 0);
        __syncthreads();
        scatter(acc_l, fin_l, 0);
        __syncthreads();
        gather(acc_l, fin_l, 0);
    }

    if constexpr (!EARLY) {
        // the table DMA above is outside the compiler's counts: wait for it before the set-up reads it
        if constexpr (NEEDLUT) vm_wait<0>();
        __syncthreads();
        fl = epi_setup<EPI, SRC, 64, 64, 256>(p, pre, L2048, s.sh);
    }
    int er[1] = {0};
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
        if (ms == wave) er[0] = er4[ms];
    fused_epilogue<EPI, SRC, TileKW>(p, fin_h, fin_l, m0 + 16 * wave, n0, 0, s.sh, fl, er);
}

template <int SRC, int EPI>
hipError_t launch_kwave_t(const GemmParams& p, hipStream_t st) {
    hipLaunchKernelGGL((kwave_kernel<SRC, EPI>), dim3(unsigned(p.mtiles * p.ntiles)), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace vk

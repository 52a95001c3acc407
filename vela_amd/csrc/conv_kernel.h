// Implicit 3x3 / pad 1 / stride 1 convolution with halo reuse, for the SRC_CONV16 source (NHWC
// int16 image, K index tap*C + c, tap = 3*ky + kx, src/gemm_hl.cu:104-114 semantics).
//
// A tile of 128 output rows is TR = 128 / Wo complete output rows of one image. For each 64-channel
// chunk the block loads the tile's input patch once -- PR = TR + 2 input rows of PC = W + 2 pixels
// (zero halo), 128 bytes per pixel -- into LDS, and the nine taps of that chunk read their MFMA
// fragments from it at a per-tap pixel offset ky*PC + kx. The im2col operand is never formed, in
// HBM or in LDS: with TR >= 8 the patch holds 1.4-1.6x the tile's own pixels instead of the 9x of
// the tap tiles. W streams one 64-deep step per tap, as in gemm_dma_kernel. K runs chunk-major
// (chunk, tap) instead of tap-major; the integer sums are exact, so the order changes no bit.
//
// LDS: W in a 3-stage ring (8 KB per step), the patch in a 2-slot ring (one chunk computing, the
// next loading); both arrive by buffer-load DMA. About 79 KB per block, two blocks per CU; the
// GELU-table epilogues (16 KB more) stay on gemm_dma_kernel.
//
// Selection (host side): stride 1, C % 64 == 0, Wo <= 16 so that a tile holds at least eight
// output rows, Ho a multiple of TR, and a patch of at most 208 pixels. On MI355X this measured
// 2-7% faster than the tile kernels for 16x16 images; for wider images the 128-row tiles (a patch
// would not fit 64-row tiles at three blocks per CU) leave CUs idle in the last round and lost.
#pragma once
#include "gemm_kernel.h"

namespace vk {

struct HaloCfg {
    static constexpr int BM = 128, BN = 128;
    using T = Tile<BM, BN, 4, 1>;
    static constexpr int W_BYTES = BN * 64;
    static constexpr int W_INS = W_BYTES / 1024 / 4;        // W DMA instructions per wave per step
    static constexpr int NSTW = 3;                           // W stages
    static constexpr int P_CAP = 26;                         // patch slot, in 1 KB DMA instructions (208 pixels)
    static constexpr int P_BYTES = P_CAP * 1024;
    // patch instructions of wave w: j = w, w + 4, ... < P_CAP
    static constexpr int p_ins(int w) { return (P_CAP - w + 3) / 4; }
    static constexpr int P_INS_MAX = (P_CAP + 3) / 4;
};

// Host-side selection of the halo kernel for a SRC_CONV16 problem.
inline bool halo_fits(int H, int W, int C, int stride, int Ho, int Wo) {
    if (stride != 1 || Ho != H || Wo != W || (C & 63) || Wo > 16 || HaloCfg::BM % Wo) return false;
    const int TR = HaloCfg::BM / Wo;
    if (Ho % TR) return false;
    return (TR + 2) * (W + 2) * 128 <= HaloCfg::P_BYTES;
}

template <int EPI>
__global__ void __launch_bounds__(256, 2) conv_halo_kernel(const GemmParams p) {
    prefetch_args();
    using HC = HaloCfg;
    constexpr int BM = HC::BM;
    using T = typename HC::T;
    constexpr int BN = HC::BN, MS = T::MS, NS = T::NS, NSTW = HC::NSTW;
    constexpr bool FUSED = EPI != EPI_PARTIAL;
    static_assert(EPI != EPI_GEGLU && EPI != EPI_GELU, "GELU-table epilogues run on gemm_dma_kernel");

    __shared__ __attribute__((aligned(16))) unsigned char smemW[NSTW * HC::W_BYTES];
    __shared__ __attribute__((aligned(16))) unsigned char smemP[2 * HC::P_BYTES];
    __shared__ __attribute__((aligned(16))) EpiShared<FUSED ? BN : 1, false, EPI == EPI_PLAIN_GN> sh;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const TileIdx ti = tile_index(p);
    const int m0 = ti.mt * BM, n0 = ti.nt * BN;
    const int nC = p.C >> 6;
    const int cb = ti.ks * p.kper, ce = min(nC, cb + p.kper);   // this unit's channel chunks
    const int steps = (ce - cb) * 9;

    // ---- tile geometry: TR output rows of Wo pixels from output row oy0 of image img0; patch PR x PC
    const int HoWo = p.Ho * p.Wo;
    const int TR = BM / p.Wo, PC = p.W + 2, NP = (TR + 2) * PC;
    const int img0 = m0 / HoWo, oy0 = (m0 - img0 * HoWo) / p.Wo;

    // ---- loads that complete before every DMA below (see gemm_dma_kernel)
    const int rbase = m0 + wave * T::WTM;
    int er[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
        const int r = rbase + ms * 16 + (lane & 15);
        er[ms] = r < p.Mreal ? row_shift<SRC_CONV16>(p, r) : 0;
    }
    TilePre pre{};
    if constexpr (FUSED) pre = load_tile_pre<EPI, SRC_CONV16, BM, BN>(p, m0, n0);

    const v4i rW = make_rsrc_words(p.w, p.w_bytes);
    const v4i rA = make_rsrc_words(p.a0, p.a0_bytes);

    // ---- W lane state (as gemm_dma_kernel)
    unsigned w_off[HC::W_INS];
#pragma unroll
    for (int j = 0; j < HC::W_INS; ++j) {
        const int R = 8 * (wave * HC::W_INS + j) + (lane >> 3), lc = (lane & 7) ^ swz16_key(R);   // pswz, as gemm_dma_kernel
        const int lr = 2 * R + (lc >> 2);
        const int nrow = n0 + (FUSED ? wrow_of_lds<EPI, BN>(lr) : lr);
        const int wk = 16 * (lc & 3);
        w_off[j] = nrow < p.Nreal ? unsigned(nrow) * unsigned(p.ldw) + unsigned(wk) : OOB;
    }
    // ---- patch lane state: instruction q of this wave covers patch pixels 8*(4q + wave) + lane/8,
    // chunk position lane%8 holding the global 16-byte chunk that the swizzle puts there; pixels
    // outside the image (the halo) or past the patch read as zeros
    unsigned p_off[HC::P_INS_MAX];
#pragma unroll
    for (int q = 0; q < HC::P_INS_MAX; ++q) {
        const int P = 8 * (4 * q + wave) + (lane >> 3);
        unsigned off = OOB;
        if (4 * q + wave < HC::P_CAP && P < NP) {
            const int pr = P / PC, pc = P - pr * PC;
            const int iy = oy0 - 1 + pr, ix = pc - 1;
            if (m0 < p.Mreal && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W) {
                const int chunk = (lane & 7) ^ swz16_key(P);
                off = unsigned((((img0 * p.H + iy) * p.W + ix) * p.C) * 2 + chunk * 16);
            }
        }
        p_off[q] = off;
    }
    // ---- fragment rows: tile row -> patch pixel of tap (0, 0)
    int P0[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
        const int prow = wave * T::WTM + ms * 16 + (lane & 15);
        const int py = prow / p.Wo, px = prow - py * p.Wo;
        P0[ms] = py * PC + px;
    }

    auto issueW = [&](int g, int slot) {
        const int chunk = cb + g / 9, tap = g - (g / 9) * 9;
        const unsigned kbase = unsigned(tap * p.C + chunk * 64);
        const unsigned sbase = lds_addr(smemW) + slot * HC::W_BYTES;
#pragma unroll
        for (int j = 0; j < HC::W_INS; ++j) dma16(rW, w_off[j], kbase, sbase + (wave * HC::W_INS + j) * 1024);
    };
    auto issueP = [&](int chunk, int slot) {
        const unsigned sbase = lds_addr(smemP) + slot * HC::P_BYTES;
        const unsigned coff = unsigned(chunk) * 128u;   // 64 channels of int16
#pragma unroll
        for (int q = 0; q < HC::P_INS_MAX; ++q)
            if (4 * q + wave < HC::P_CAP)
                dma16(rA, p_off[q] == OOB ? OOB : p_off[q] + coff, 0u, sbase + (4 * q + wave) * 1024);
    };

    // first patch and the first two W steps load while the tables are still ahead
    if (steps > 0) issueP(cb, 0);
    if (steps > 0) issueW(0, 0);
    if (steps > 1) issueW(1, 1);

    bool e_any = false;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) e_any |= er[ms] != 0;
    const bool wave_e0 = __builtin_amdgcn_ballot_w64(e_any) == 0;

    v4i acc_h[NS][MS], acc_l[NS][MS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            acc_h[ns][ms] = v4i{0, 0, 0, 0};
            acc_l[ns][ms] = v4i{0, 0, 0, 0};
        }

    auto compute = [&](int wslot, int pslot, int doff) {
        const unsigned char* sW = smemW + wslot * HC::W_BYTES;
        const unsigned char* sP = smemP + pslot * HC::P_BYTES;
        const int fr = lane & 15, fg = lane >> 4;
        v4i hf[MS], lf[MS];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            const int P = P0[ms] + doff;
            const v4i x0 = *reinterpret_cast<const v4i*>(sP + swz16(P, 2 * fg));
            const v4i x1 = *reinterpret_cast<const v4i*>(sP + swz16(P, 2 * fg + 1));
            unsigned d[8] = {unsigned(x0[0]), unsigned(x0[1]), unsigned(x0[2]), unsigned(x0[3]),
                             unsigned(x1[0]), unsigned(x1[1]), unsigned(x1[2]), unsigned(x1[3])};
            if (wave_e0) clamp16_pairs(d);
            else quant16_pairs(d, er[ms]);
            split16x16(d, hf[ms], lf[ms]);
        }
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
            const int row = (FUSED ? wsub_row<EPI, T>(0, ns) : ns * 16) + fr;
            const v4i wf = *reinterpret_cast<const v4i*>(sW + pswz(row, fg));
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                acc_h[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, hf[ms], acc_h[ns][ms], 0, 0, 0);
                acc_l[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, lf[ms], acc_l[ns][ms], 0, 0, 0);
            }
        }
    };

    // ---- K loop: step g = (chunk, tap). At tap 0 of chunk c the patch of chunk c + 1 starts
    // loading (its slot held chunk c - 1, finished by every wave at this barrier), then W step g + 2.
    // Waits: before step g, the DMA issued after W(g) is W(g + 1), plus, at tap 1, the patch of the
    // next chunk (issued between W(g) and W(g + 1)); the patch of chunk c itself is older than W(g).
    const bool wave_hi = wave >= (HC::P_CAP & 3 ? (HC::P_CAP & 3) : 4);   // waves issuing one patch instruction fewer
    int tap = 0, chunk = cb, wslot = 0;
    for (int g = 0; g < steps; ++g) {
        if (g + 1 >= steps) vm_wait<0>();
        else if (tap == 1 && chunk + 1 < ce) {
            if (wave_hi) vm_wait<HC::p_ins(3) + HC::W_INS>();
            else vm_wait<HC::P_INS_MAX + HC::W_INS>();
        } else vm_wait<HC::W_INS>();
        block_barrier();
        if (tap == 0 && chunk + 1 < ce) issueP(chunk + 1, (chunk + 1 - cb) & 1);
        if (g + 2 < steps) issueW(g + 2, wslot == 0 ? 2 : wslot - 1);
        const int ky = (tap * 11) >> 5, kx = tap - 3 * ky;
        compute(wslot, (chunk - cb) & 1, ky * PC + kx);
        wslot = wslot == NSTW - 1 ? 0 : wslot + 1;
        if (++tap == 9) { tap = 0; ++chunk; }
    }

    if constexpr (EPI == EPI_PARTIAL) {
        store_partial<T>(p, acc_h, acc_l, rbase, n0, ti.ks);
    } else {
        const EpiFlags fl = epi_setup<EPI, SRC_CONV16, BM, BN, 256>(p, pre, 0, sh);
        fused_epilogue<EPI, SRC_CONV16, T>(p, acc_h, acc_l, rbase, n0, 0, sh, fl, er);
        if constexpr (EPI == EPI_PLAIN_GN) gn_flush(p, sh);
    }
}

inline hipError_t launch_conv_halo(int epi, const GemmParams& p, hipStream_t st) {
    dim3 grid(unsigned(p.mtiles * p.ntiles * p.ksplit));
    switch (epi) {
    case EPI_PLAIN: hipLaunchKernelGGL(conv_halo_kernel<EPI_PLAIN>, grid, dim3(256), 0, st, p); break;
    case EPI_PLAIN_GN: hipLaunchKernelGGL(conv_halo_kernel<EPI_PLAIN_GN>, grid, dim3(256), 0, st, p); break;
    case EPI_SPLIT3: hipLaunchKernelGGL(conv_halo_kernel<EPI_SPLIT3>, grid, dim3(256), 0, st, p); break;
    case EPI_PARTIAL: hipLaunchKernelGGL(conv_halo_kernel<EPI_PARTIAL>, grid, dim3(256), 0, st, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace vk

// Row-stationary ("stripe") hi/lo GEMM for shallow K (Kp <= 640) with int16 rows (SRC_I16) or int8
// planes (SRC_I8), epilogues PLAIN (+ residual), GEGLU and GELU, with or without the row maximum.
//
// A block owns BM activation rows and a range of W rows (output columns). Each wave loads its rows
// once, splits them into hi/lo MFMA fragments and keeps those in registers for the whole block;
// W streams through LDS in chunks of CH rows (a 2-stage ring filled by buffer-load DMA), and each
// chunk is multiplied and requantised before the next. So an activation row is read from memory
// and split once per block instead of once per 128-column tile, the GELU table and the per-column
// constants are set up once per block, and the row maximum of a wave's rows over the block's
// columns needs one atomic per row at the end.
//
// Epilogue (src/gemm_hl.cu:40-52, 279-302). When every row of the block has e == 0 and no element
// can saturate (checked per block from max |m| 2^-s and max |b|), b is folded into the FMA constant:
// y = floor(A m 2^-s + (128 wsum m 2^-s + 1/2 + b)), exact in FP64 because Kp |m| < 2^30. GEGLU then
// takes phi(g) from the table as (1024 L[i] + (L[i+1] - L[i]) f) >> 10 (one 24-bit multiply-add),
// ge = floor((g phi + 2^15) 2^-16) and y = sat32(floor(a 2^-16 ge + 1/2)); both products are exact
// below 2^53 or saturate monotonically. Other blocks run the general FP64 form with separate
// saturating adds, or the reference's int64 formula element by element when a shift or multiplier
// is outside the FP64 range.
//
// Memory ordering: the W DMA of chunk c + 1 is issued right after the barrier of chunk c, and the
// only vector-memory instructions after it in chunk c are that chunk's output stores, a fixed
// number per lane (every lane stores unconditionally; rows and columns outside the output go to
// an out-of-range buffer offset, which the hardware drops). So waiting for at most that many
// outstanding operations completes the DMA. Blocks whose epilogue loads from memory (residual, b
// of the general form, the int64 form) wait for all of them instead.
#pragma once
#include "gemm_kernel.h"

namespace vk {

template <int MS_, int NKM_, int CH_>
struct Stripe {
    static constexpr int MS = MS_;       // 16-row MFMA subtiles per wave (rows per wave = 16 MS)
    static constexpr int NKM = NKM_;     // 64-deep K steps held in registers (Kp <= 64 NKM)
    static constexpr int CH = CH_;       // W rows per chunk
    static constexpr int NS = CH / 16;   // 16-column MFMA subtiles per chunk
    static constexpr int BM = 64 * MS;   // four waves stacked along M
    static constexpr int KSTEP = CH * 64;            // LDS bytes of one K step of a chunk
    static constexpr int STAGE = NKM * KSTEP;        // LDS bytes of one chunk
    static constexpr int NCOLS = 1280;               // W rows (table columns) per block, at most
    static constexpr int CMAX = NCOLS / CH;          // chunks per block, at most
    static constexpr int CPT = NCOLS / 256;          // table columns per thread
    static constexpr int DMA_INS = STAGE / 1024 / 4; // DMA instructions per wave per chunk
    static_assert(STAGE % 4096 == 0 && NS % 2 == 0, "stripe geometry");
};
typedef Stripe<2, 5, 64> StripeA;    // Kp <= 320: 32 rows per wave, 64-row chunks
typedef Stripe<1, 10, 32> StripeB;   // Kp <= 640: 16 rows per wave, 32-row chunks

struct alignas(16) ColConst {
    double ms;   // m 2^-s
    double wm;   // 128 wsum m 2^-s; + 1/2 when e == 0; + b as well when the block folds b
};

template <class S, bool LUT>
struct StripeShared {
    unsigned char w[2][S::STAGE];
    ColConst tab[S::NCOLS];
    int2 lut[LUT ? 2050 : 1];   // lut[i + 1] = (1024 L[i], L[i+1] - L[i]); lut[0] below, lut[2049] above the table
    unsigned long long umax;
    int flag[8];                // emin, emax, smin, smax, column bound failed, table range failed, max |b|, b not foldable
};

// byte offset inside sh.lut of the raw table as the DMA delivers it (entries 0..2047)
constexpr unsigned STRIPE_LUT_RAW = 8192;

template <int SRC, int EPI, class S>
__global__ void __launch_bounds__(256, 2) stripe_kernel(const GemmParams p) {
    constexpr int MS = S::MS, NS = S::NS, NKM = S::NKM, CH = S::CH, BM = S::BM;
    constexpr bool NEEDLUT = EPI == EPI_GEGLU || EPI == EPI_GELU;
    constexpr bool GEGLU = EPI == EPI_GEGLU;
    constexpr bool SMALLK = NKM * 64 <= 496;   // |256 Chi + Clo| < 2^31
    constexpr int NOUT = GEGLU ? NS / 2 : NS;  // output subtiles per chunk
    constexpr int STORES = NOUT * MS;          // output stores per lane per chunk
    static_assert(SRC == SRC_I16 || SRC == SRC_I8, "stripe sources");
    static_assert(EPI == EPI_PLAIN || EPI == EPI_GEGLU || EPI == EPI_GELU, "stripe epilogues");

    __shared__ __attribute__((aligned(16))) StripeShared<S, NEEDLUT> sh;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 15, fg = lane >> 4;
    const TileIdx ti = tile_index(p);
    const int m0 = ti.mt * BM;
    const int nch = (p.Nreal + CH - 1) / CH;
    const int cb = ti.nt * p.kper, ce = min(nch, cb + p.kper);   // this block's chunks
    const int nK = (p.Kp + 63) >> 6;
    const int rbase = m0 + wave * 16 * MS;
    const int nlim = GEGLU ? (p.Nreal >> 1) : p.Nreal;
    if (cb >= ce) return;   // (the host sizes the grid so that every block has a chunk)

    if (tid == 0) {
        sh.flag[0] = INT_MAX; sh.flag[1] = INT_MIN; sh.flag[2] = INT_MAX; sh.flag[3] = INT_MIN;
        sh.flag[4] = 0; sh.flag[5] = 0; sh.flag[6] = 0; sh.flag[7] = 0;
        sh.umax = 0;
    }

    // ---- the wave's activation rows: loads first (they are older than every DMA below)
    int er[MS];
    unsigned yoff[MS];   // byte offset of the output row, or out of range
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
        const int r = rbase + ms * 16 + fr;
        er[ms] = (r < p.Mreal && p.e) ? p.e[r] : 0;
        yoff[ms] = r < p.Mreal ? unsigned(r) * unsigned(p.ldy) * 4u : OOB;
    }
    v4i hf[MS][NKM], lf[MS][NKM];
    {
        const __amdgpu_buffer_rsrc_t rA0 = make_rsrc(p.a0, p.a0_bytes);
        const __amdgpu_buffer_rsrc_t rA1 = make_rsrc(SRC == SRC_I8 ? p.a1 : p.a0, SRC == SRC_I8 ? p.a1_bytes : p.a0_bytes);
        v4i raw[MS][NKM][SRC == SRC_I16 ? 2 : 1];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
            const int r = rbase + ms * 16 + fr;
            const bool rok = r < p.Mreal;
#pragma unroll
            for (int ks = 0; ks < NKM; ++ks) {
                const int k0 = ks * 64 + 16 * fg;
                if (ks < nK) {
                    if constexpr (SRC == SRC_I16) {
                        // 16 int16 values = two 16-byte pieces; K % 8 == 0, so each piece is all in or all out
                        const unsigned off = (unsigned(r) * unsigned(p.lda) + unsigned(k0)) * 2u;
                        raw[ms][ks][0] = bload16(rA0, rok && k0 < p.K ? off : OOB);
                        raw[ms][ks][1] = bload16(rA0, rok && k0 + 8 < p.K ? off + 16u : OOB);
                    } else {
                        const unsigned off = unsigned(r) * unsigned(p.lda) + unsigned(k0);
                        const bool ok = rok && k0 < p.Kp;
                        hf[ms][ks] = bload16(rA0, ok ? off : OOB);
                        lf[ms][ks] = bload16(rA1, ok ? off : OOB);
                    }
                } else {
                    if constexpr (SRC == SRC_I16) raw[ms][ks][0] = raw[ms][ks][1] = v4i{0, 0, 0, 0};
                    else hf[ms][ks] = lf[ms][ks] = v4i{0, 0, 0, 0};
                }
            }
        }
        if constexpr (SRC == SRC_I16) {
#pragma unroll
            for (int ms = 0; ms < MS; ++ms)
#pragma unroll
                for (int ks = 0; ks < NKM; ++ks) {
                    const v4i x0 = raw[ms][ks][0], x1 = raw[ms][ks][1];
                    const unsigned d[8] = {unsigned(x0[0]), unsigned(x0[1]), unsigned(x0[2]), unsigned(x0[3]),
                                           unsigned(x1[0]), unsigned(x1[1]), unsigned(x1[2]), unsigned(x1[3])};
                    split16x16(d, hf[ms][ks], lf[ms][ks]);
                }
        }
    }

    // ---- DMA: the GELU table (raw), then W chunk cb
    if constexpr (NEEDLUT) {
        const v4i rL = make_rsrc_words(p.Lphi, 2049u * 4u);
        const unsigned lbase = lds_addr(sh.lut) + STRIPE_LUT_RAW;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const unsigned c = unsigned(wave * 2 + j) * 1024u;
            dma16(rL, unsigned(lane) * 16u, c, lbase + c);
        }
    }
    const int L2048 = NEEDLUT ? p.Lphi[2048] : 0;
    const v4i rW = make_rsrc_words(p.w, p.w_bytes);
    // instruction j of this wave fills K step ks, LDS rows 16 rg .. 16 rg + 15 of a chunk; lane l
    // reads 16 bytes of W row w_row (chunk-relative) at K offset w_k (its swizzled position)
    constexpr int RG = CH / 16;
    unsigned w_off[S::DMA_INS];
    int w_row[S::DMA_INS];
#pragma unroll
    for (int j = 0; j < S::DMA_INS; ++j) {
        const int q = wave * S::DMA_INS + j, ks = q / RG, rg = q - ks * RG;
        const int lr = 16 * rg + (lane >> 2);
        w_row[j] = wrow_of_lds<EPI, CH>(lr);
        const int wk = ks * 64 + 16 * ((lane & 3) ^ swz_key(lr));
        w_off[j] = wk < p.Kp ? unsigned(w_row[j]) * unsigned(p.ldw) + unsigned(wk) : OOB;
    }
    auto issue = [&](int c, int stage) {
        const int n0 = c * CH;
        const unsigned sbase = lds_addr(sh.w[stage]);
#pragma unroll
        for (int j = 0; j < S::DMA_INS; ++j) {
            const int q = wave * S::DMA_INS + j, ks = q / RG, rg = q - ks * RG;
            const bool ok = n0 + w_row[j] < p.Nreal;
            dma16(rW, ok ? w_off[j] : OOB, unsigned(n0) * unsigned(p.ldw), sbase + unsigned(ks * S::KSTEP + rg * 1024));
        }
    };
    if (cb < ce) issue(cb, 0);

    // ---- block set-up: column constants of chunks [cb, ce), the expanded GELU table, flags
    vm_wait<S::DMA_INS>();   // the table DMA (older than chunk cb's)
    block_barrier();
    EpiFlags fl;
    {
        constexpr int LPT = NEEDLUT ? (2050 + 255) / 256 : 1;
        int2 lv[LPT];
        int lbad = 0;
        if constexpr (NEEDLUT) {
            const int* raw = reinterpret_cast<const int*>(reinterpret_cast<const char*>(sh.lut) + STRIPE_LUT_RAW);
#pragma unroll
            for (int q = 0; q < LPT; ++q) {
                const int i = tid + 256 * q;
                int2 v = make_int2(0, 0);
                if (i == 2049) v = make_int2(65536 << 10, 0);
                else if (i >= 1 && i < 2049) {
                    const int a = raw[i - 1], nx = i - 1 == 2047 ? L2048 : raw[i];
                    if (a < 0 || a > 65536 || nx < 0 || nx > 65536) lbad = 1;
                    v = make_int2(int(unsigned(a) << 10), nx - a);
                }
                lv[q] = v;
            }
        }
        const int ncols = (ce - cb) * CH;
        int bb[S::CPT];
        int smn = INT_MAX, smx = INT_MIN, bad = 0, bmx = 0, nofold = 0;
        double um = 0.0;
#pragma unroll
        for (int q = 0; q < S::CPT; ++q) {
            const int j = tid + 256 * q;
            bb[q] = 0;
            if (j < ncols) {
                const int n = cb * CH + (j / CH) * CH + wrow_of_lds<EPI, CH>(j % CH);
                double ms = 0.0, wmv = 0.0;
                if (n < p.Nreal) {
                    const int4 c = p.cst[n];
                    const i64 mag = (c.x < 0 ? -i64(c.x) : i64(c.x)) * i64(p.Kp);
                    if (mag >= (1LL << 30) || c.y < -1000 || c.y > 1000) bad = 1;
                    smn = min(smn, c.y);
                    smx = max(smx, c.y);
                    if (c.y >= -1000 && c.y <= 1000) {
                        ms = ldexp(double(c.x), -c.y);
                        wmv = ldexp(128.0 * (double(c.w) * double(c.x)), -c.y);
                        // |acc m 2^-s| <= 2^22 Kp |m| 2^-s, since |acc| <= 32768 * 128 * Kp
                        um = max(um, ldexp(4194304.0 * double(p.Kp) * fabs(double(c.x)), -c.y));
                        // wm + 1/2 + b is exact when |b| 2^s < 2^51 (numerator below 2^53)
                        if (ldexp(fabs(double(c.z)), c.y) >= 2251799813685248.0) nofold = 1;
                    }
                    bb[q] = c.z;
                    bmx = max(bmx, int(min(uabs(c.z), 0x7fffffffu)));
                }
                sh.tab[j] = ColConst{ms, wmv};
            }
        }
        int emn = INT_MAX, emx = INT_MIN;
        if (tid < BM && m0 + tid < p.Mreal) emn = emx = p.e ? p.e[m0 + tid] : 0;
#pragma unroll
        for (int o = 32; o; o >>= 1) {
            emn = min(emn, __shfl_xor(emn, o));
            emx = max(emx, __shfl_xor(emx, o));
            smn = min(smn, __shfl_xor(smn, o));
            smx = max(smx, __shfl_xor(smx, o));
            bad |= __shfl_xor(bad, o);
            bmx = max(bmx, __shfl_xor(bmx, o));
            nofold |= __shfl_xor(nofold, o);
            um = max(um, __shfl_xor(um, o));
            if constexpr (NEEDLUT) lbad |= __shfl_xor(lbad, o);
        }
        if (lane == 0) {
            if (emn <= emx) { atomicMin(&sh.flag[0], emn); atomicMax(&sh.flag[1], emx); }
            if (smn <= smx) { atomicMin(&sh.flag[2], smn); atomicMax(&sh.flag[3], smx); }
            if (bad) atomicOr(&sh.flag[4], 1);
            if (lbad) atomicOr(&sh.flag[5], 1);
            atomicMax(&sh.flag[6], bmx);
            if (nofold) atomicOr(&sh.flag[7], 1);
            atomicMax(&sh.umax, __double_as_longlong(um));
        }
        __syncthreads();   // raw table read by everyone, all flags in
        if constexpr (NEEDLUT) {
#pragma unroll
            for (int q = 0; q < LPT; ++q) {
                const int i = tid + 256 * q;
                if (i < 2050) sh.lut[i] = lv[q];
            }
        }
        const i64 emin = sh.flag[0], emax = sh.flag[1], smin = sh.flag[2], smax = sh.flag[3];
        fl.fast = !sh.flag[4] && (smin - emax >= 1) && (smax - emin <= 52) && emin >= -1000 && emax <= 1000;
        if (NEEDLUT && sh.flag[5]) fl.fast = false;
        fl.ezero = emin > emax || (emin == 0 && emax == 0);
        fl.fold = fl.fast && fl.ezero && !sh.flag[7] && __longlong_as_double(sh.umax) + double(sh.flag[6]) + 2.0 < 2147483647.0;
        if (fl.ezero) {
            // the FMA constant of the e == 0 forms: wm + 1/2, and + b when folded (exact, see above)
#pragma unroll
            for (int q = 0; q < S::CPT; ++q) {
                const int j = tid + 256 * q;
                if (j < ncols) sh.tab[j].wm = (sh.tab[j].wm + 0.5) + (fl.fold ? double(bb[q]) : 0.0);
            }
        }
        __syncthreads();
    }

    const __amdgpu_buffer_rsrc_t rY = make_rsrc(p.Y, p.y_bytes);
    const __amdgpu_buffer_rsrc_t rR = make_rsrc(p.R ? p.R : p.Y, p.y_bytes);
    // per-wave row maximum so far: max |y| = max(ymax, -ymin)
    int ymax[MS], ymin[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) { ymax[ms] = 0; ymin[ms] = 0; }
    double pr[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) pr[ms] = ldexp(1.0, min(max(er[ms], -1000), 1000));
    const bool lean = fl.fold && !p.R;   // the epilogue issues stores only

    // GELU factor: z = x + 2^20 clamped to [-1, 2^21]; entry (z >> 10) + 1 = (x >> 10) + 1025 and
    // z & 1023 = x & 1023; (1024 L[i] + d f) >> 10 = L[i] + ((d f) >> 10) (|d f| < 2^27)
    auto phi = [&](int x) -> int {
        const int xc = min(max(x, -1048577), 1048576);
        const int2 t = sh.lut[(xc >> 10) + 1025];
        return (t.x + __mul24(t.y, xc & 1023)) >> 10;
    };
    auto comb = [&](int h, int l) -> double {
        if constexpr (SMALLK) return double((h << 8) + l);
        else return __builtin_fma(double(h), 256.0, double(l));
    };

    for (int c = cb; c < ce; ++c) {
        const int stage = (c - cb) & 1;
        // chunk c's DMA is done once at most the previous chunk's stores are outstanding
        if (c > cb && lean) vm_wait<STORES>();
        else vm_wait<0>();
        block_barrier();
        if (c + 1 < ce) issue(c + 1, stage ^ 1);

        v4i acc_h[NS][MS], acc_l[NS][MS];
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                acc_h[ns][ms] = v4i{0, 0, 0, 0};
                acc_l[ns][ms] = v4i{0, 0, 0, 0};
            }
        const unsigned char* sW = sh.w[stage];
#pragma unroll
        for (int ks = 0; ks < NKM; ++ks) {
            if (ks < nK) {
#pragma unroll
                for (int ns = 0; ns < NS; ++ns) {
                    const v4i wf = *reinterpret_cast<const v4i*>(sW + ks * S::KSTEP + swz(ns * 16 + fr, fg));
#pragma unroll
                    for (int ms = 0; ms < MS; ++ms) {
                        acc_h[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, hf[ms][ks], acc_h[ns][ms], 0, 0, 0);
                        acc_l[ns][ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, lf[ms][ks], acc_l[ns][ms], 0, 0, 0);
                    }
                }
            }
        }

        // ---- epilogue of chunk c: output subtile i covers table rows i*16 + 4 fg + v (GEGLU: a
        // columns; the g columns are CH/2 further), output columns ocol0 + i*16 + 4 fg + v
        const int tb = (c - cb) * CH;
        const int ocol0 = GEGLU ? c * (CH / 2) : c * CH;
#pragma unroll
        for (int i = 0; i < NOUT; ++i) {
            const int lr = i * 16 + 4 * fg;
            const int ncol = ocol0 + lr;
            const bool cok = ncol < nlim;   // nlim % 4 == 0: the lane's four columns are all in or all out
            const int ig = GEGLU ? i + NS / 2 : i;
            ColConst ca[4], cg[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                ca[v] = sh.tab[tb + lr + v];
                if constexpr (GEGLU) cg[v] = sh.tab[tb + CH / 2 + lr + v];
            }
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                int y[4];
                if (fl.fold) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const double ya = __builtin_floor(__builtin_fma(comb(acc_h[i][ms][v], acc_l[i][ms][v]), ca[v].ms, ca[v].wm));
                        if constexpr (GEGLU) {
                            const double yg = __builtin_floor(__builtin_fma(comb(acc_h[ig][ms][v], acc_l[ig][ms][v]), cg[v].ms, cg[v].wm));
                            const double ge = __builtin_floor(__builtin_fma(yg, double(phi(int(yg))), 32768.0) * (1.0 / 65536.0));
                            y[v] = cvt_sat(__builtin_floor(__builtin_fma(ya * (1.0 / 65536.0), ge, 0.5)));
                        } else if constexpr (EPI == EPI_GELU) {
                            y[v] = int(__builtin_floor(__builtin_fma(ya, double(phi(int(ya))), 32768.0) * (1.0 / 65536.0)));
                        } else {
                            y[v] = int(ya);
                        }
                    }
                } else if (fl.fast) {
                    // general FP64 form: floor(A m 2^-(s-e) + 1/2) saturated, + b saturated
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        auto one = [&](int h, int l, const ColConst& k, int col) -> int {
                            const int n = cok ? col : 0;
                            const int b = p.cst[n].z;
                            double X;
                            if (fl.ezero) X = __builtin_fma(comb(h, l), k.ms, k.wm);
                            else X = __builtin_fma(__builtin_fma(comb(h, l), k.ms, k.wm), pr[ms], 0.5);
                            return add_sat(cvt_sat(__builtin_floor(X)), b);
                        };
                        const int na = GEGLU ? 2 * (ncol + v) : ncol + v;
                        const int ya = one(acc_h[i][ms][v], acc_l[i][ms][v], ca[v], na);
                        if constexpr (GEGLU) {
                            const int yg = one(acc_h[ig][ms][v], acc_l[ig][ms][v], cg[v], na + 1);
                            const double ge = __builtin_floor(__builtin_fma(double(yg), double(phi(yg)), 32768.0) * (1.0 / 65536.0));
                            y[v] = cvt_sat(__builtin_floor(__builtin_fma(double(ya), ge, 32768.0) * (1.0 / 65536.0)));
                        } else if constexpr (EPI == EPI_GELU) {
                            y[v] = int(__builtin_floor(__builtin_fma(double(ya), double(phi(ya)), 32768.0) * (1.0 / 65536.0)));
                        } else {
                            y[v] = ya;
                        }
                    }
                } else {
                    // the reference's int64 formula
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int col = cok ? ncol + v : 0;
                        if constexpr (GEGLU) {
                            const int4 ka = p.cst[2 * col], kg = p.cst[2 * col + 1];
                            const int ya = epi1_exact(acc_h[i][ms][v], acc_l[i][ms][v], ka.x, ka.y, ka.z, ka.w, er[ms]);
                            const int yg = epi1_exact(acc_h[ig][ms][v], acc_l[ig][ms][v], kg.x, kg.y, kg.z, kg.w, er[ms]);
                            y[v] = geglu_exact(ya, yg, p.Lphi);
                        } else {
                            const int4 k = p.cst[col];
                            int yy = epi1_exact(acc_h[i][ms][v], acc_l[i][ms][v], k.x, k.y, k.z, k.w, er[ms]);
                            if constexpr (EPI == EPI_GELU) yy = gelu_exact(yy, p.Lphi);
                            y[v] = yy;
                        }
                    }
                }
                const unsigned off = cok ? yoff[ms] + unsigned(ncol) * 4u : OOB;
                if constexpr (EPI == EPI_PLAIN) {
                    if (p.R) {
                        const v4i rv = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rR, int(off), 0, 0));
#pragma unroll
                        for (int v = 0; v < 4; ++v) y[v] = add_sat(y[v], rv[v]);
                    }
                }
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v4i{y[0], y[1], y[2], y[3]}),
                                                       rY, int(off), 0, 0);
                if (p.rowmax && cok) {
                    ymax[ms] = max(max(ymax[ms], y[0]), max(y[1], max(y[2], y[3])));
                    ymin[ms] = min(min(ymin[ms], y[0]), min(y[1], min(y[2], y[3])));
                }
            }
        }
    }

    if (p.rowmax) {
        // lanes fr, fr + 16, fr + 32, fr + 48 hold the same row: one atomic per row and wave
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

template <int SRC, class S>
hipError_t launch_stripe_t(int epi, const GemmParams& p, hipStream_t st) {
    const dim3 grid(unsigned(p.mtiles * p.ntiles));
    switch (epi) {
    case EPI_PLAIN: hipLaunchKernelGGL((stripe_kernel<SRC, EPI_PLAIN, S>), grid, dim3(256), 0, st, p); break;
    case EPI_GEGLU: hipLaunchKernelGGL((stripe_kernel<SRC, EPI_GEGLU, S>), grid, dim3(256), 0, st, p); break;
    case EPI_GELU: hipLaunchKernelGGL((stripe_kernel<SRC, EPI_GELU, S>), grid, dim3(256), 0, st, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_stripe(int src, int shape, int epi, const GemmParams& p, hipStream_t st);

}  // namespace vk

/*
 * TEST INFRASTRUCTURE ONLY -- CPU restatement of the reference's W8A16 hi/lo integer GEMM path.
 *
 * This header and oracle.c are the correctness oracle (and the timed CPU baseline) for the MI355X
 * library in vela_amd/. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * the built liboracle.so, and only as the checker. The product path never calls it.
 *
 * Every function cites the reference (emanwrxsti/vela, paths relative to the repository root) whose
 * behaviour it restates. Integer overflow that is undefined behaviour in the reference's C++ (int64
 * products, int32 LUT interpolation) is restated with two's-complement wrapping, which is what the
 * GPU hardware executing the reference produces.
 */
#ifndef VELA_ORACLE_H
#define VELA_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Source and epilogue codes: the reference's GemmSrc / GemmEpi values (src/gemm_hl.h:8-9) plus the
 * two int16 sources of this build (SRC_I16 = packed 16-bit view of the hi/lo planes, SRC_CONV16 =
 * NHWC int16 image with the SRC_CONV32 semantics). */
enum { ORC_SRC_I8 = 0, ORC_SRC_X32 = 1, ORC_SRC_CONV32 = 2, ORC_SRC_I16 = 3, ORC_SRC_CONV16 = 4 };
enum { ORC_EPI_PLAIN = 0, ORC_EPI_SPLIT3 = 1, ORC_EPI_GEGLU = 2, ORC_EPI_GELU = 3 };

typedef struct OrcGemm {
    /* A operand (src/gemm_hl.h:12-17) */
    int src;
    const int8_t* hi; const int8_t* lo; int ld8;   /* SRC_I8 planes */
    const int32_t* e;                                /* per-row shift: SRC_I8 / SRC_I16 / SRC_CONV* (NULL = 0) */
    const int32_t* x; int ldx; const uint32_t* xrowmax; /* SRC_X32 */
    const int16_t* q16; int ld16;                    /* SRC_I16 */
    const int32_t* img; const int16_t* img16;        /* SRC_CONV32 / SRC_CONV16, NHWC */
    int K, H, W, C, stride, Ho, Wo;
    /* problem */
    int Mreal, Nreal, Kp;
    const int8_t* w; int ldw;                        /* W [Np x Kp], row n = output column n */
    const int32_t* cst;                              /* int4 {m, s, b, wsum} per column */
    /* epilogue (src/gemm_hl.h:18-22) */
    int epi;
    int32_t* Y; int ldy; const int32_t* residual;
    int Cs; int32_t* Y1; int32_t* Y2;
    const int32_t* Lphi;
    uint32_t* rowmax;
} OrcGemm;

void orc_set_threads(int n);
int orc_get_threads(void);

/* ---- exact integer primitives: src/intops.cuh */
int64_t orc_sat32(int64_t v);
int64_t orc_rshr(int64_t v, int64_t s);
int orc_row_exp(int64_t m);
int64_t orc_quant16(int64_t v, int e);
int32_t orc_quant16_32(int32_t v, int e);
int32_t orc_lut16i(int64_t x, const int32_t* L);
void orc_split16(int64_t a, int8_t* hi, int8_t* lo);
int32_t orc_epi1(int32_t chi, int32_t clo, const int32_t* c4, int32_t er);
int32_t orc_geglu(int32_t a, int32_t g, const int32_t* L);
int32_t orc_gelu(int32_t y, const int32_t* L);
/* element-wise batch forms of the primitives, for the known-answer tests */
void orc_rshr_n(const int64_t* v, const int64_t* s, int64_t* out, size_t n);
void orc_row_exp_n(const int64_t* m, int32_t* out, size_t n);
void orc_quant16_32_n(const int32_t* v, const int32_t* e, int32_t* out, size_t n);
void orc_lut16i_n(const int64_t* x, const int32_t* L, int32_t* out, size_t n);
void orc_epi1_n(const int32_t* chi, const int32_t* clo, const int32_t* c4, const int32_t* er, int32_t* out, size_t n);

/* ---- A-operand producers and cuBLASLt-path epilogues: src/kernels.cu, src/gemm_hl.cu */
void orc_quant_rows(const int32_t* X, int M, int K, int ldx, int8_t* hi, int8_t* lo, int32_t* e, int Kp);
void orc_pixmax(const int32_t* X, int rows, int C, uint32_t* pm);
void orc_im2col3(const int32_t* X, const uint32_t* pm, int B, int H, int W, int C, int stride,
                 int8_t* hi, int8_t* lo, int32_t* e, int Kp);
void orc_conv_e(const uint32_t* pm, int B, int H, int W, int stride, int32_t* e);
void orc_epilogue(const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int32_t* cst,
                  const int32_t* e, int32_t* Y, int ldy, const int32_t* R);
void orc_epilogue_split(const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int32_t* cst,
                        const int32_t* e, int Cs, int32_t* Y0, int32_t* Y1, int32_t* Y2);
void orc_epilogue_geglu_q(const int32_t* Chi, const int32_t* Clo, int M, int F, int ldc, const int32_t* cst,
                          const int32_t* e, const int32_t* L, int8_t* hi, int8_t* lo, int32_t* eo, int Kp);

/* GroupNorm statistics (EPI_PLAIN, k_epilogue with gs): accumulate into sum/mn/mx [(M / T) * 32] */
void orc_gn_accumulate(const int32_t* Y, int M, int N, int ldy, int T, int64_t* sum, int32_t* mn, int32_t* mx);
void orc_gn_ref_tile(int Mp, int Np, int Kp, int src8, int* BMr, int* BNr);
void orc_gn_tiles(const int32_t* Y, int M, int N, int ldy, int T, int BMr, int BNr, int64_t* sum, int32_t* mn, int32_t* mx);
void orc_gn_blocks(const int32_t* Y, int M, int N, int ldy, int T, int64_t* sum, int32_t* mn, int32_t* mx);
/* EPI_QKV outputs from the plain output Y [M x 3C]: head-quantised q/k planes and V [M x C] */
void orc_qkv_heads(const int32_t* Y, int M, int ldy, int C, int heads, int T, int TpQ, int TpK,
                   int8_t* qhi, int8_t* qlo, int32_t* qe, int64_t* qhs, int64_t* qls, int64_t* qts,
                   int8_t* khi, int8_t* klo, int32_t* ke, int64_t* khs, int64_t* kls, int64_t* kts, int32_t* V);

/* ---- the GEMMs */
/* one row of the A operand as hi/lo planes (Kp bytes each) and its shift e; returns 0 or -1 */
int orc_a_row(const OrcGemm* g, int r, int8_t* hi, int8_t* lo, int32_t* e);
/* the hi/lo GEMM with its fused epilogue (src/gemm_hl.cu:65-310); rows [r0, r1) only (r1 <= 0: all) */
int orc_gemm_hl_rows(const OrcGemm* g, int r0, int r1);
int orc_gemm_hl(const OrcGemm* g);
/* per-plane int32 dot products only: Chi/Clo [Mreal x ldc] */
int orc_gemm_planes(const OrcGemm* g, int32_t* Chi, int32_t* Clo, int ldc);
/* C = A * W^T, int8 x int8 -> int32, strided batch (src/gemm.cu:46-70) */
void orc_i8gemm(const int8_t* A, int lda, long long sA, const int8_t* W, int ldw, long long sW,
                int32_t* C, int ldc, long long sC, int M, int N, int K, int batch);

/* ---- weight preparation: src/engine.cu:26-44 (tap-major permutation, wsum, cst) */
void orc_prep_weight(const int8_t* w, int N, int K, int conv3, const int32_t* m, const int32_t* s,
                     const int32_t* b, int Np, int Kp, int8_t* wout, int32_t* cst_out);
/* interleave two linears row-wise (a0, g0, a1, g1, ...): src/engine.cu:81-88 */
void orc_interleave2(const int8_t* wa, const int32_t* ca, const int8_t* wg, const int32_t* cg, int N, int Kp,
                     int8_t* wout, int32_t* cout);

/* ---- integer normalisations: src/kernels.cu:172-305,349-420 with src/intops.cuh:18-56.
 * Records use the GnStat layout (src/kernels.h:9): sum, mn, mx, mean, e, ss, sd. */
typedef struct OrcGnStat {
    int64_t sum;
    int32_t mn, mx;
    int64_t mean;
    int32_t e;
    int64_t ss, sd;
} OrcGnStat;
int64_t orc_floor_div(int64_t a, int64_t b);                 /* src/intops.cuh:18 */
int64_t orc_isqrt(int64_t v);                                /* src/intops.cuh:51-56 */
void orc_gn_init(OrcGnStat* gs, int cnt);                    /* src/kernels.cu:173 */
void orc_gn_stats1(const int32_t* X, int B, int T, int C, int groups, OrcGnStat* gs);  /* :175-183 sum/mn/mx (accumulates) */
void orc_gn_fin1(OrcGnStat* gs, int cnt, int64_t n);          /* :185-192 */
void orc_gn_stats2(const int32_t* X, int B, int T, int C, int groups, OrcGnStat* gs);  /* :193-201 ss (accumulates) */
void orc_gn_fin2(OrcGnStat* gs, int cnt, int64_t n, int64_t den);                       /* :203-210 */
void orc_gn_apply(const int32_t* X, int B, int T, int C, int groups, const OrcGnStat* gs, const int64_t* g, const int64_t* beta, int32_t* Y);  /* :211-219 */
/* :287-305 (k_gn_apply_row): Y + pm, or the int16 view when hi != NULL (Lsig may be NULL) */
void orc_gn_apply_row(const int32_t* X, int B, int T, int C, int groups, const OrcGnStat* gs, const int32_t* g, const int32_t* beta,
                      const int32_t* Lsig, int32_t* Y, uint32_t* pm, int8_t* hi, int8_t* lo, int32_t* e, int Kp);
void orc_lnorm(const int32_t* X, int M, int C, const int64_t* g, const int64_t* beta, int64_t den, int32_t* Y);       /* :221-246 */
void orc_lnorm_q(const int32_t* X, int M, int C, const int32_t* g, const int32_t* beta, int64_t den, int8_t* hi, int8_t* lo,
                 int32_t* e, int Kp);                                                                                 /* :349-390 */

/* ---- the elementwise kernels between the GEMMs (src/kernels.h:31-35, src/kernels.cu:537-561) */
void orc_act(int32_t* X, size_t n, const int32_t* L);                                 /* :537 in place */
void orc_geglu_n(int32_t* A, const int32_t* G, size_t n, const int32_t* L);          /* :538-542 in place */
void orc_add(int32_t* X, const int32_t* Y, size_t n);                                 /* :543 in place */
/* :544-556: out = [A | B] per row; gs (may be NULL): GroupNorm records by the per-256-element rule */
void orc_concat(const int32_t* A, int Ca, const int32_t* B, int Cb, int rows, int32_t* out, OrcGnStat* gs, int T);
void orc_upsample2(const int32_t* X, int B, int H, int W, int C, int32_t* out);     /* :557-561 */

/* ---- attention: the operand producers and the exact softmax attention (src/kernels.h:42-50,61,
 * src/kernels.cu:611-672,799-805; src/attn.cu:1-6 with src/kernels.cu:673-722 as its unfused form).
 * Heads of 64, G = B * heads groups; Q/K planes [G * Tp x 64] with e, hs, ls, tsum per row; V
 * transposed planes [G * 64 x Tkp] with ev and vsum per (g, d). Lexp: 1025 exp-table entries. */
void orc_quant_heads(const int32_t* X, int B, int T, int C, int heads, int Tp, int8_t* hi, int8_t* lo, int32_t* e, int64_t* hs,
                     int64_t* ls, int64_t* tsum);                                                                   /* :611-631 */
void orc_quant_heads_pad(int G, int T, int Tp, int8_t* hi, int8_t* lo, int32_t* e, int64_t* hs, int64_t* ls, int64_t* tsum);  /* :799-805 */
void orc_quant_v(const int32_t* X, int B, int Tk, int C, int heads, int Tkp, int8_t* vth, int8_t* vtl, int32_t* ev, int64_t* vsum);  /* :632-672 */
/* out[(b * Tq + q) * C + h * 64 + d] for q < Tq; rowmax[b * Tq + q] = max(rowmax, |out|) when rowmax != NULL */
void orc_attention(const int8_t* qh, const int8_t* ql, const int32_t* eq, const int8_t* kh, const int8_t* kl, const int32_t* ek,
                   const int8_t* vth, const int8_t* vtl, const int32_t* ev, int B, int heads, int Tq, int Tqp, int Tk, int Tkp,
                   int causal, const int64_t* Lexp, int C, int32_t* out, uint32_t* rowmax);

#ifdef __cplusplus
}
#endif
#endif

/*
 * vgemm -- MI355X (gfx950) W8A16 hi/lo-split integer GEMM: the C ABI of libvgemm.so.
 *
 * Drop-in for the GEMM path of emanwrxsti/vela (supr-meow-vela). Each entry point names the
 * reference interface it replaces (file:line in that repository). All pointers are device pointers
 * unless stated; `stream` is a hipStream_t (NULL = the null stream). Every call is asynchronous on
 * the stream, allocates no device memory and is legal inside hipStreamBeginCapture. Return value:
 * VGEMM_OK, or a negative code with a message in vgemm_last_error() (thread-local).
 *
 * Arithmetic contract (src/gemm_hl.h:1-3):
 *   q   = 256*hi + lo + 128                      (the 16-bit activation; hi = q>>8, lo = (q&255)-128)
 *   acc = sum_k q[r,k] * W[n,k] = 256*Chi + Clo + 128*wsum[n]
 *   Y[r,n] = sat32(rshr(acc * m[n], s[n] - e[r]) + b[n])     (+ residual, saturated)
 * with cst[n] = int4 {m, s, b, wsum} and rshr/sat32 as in src/intops.cuh:9-17. Outputs are bit-exact.
 */
#ifndef VGEMM_H
#define VGEMM_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    VGEMM_OK = 0,
    VGEMM_ERR_ARG = -1,      /* invalid argument or unsupported shape (reference: std::runtime_error) */
    VGEMM_ERR_HIP = -2,      /* a HIP runtime call failed */
    VGEMM_ERR_UNSUPPORTED = -3
};

/* Epilogues: meow::GemmEpi values (src/gemm_hl.h:8). */
enum { VGEMM_EPI_PLAIN = 0, VGEMM_EPI_SPLIT3 = 1, VGEMM_EPI_GEGLU = 2, VGEMM_EPI_GELU = 3, VGEMM_EPI_QKV = 4 };

/* A sources: meow::GemmSrc values (src/gemm_hl.h:9) plus two int16 sources of this library:
 *   VGEMM_SRC_I16    : int16 q [rows x ld16] -- the hi/lo planes of SRC_I8 stored as one 16-bit
 *                      value (half the bytes of the int32 activations, the same bytes as the planes);
 *                      split into signed hi / offset lo int8 on load. e[row] as for SRC_I8.
 *   VGEMM_SRC_CONV16 : SRC_CONV32 semantics on an NHWC int16 image. */
enum { VGEMM_SRC_I8 = 0, VGEMM_SRC_X32 = 1, VGEMM_SRC_CONV32 = 2, VGEMM_SRC_I16 = 3, VGEMM_SRC_CONV16 = 4 };

/* A operand: meow::ASrc (src/gemm_hl.h:12-17), same fields in the same order, plus q16/ld16/img16. */
typedef struct VgemmASrc {
    int src;
    const int8_t* hi; const int8_t* lo; int ld8; const int32_t* e;         /* SRC_I8 (e may be NULL = 0) */
    const int32_t* x; int ldx; const uint32_t* rowmax; int K;              /* SRC_X32 (K = real columns) */
    const int32_t* img; int H, W, C, stride, Ho, Wo;                       /* SRC_CONV32 (K = 9C, C % 16 == 0) */
    /* Convolution sources (SRC_CONV32, SRC_CONV16) with e == NULL and rowmax != NULL: rowmax holds the
     * image's per-pixel maximum |x| ([B*H*W], as k_pixmax writes it, or the AEpi.rowmax of the GEMM
     * that produced the image) and each output row's shift is derived in the kernel by k_conv_e's
     * rule (src/gemm_hl.cu:335-341), so no k_conv_e launch or e buffer is needed. */
    const int16_t* q16; int ld16;                                          /* SRC_I16 (K % 8, ld16 % 8) */
    const int16_t* img16;                                                  /* SRC_CONV16 (C % 8 == 0, C <= 16384) */
} VgemmASrc;

/* GroupNorm statistics record: meow::GnStat (src/kernels.h:9), same fields and layout (48 bytes). The
 * GEMM epilogue accumulates sum, mn and mx; mean, e, ss and sd belong to the normalisation after it. */
typedef struct VgemmGnStat {
    int64_t sum;
    int32_t mn, mx;
    int64_t mean;
    int32_t e;
    int64_t ss, sd;
} VgemmGnStat;

/* Epilogue description: meow::AEpi (src/gemm_hl.h:18-26) in the same order, plus an optional
 * split-K workspace (ws, ws_bytes; none = no split-K). Fields an epilogue does not read are ignored,
 * as the reference ignores them (src/gemm_hl.cu:176-177, 279-296): gnstat outside EPI_PLAIN, the
 * residual on EPI_GEGLU / EPI_SPLIT3 / EPI_QKV, rowmax on EPI_SPLIT3 / EPI_QKV.
 *   gnstat/gnT (EPI_PLAIN): add the sum, min and max of every output y (after the residual) to
 *     gnstat[(row / gnT) * 32 + col / (Nreal / 32)]; Nreal % 32 == 0, gnT % 64 == 0; the caller
 *     initialises the records (vgemm_gn_init). src/gemm_hl.cu:175-177, 285-287, 306-309.
 *   EPI_QKV: Nreal = 3C, C = 64*heads, rows = B*T. Columns [0, C) (q) and [C, 2C) (k) are quantised per
 *     row and head (e = row_exp(max |y| over the head's 64 columns)) into hi/lo int8
 *     [(b*heads + head)*Tp + t][64] with e and the int64 sums of hi, lo and q per row and head
 *     (Tp = TpQ for q, TpK for k; rows t >= T are not written); columns [2C, 3C) (v) go to Y2 [rows x C]
 *     as int32. Y is not used. src/gemm_hl.cu:179-241. */
typedef struct VgemmAEpi {
    int epi; int32_t* Y; int ldy; const int32_t* residual;
    int Cs; int32_t* Y1; int32_t* Y2; const int32_t* Lphi;
    uint32_t* rowmax;                   /* optional: atomicMax of |y| per output row (caller zeroes it) */
    void* gnstat; int gnT;              /* optional GroupNorm statistics (VgemmGnStat records) */
    int heads, T, TpQ, TpK, C;          /* EPI_QKV geometry */
    int8_t *qhi, *qlo, *khi, *klo; int32_t *qe, *ke;
    int64_t *qhs, *qls, *qts, *khs, *kls, *kts;
    void* ws; size_t ws_bytes;          /* optional split-K workspace (device memory) */
} VgemmAEpi;

/* Fill an ASrc / AEpi with the reference's default member values (src = SRC_I8, stride = 1, rest 0). */
void vgemm_asrc_init(VgemmASrc* a);
void vgemm_aepi_init(VgemmAEpi* e);

/* meow::k_gemm_hl2 (src/gemm_hl.h:27, src/gemm_hl.cu:350-370). W [Np x Kp] int8 (ld ldw), row n =
 * output column n; rows of A >= Mreal and columns >= Nreal are neither read as data nor written. */
int vgemm_hl2(void* stream, const VgemmASrc* A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal,
              int Kp, const int32_t* cst, const VgemmAEpi* E);

/* No counterpart in the reference's fused GEMM: the int16 view of the output instead of Y (the
 * semantics of its quant_row_out, src/kernels.cu:317-331, as k_epilogue_geglu_q / k_quant_rows give
 * them): per output row r < Mreal, e = row_exp(max |y|) into V->e[r], q = quant16_32(y, e) into the
 * planes V->hi / V->lo [Mreal x V->ld] (hi = q >> 8, lo = (q & 255) - 128), columns [nout, ld) padded
 * with (0, -128). EPI_PLAIN / EPI_GEGLU / EPI_GELU with int16 rows or int8 planes; E's residual,
 * rowmax and statistics must be NULL and E->Y is not written; V->ld % 16 == 0, planes 16-byte
 * aligned. Needs vgemm_view_workspace_bytes() of workspace in E->ws. Kp <= 320 runs the fused
 * row-stationary form (three kernels); deeper K writes the GEMM's int32 rows into the workspace and
 * quantises them (the tile kernels, then k_quant_rows). */
typedef struct VgemmView {
    int8_t* hi; int8_t* lo; int32_t* e; int ld;
} VgemmView;
int vgemm_hl2_view(void* stream, const VgemmASrc* A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal,
                   int Kp, const int32_t* cst, const VgemmAEpi* E, const VgemmView* V);

/* No counterpart in the reference: vgemm_hl2 for callers that cannot allocate device memory (code
 * under stream capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments, same
 * results; AEpi.ws / ws_bytes are ignored and the split-K partials go to a static device workspace
 * of VGEMM_NOALLOC_WS_BYTES (64 MiB) that each GPU holds until the process ends. A call whose split
 * would need more returns VGEMM_ERR_UNSUPPORTED (no BASELINE or UNet shape does: the largest needs
 * 60 MiB). Every call on one GPU shares that GPU's workspace: calls that overlap on one GPU (other
 * streams, other threads) race. No hipMalloc, hipFree or allocating library call is made. */
#define VGEMM_NOALLOC_WS_BYTES ((size_t)64 << 20)
int vgemm_hl2_noalloc(void* stream, const VgemmASrc* A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal,
                      int Kp, const int32_t* cst, const VgemmAEpi* E);

/* meow::k_gemm_hl (src/gemm_hl.h:30-33, src/gemm_hl.cu:371-376): SRC_I8 planes + epilogue. */
int vgemm_hl(void* stream, const int8_t* Ahi, const int8_t* Alo, int lda, int Mp, int Mreal,
             const int8_t* W, int ldw, int Np, int Nreal, int Kp, const int32_t* cst, const int32_t* e,
             int32_t* Y, int ldy, const int32_t* residual, int epi, int Cs, int32_t* Y1, int32_t* Y2,
             const int32_t* Lphi);

/* meow::k_conv_e (src/gemm_hl.h:29, src/gemm_hl.cu:335-349): e[row] = row_exp(max over the 3x3
 * window of pm), rows = B*Ho*Wo. */
int vgemm_conv_e(void* stream, const uint32_t* pm, int B, int H, int W, int stride, int32_t* e);

/* meow::gemm_hl_supported (src/gemm_hl.h:34, src/gemm_hl.cu:344): Mp % 64, Np % 64, Kp % 16. */
int vgemm_supported(int Mp, int Np, int Kp);

/* meow::g_gemm_hl_variant (src/gemm_hl.h:35, src/gemm_hl.cu:345): tile override, -1 = automatic.
 * This library's variants: 0 = 128x128 tiles, 1 = 64x128, 2 = 128x64, 3 = 128x256 (rows x columns),
 * 4 = the row-stationary kernel (Kp <= 320), 5 = the K-split-over-waves kernel (64x64 tiles, the
 * four waves of a block splitting K); 4 and 5 apply to the calls their kernels serve and leave the
 * others to automatic selection, as do values outside the table. */
void vgemm_set_variant(int v);
int vgemm_get_variant(void);

/* Output rows per tile (128) of the halo-reuse 3x3 kernel that vgemm_hl2 runs for a SRC_CONV16 source
 * with this geometry and epilogue when no variant is forced, or 0 when such calls run the
 * implicit-im2col tile kernels. The halo kernel takes stride 1, C % 64 == 0, output rows of at most
 * 16 pixels (eight or more whole rows per tile), H a multiple of the rows per tile, and no GELU-table
 * epilogue. No counterpart in the reference; for tests and tuning. */
int vgemm_conv16_halo_rows(int H, int W, int C, int stride, int epi);

/* Split-K: force the number of K partitions (0 = automatic, 1 = never). */
void vgemm_set_splitk(int s);
/* No counterpart in the reference. A vgemm_hl2 call without AEpi.ws whose shape wants a K split
 * (deep K over fewer tiles than CUs) uses a workspace the library allocates for its (device, stream)
 * on the first such call outside stream capture and keeps until the process ends (a later call that
 * needs more gets a larger one; none is freed, as captured graphs may refer to them); under capture
 * with none yet it runs unsplit. A graph captured with such calls uses its capture stream's
 * workspace: replay it on that stream. on = 0 turns this off (every call without AEpi.ws then runs
 * unsplit); default on. */
void vgemm_set_stream_workspaces(int on);
/* Tile order over the XCDs: -1 automatic, 0 row stripes per XCD, 1 column groups per XCD. The order
 * changes which blocks share an L2, never a result bit. No counterpart in the reference (its tile
 * raster is CUDA's block order); a tuning and test knob like vgemm_set_splitk. */
void vgemm_set_tile_order(int order);
/* ---- Integer normalisations on either side of the GEMM (src/kernels.h:21-24,59-63,66-67), bit-exact
 * with src/kernels.cu:172-305,349-420: GroupNorm of X[B, T, C] (NHWC rows, `groups` groups of C /
 * groups channels) from VgemmGnStat records -- gathered by a GEMM epilogue (AEpi.gnstat, after
 * vgemm_gn_init) and finalised by vgemm_gn_fin1, or by vgemm_gn_stats1 -- and LayerNorm rows.
 * C % 4 == 0 and C <= 2560 throughout; groups <= 64 (32 for gn_apply_row) and C % groups == 0; X, Y, g and beta 16-byte
 * aligned; int16-view planes hi/lo [rows x Kp] with Kp >= C, Kp % 4 == 0, 4-byte aligned. */
int vgemm_gn_stats1(void* stream, const int32_t* X, int B, int T, int C, int groups, void* gs);   /* k_gn_stats1: init, sum/min/max, fin1 */
int vgemm_gn_fin1(void* stream, void* gs, int cnt, int64_t n);                                   /* k_gn_fin1: mean, e (n = T * C / groups) */
int vgemm_gn_stats2(void* stream, const int32_t* X, int B, int T, int C, int groups, int64_t den, void* gs);   /* k_gn_stats2: ss, fin2 (sd) */
int vgemm_gn_apply(void* stream, const int32_t* X, int B, int T, int C, int groups, const void* gs, const int64_t* g, const int64_t* beta,
                   int32_t* Y);                                                                    /* k_gn_apply (elementwise, 64-bit g/beta) */
/* k_gn_apply_row: + SiLU through Lsig when not NULL; int32 Y plus pm[row] = max |y| (pm may be NULL), or
 * the int16 view hi/lo/e when hi != NULL. pm is what a following convolution takes as ASrc.rowmax. */
int vgemm_gn_apply_row(void* stream, const int32_t* X, int B, int T, int C, int groups, const void* gs, const int32_t* g,
                       const int32_t* beta, const int32_t* Lsig, int32_t* Y, uint32_t* pm, int8_t* hi, int8_t* lo, int32_t* e, int Kp);
int vgemm_lnorm(void* stream, const int32_t* X, int M, int C, const int64_t* g, const int64_t* beta, int64_t den, int32_t* Y);   /* k_lnorm */
int vgemm_lnorm_q(void* stream, const int32_t* X, int M, int C, const int32_t* g, const int32_t* beta, int64_t den, int8_t* hi,
                  int8_t* lo, int32_t* e, int Kp);                                                 /* k_lnorm_q: the int16 view of the row */

/* Workspace bytes the int16 view (vgemm_hl2_view) of an Mreal x Nreal x Kp call with this epilogue
 * needs: for Kp <= 320 the row maxima, one exponent byte and one 32-bit mask per (row, 32 output
 * columns); deeper, the int32 output rows and the GEMM's split-K workspace at the current settings. */
size_t vgemm_view_workspace_bytes(int Mreal, int Nreal, int Kp, int epi);
/* Workspace bytes vgemm_hl2 uses for this shape at the current settings (0 = no split-K). */
size_t vgemm_workspace_bytes(int Mp, int Mreal, int Np, int Nreal, int Kp, int epi);

/* meow::Gemm (src/gemm.h:12-23, src/gemm.cu:7-70): C[M,N] = A[M,K] * W[N,K]^T, int8 x int8 -> int32,
 * row-major, optional strided batch. K % 16 == 0, N % 4 == 0, 16-byte aligned pointers.
 * The handle replaces the cuBLASLt plan cache (this library keeps no plans). vgemm_i8_create allocates
 * ws_bytes of device memory on the current device, as the reference's Gemm::init allocates cuBLASLt's
 * workspace (src/gemm.cu:7-11): a call with batch 1, deep K (>= 2048) and fewer output tiles than
 * CUs splits K into it and sums the ranges in a second kernel. Calls on one handle share that
 * workspace and must not overlap; 0 bytes disables the split. */
int vgemm_i8_create(size_t ws_bytes, void** handle);
int vgemm_i8_destroy(void* handle);
int vgemm_i8_run(void* handle, void* stream, const int8_t* A, int lda, long long strideA, const int8_t* W, int ldw,
                 long long strideW, int32_t* C, int ldc, long long strideC, int M, int N, int K, int batch);

/* A-operand producers and cuBLASLt-path epilogues (src/kernels.h:11-21, 68-70). */
/* meow::k_quant_rows (src/kernels.h:12-13): per-row quantisation of X[M,K] into hi/lo [Mp32 x Kp] + e. */
int vgemm_quant_rows(void* stream, const int32_t* X, int M, int K, int ldx, int8_t* hi, int8_t* lo, int32_t* e, int Kp);
/* meow::k_epilogue (src/kernels.h:14-17). gs (VgemmGnStat records, or null): add the sum, min and max
 * of every output (after the residual) to gs[(row / T) * 32 + col / (N / 32)]; needs N % 32 == 0 and
 * (T*N) % 1024 == 0. */
int vgemm_epilogue(void* stream, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int32_t* cst,
                   const int32_t* e, int32_t* Y, int ldy, const int32_t* residual, void* gs, int T);
/* meow::k_pixmax (src/kernels.h:18-19). */
int vgemm_pixmax(void* stream, const int32_t* X, int rows, int C, uint32_t* pm);
/* meow::k_im2col3 (src/kernels.h:20-21). */
int vgemm_im2col3(void* stream, const int32_t* X, const uint32_t* pm, int B, int H, int W, int C, int stride,
                  int8_t* hi, int8_t* lo, int32_t* e, int Kp);
/* meow::k_epilogue_split (src/kernels.h:68-69). */
int vgemm_epilogue_split(void* stream, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int32_t* cst,
                         const int32_t* e, int Cs, int32_t* Y0, int32_t* Y1, int32_t* Y2);
/* meow::k_epilogue_geglu_q (src/kernels.h:70). */
int vgemm_epilogue_geglu_q(void* stream, const int32_t* Chi, const int32_t* Clo, int M, int F, int ldc, const int32_t* cst,
                           const int32_t* e, const int32_t* Lphi, int8_t* hi, int8_t* lo, int32_t* eo, int Kp);

/* Graph capture of a GEMM sequence (src/engine.cu:625-630, 661-667 capture the forward). begin/end
 * wrap hipStreamBeginCapture (thread-local mode) / hipStreamEndCapture + hipGraphInstantiate. */
int vgemm_graph_begin(void* stream);
int vgemm_graph_end(void* stream, void** exec);
int vgemm_graph_launch(void* exec, void* stream);
int vgemm_graph_destroy(void* exec);

/* Fill `count` uint32 words with `value` by a kernel (capture-safe replacement for the
 * cudaMemsetAsync that zeroes rowmax buffers, src/engine.cu:161). */
int vgemm_fill_u32(void* stream, uint32_t* p, size_t count, uint32_t value);

/* ---- integer elementwise kernels between the GEMMs (src/kernels.h:31-35, src/kernels.cu:537-566,
 * launchers :767-771), bit-exact; in place where the reference is. L is a 2049-entry Q16 table
 * (lut.sigmoid for SiLU, lut.phi for GELU), interpolated by lut16i. */
int vgemm_act(void* stream, int32_t* X, size_t n, const int32_t* L);                       /* k_act: x = sat32(rshr(x lut(x), 16)) */
int vgemm_geglu(void* stream, int32_t* A, const int32_t* G, size_t n, const int32_t* L);   /* k_geglu: a = sat32(rshr(a sat32(rshr(g lut(g), 16)), 16)) */
int vgemm_add(void* stream, int32_t* X, const int32_t* Y, size_t n);                        /* k_add: x = sat32(x + y) */
/* k_concat: out[r] = [A[r] (Ca) | B[r] (Cb)] for rows rows; with gs (GnStat[samples * 32]) also the
 * GroupNorm sum/min/max of out per the reference's rule (per 256-element region, T rows per sample;
 * needs (Ca + Cb) % 32 == 0 and (T (Ca + Cb)) % 256 == 0, else "concat GN stats: shape"). */
int vgemm_concat(void* stream, const int32_t* A, int Ca, const int32_t* B, int Cb, int rows, int32_t* out, void* gs, int T);
int vgemm_upsample2(void* stream, const int32_t* X, int B, int H, int W, int C, int32_t* out);   /* k_upsample2: NHWC nearest x2 */

/* meow::k_gn_init (src/kernels.h:25, src/kernels.cu:173): sum = ss = 0, mn = INT_MAX, mx = INT_MIN for
 * `count` VgemmGnStat records, by a kernel (capture-safe). */
int vgemm_gn_init(void* stream, void* gs, int count);

/* Last error message of this thread ("" if none). */
const char* vgemm_last_error(void);
/* Library version string. */
const char* vgemm_version(void);

/* ---- attention (src/kernels.h:42-50,61,73-77). Heads of 64 values, G = B * heads groups.
 * Q/K operands: X[B, T, C] -> hi/lo planes [G * Tp x 64], e / hs / ls / tsum per (g, t) row; rows
 * t >= T hold the value 0 (hi 0, lo -128, ls -8192). V: X[B, Tk, C] -> transposed planes
 * [G * 64 x Tkp] with ev and vsum per (g, d); Tkp % 64 == 0, planes 16-byte aligned; scratch unused. */
int vgemm_quant_heads(void* stream, const int32_t* X, int B, int T, int C, int heads, int Tp, int8_t* hi, int8_t* lo, int32_t* e, int64_t* hs,
                      int64_t* ls, int64_t* tsum);
int vgemm_quant_heads_pad(void* stream, int G, int T, int Tp, int8_t* hi, int8_t* lo, int32_t* e, int64_t* hs, int64_t* ls, int64_t* tsum);
int vgemm_quant_v(void* stream, const int32_t* X, int B, int Tk, int C, int heads, int Tkp, int8_t* vthi, int8_t* vtlo, int32_t* ev, int64_t* vsum,
                  uint32_t* scratch);
/* meow::k_fused_attention (src/kernels.h:73-77, src/attn.cu:551-600): exact softmax attention of the
 * quantised operands, out[(b * Tq + q) * C + h * 64 + d] (rshr(O, 15 - ev)), rowmax[b * Tq + q] =
 * max(rowmax, |out|) when rowmax != NULL. Tqp % 64 == 0, Tkp % 64 == 0, C % 4 == 0, operands and out
 * 16-byte aligned; Lexp holds 1025 entries in [0, 2^31). vsum, gmx and gr are accepted and unused
 * (one launch keeps the row statistics on chip). */
int vgemm_fused_attention(void* stream, const int8_t* qhi, const int8_t* qlo, const int32_t* eq, const int64_t* qhs, const int64_t* qls,
                          const int8_t* khi, const int8_t* klo, const int32_t* ek, const int64_t* ksum, const int8_t* vthi, const int8_t* vtlo,
                          const int32_t* ev, const int64_t* vsum, int B, int heads, int Tq, int Tqp, int Tk, int Tkp, int causal, const int64_t* Lexp,
                          int C, int32_t* gmx, int64_t* gr, int32_t* out, uint32_t* rowmax);

#ifdef __cplusplus
}
#endif
#endif

// C ABI of libvgemm.so (include/vgemm.h): argument checks, tile/split-K selection and dispatch.
// Shape checks and messages follow the reference (src/gemm_hl.cu:344-370, src/gemm.cu:41,
// src/kernels.cu:733); a failed check returns VGEMM_ERR_ARG where the reference throws.
#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "../../include/vgemm.h"
#include "vk_common.h"
#include "attn.h"

namespace vk {
hipError_t launch_gemm_i8(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_x32(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_conv32(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_i16(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_gemm_conv16(int variant, int epi, const GemmParams& p, int batch, hipStream_t st);
int conv_halo_bm(int epi, int H, int W, int C, int stride, int Ho, int Wo);
hipError_t launch_gemm_conv16_halo(int bm, int epi, const GemmParams& p, hipStream_t st);
hipError_t launch_gemm_raw(int variant, const GemmParams& p, int batch, hipStream_t st);
hipError_t launch_raw_reduce(const int32_t* ws, int splits, long long plane, int ldw, int M, int N, int32_t* C, int ldc, hipStream_t st);
hipError_t launch_stripe(int src, int epi, const GemmParams& p, hipStream_t st);
hipError_t launch_kwave(int src, int epi, const GemmParams& p, hipStream_t st);
hipError_t launch_stripe_view(int src, int epi, const GemmParams& p, hipStream_t st);
hipError_t launch_stripe16(int src, int epi, const GemmParams& p, hipStream_t st);
hipError_t launch_view_fix(hipStream_t st, const uint32_t* vmax, const uint8_t* vexp, const uint32_t* vmask, int M, int F, int G, int8_t* hi,
                           int8_t* lo, int ld, int32_t* e);
hipError_t launch_splitk_epilogue(int epi, const GemmParams& p, hipStream_t st);
hipError_t launch_quant_rows(hipStream_t st, const int32_t* X, int M, int K, int ldx, int8_t* hi, int8_t* lo, int32_t* e, int Kp, int rows);
hipError_t launch_pixmax(hipStream_t st, const int32_t* X, int rows, int C, uint32_t* pm);
hipError_t launch_conv_e(hipStream_t st, const uint32_t* pm, int B, int H, int W, int stride, int32_t* e);
hipError_t launch_im2col3(hipStream_t st, const int32_t* X, const uint32_t* pm, int B, int H, int W, int C, int stride, int8_t* hi, int8_t* lo,
                          int32_t* e, int Kp);
hipError_t launch_epilogue(hipStream_t st, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int4* cst, const int32_t* e,
                           int32_t* Y, int ldy, const int32_t* R, GnStat* gs, int T);
hipError_t launch_epilogue_split(hipStream_t st, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int4* cst,
                                 const int32_t* e, int Cs, int32_t* Y0, int32_t* Y1, int32_t* Y2);
hipError_t launch_epilogue_geglu_q(hipStream_t st, const int32_t* Chi, const int32_t* Clo, int M, int F, int ldc, const int4* cst,
                                   const int32_t* e, const int32_t* L, int8_t* hi, int8_t* lo, int32_t* eo, int Kp);
hipError_t launch_fill_u32(hipStream_t st, uint32_t* p, size_t n, uint32_t value);
hipError_t launch_gn_fin1(hipStream_t st, GnStat* gs, int cnt, i64 n);
hipError_t launch_gn_fin2(hipStream_t st, GnStat* gs, int cnt, i64 n, i64 den);
hipError_t launch_gn_reduce(hipStream_t st, bool sq, const int32_t* X, int B, int T, int C, int groups, GnStat* gs);
hipError_t launch_gn_apply(hipStream_t st, const int32_t* X, int B, int T, int C, int groups, const GnStat* gs, const i64* g, const i64* beta, int32_t* Y);
hipError_t launch_gn_apply_row(hipStream_t st, const int32_t* X, int M, int T, int C, int groups, const GnStat* gs, const int32_t* g, const int32_t* beta,
                               const int32_t* Lsig, int32_t* Y, uint32_t* pm, int8_t* hi, int8_t* lo, int32_t* e, int Kp);
hipError_t launch_lnorm(hipStream_t st, bool q, const int32_t* X, int M, int C, const void* g, const void* beta, i64 den, int32_t* Y, int8_t* hi, int8_t* lo,
                        int32_t* e, int Kp);
hipError_t launch_gn_init(hipStream_t st, GnStat* gs, int n);
hipError_t launch_act(hipStream_t st, int32_t* X, size_t n, const int32_t* L);
hipError_t launch_geglu(hipStream_t st, int32_t* A, const int32_t* G, size_t n, const int32_t* L);
hipError_t launch_add(hipStream_t st, int32_t* X, const int32_t* Y, size_t n);
hipError_t launch_concat(hipStream_t st, const int32_t* A, int Ca, const int32_t* B, int Cb, int rows, int32_t* out, GnStat* gs, int T);
hipError_t launch_upsample2(hipStream_t st, const int32_t* X, int B, int H, int W, int C, int32_t* out);
}  // namespace vk

namespace {

thread_local std::string g_err;
int g_variant = -1;   // meow::g_gemm_hl_variant: process-wide, written by tests only
int g_splitk = 0;
std::atomic<bool> g_sws_on{true};   // split-K workspaces of calls that bring none (stream_workspace)
int g_tile_order = -1;

__attribute__((format(printf, 2, 3))) int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return VGEMM_OK;
}

int hip_status(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(VGEMM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

// the thread-local message of vgemm_last_error, for the other translation units of the library
namespace vk {
int set_error(int code, const std::string& msg) {
    g_err = msg;
    return code;
}
void clear_error() { g_err.clear(); }
}  // namespace vk

namespace {

// Byte extent a buffer load may touch; the kernels address operands with 32-bit offsets and use
// offset 2^31 as the "outside" marker, so every extent must stay below 2^31.
constexpr long long MAX_EXTENT = (1LL << 31) - 64;

struct Tiles { int BM, BN; };
// variant 3 (128 x 256, eight waves) exists for the DMA sources only; the register-staged sources
// run it as variant 0
constexpr int NVARIANT = 4;
constexpr Tiles TILES[NVARIANT] = {{128, 128}, {64, 128}, {128, 64}, {128, 256}};
constexpr int NCU = 256;   // MI355X compute units

int cdiv(long long a, long long b) { return int((a + b - 1) / b); }

// Variant 4 forces the row-stationary kernel (stripe_kernel.h) where it applies: int16 rows or int8
// planes, epilogue PLAIN (with or without a residual) / GEGLU / GELU, Kp <= 320, output columns in
// whole groups of four and 16-byte aligned output, Y extent below 2^31. Blocks of 128 rows stream
// 64-row W chunks.
constexpr int VARIANT_STRIPE = 4;
// Variant 5 forces the K-split-over-waves kernel (kwave_kernel.h) where it applies: int16 rows, int8
// planes or int16 images with C % 64 == 0, epilogue PLAIN (with or without a residual) / SPLIT3 /
// GEGLU / GELU, no GroupNorm statistics. 64 x 64 tiles, the four waves of a block splitting K.
constexpr int VARIANT_KWAVE = 5;
// Variant 6 forces the sixteen-rows-per-wave row-stationary kernel (stripe16_kernel.h) where the
// row-stationary kernel applies without a residual; variant 4 forces stripe_kernel.h.
constexpr int VARIANT_STRIPE16 = 6;
// Automatic choice between the two: the table epilogues (GEGLU, GELU) on stripe16, whose four waves
// per SIMD hide their per-output dependency chains better (C2 GEGLU 75.3 -> 73.2 us, 32768 x 320 x
// 1280 GELU 46.6 -> 44.3 us, same box); PLAIN on stripe_kernel, whose 32-row waves read each W
// fragment for twice the rows (16-row waves double the LDS reads: 32768 x 320 x 2560 PLAIN 78.9 ->
// 83.8 us on stripe16).
bool stripe16_auto(int epi) { return epi == VGEMM_EPI_GEGLU || epi == VGEMM_EPI_GELU; }
constexpr int STRIPE_BM = 128, STRIPE_CH = 64;
constexpr int STRIPE_NCOLS = 1280;   // W rows per block, at most

bool stripe_applies(int src, int epi, const vk::GemmParams& p) {
    if (src != VGEMM_SRC_I16 && src != VGEMM_SRC_I8) return false;
    if (epi != VGEMM_EPI_PLAIN && epi != VGEMM_EPI_GEGLU && epi != VGEMM_EPI_GELU) return false;
    if (p.R && epi != VGEMM_EPI_PLAIN) return false;   // the kernel adds a residual to PLAIN outputs only
    if (p.Kp > 320 || !p.vec_store) return false;
    const int nout = epi == VGEMM_EPI_GEGLU ? p.Nreal / 2 : p.Nreal;
    if (nout % 4) return false;
    // the kernel forms 32-bit byte offsets for every row of a 128-row stripe, pad rows included:
    // all of them must stay below 2^31, so that rows at or past Mreal fail the buffer range check
    // instead of wrapping back into Y
    const long long rows = (long long)cdiv(p.Mreal, STRIPE_BM) * STRIPE_BM;
    const long long yext = ((rows - 1) * p.ldy + nout) * 4;
    return yext <= MAX_EXTENT;
}

bool kwave_applies(int src, int epi, const vk::GemmParams& p) {
    if (src != VGEMM_SRC_I16 && src != VGEMM_SRC_I8 && !(src == VGEMM_SRC_CONV16 && p.C % 64 == 0)) return false;
    if (epi != VGEMM_EPI_PLAIN && epi != VGEMM_EPI_SPLIT3 && epi != VGEMM_EPI_GEGLU && epi != VGEMM_EPI_GELU) return false;
    return !p.gnstat;
}

// Automatic use, for unsplit calls only: at most 640 rows and 1280 columns over Kp >= 1024 (measured:
// the 512-row 3x3 convolutions of 1280 channels 99 -> 65 us and 191 -> 115 us without a workspace,
// 512 x 1280 x 2560 linears 23.3 -> 21.0 us; wider or taller shapes stay on the tiled kernels), or,
// for row sources (p.C == 0: the sweep behind this measured linears only), at most 1024 rows and
// 1280 columns over Kp >= 768 with a grid of at most one 64x64 block per CU (768 x 1280 x 1280
// 13.1 -> 12.6 us, 616 x 768 x 1280 9.8 -> 9.4; grids of 320 blocks and more are up to 1.8x slower
// there: 1024 x 1280 x 1280 23.3 against 13.3 us).
bool kwave_auto(const vk::GemmParams& p) {
    if (p.Mreal <= 640 && p.Nreal <= 1280 && p.Kp >= 1024) return true;
    return p.C == 0 && p.Mreal <= 1024 && p.Nreal <= 1280 && p.Kp >= 768 &&
           (long long)cdiv(p.Mreal, 64) * cdiv(p.Nreal, 64) <= NCU;
}

// Blocks = row stripes x column ranges: as few column ranges as the table allows, raised until
// there are two blocks per CU. Returns the column ranges and the chunks of each.
void stripe_ranges(const vk::GemmParams& p, int& cs, int& kper) {
    const int nch = cdiv(p.Nreal, STRIPE_CH);
    const int mt = cdiv(p.Mreal, STRIPE_BM);
    cs = std::max(cdiv(nch, STRIPE_NCOLS / STRIPE_CH), std::min(nch, cdiv(2 * NCU, mt)));
    kper = cdiv(nch, cs);
    cs = cdiv(nch, kper);
}

// Automatic use, with no per-row shifts (rows with e != 0 leave the kernels' integer epilogue for
// their slow int64 form; the tile kernels cover them):
//  * many rows (a block keeps its rows in registers and streams its columns, so the kernels need a
//    few hundred row stripes to fill the GPU); residual calls qualify, the kernel loading a batch's
//    residuals ahead of its arithmetic (UNet 32768 x 320 x 320 residual layers: 23.1 us against
//    28.0 us on the tile kernels);
//  * or a grid of at most one block per CU (few rows: each block then one or a few chunks), where
//    the row-stationary set-up is shorter than the tile kernels' (C1 4096 x 320 x 320 7.40 -> 7.14 us,
//    1024..2048 x 320 x 320..1280 4 % faster; grids of 320 blocks stay on the tile kernels, which are
//    faster there: 4096 x 320 x 640 8.8 against 10.5 us);
//  * or, from 1024 rows, a 64x128 tile grid of at least 3.75 tiles per CU (960), where the tile
//    kernels run several rounds of short blocks while the row-stationary kernels stream the columns
//    through resident blocks (8192 x 320 x 2560 PLAIN 31.0 -> 21.4 us, 4096 x 320 x 2560 GEGLU
//    20.0 -> 16.0, 8192 x 160 x 1280 PLAIN 18.1 -> 13.2, with a residual 8192 x 320 x 1280
//    29.4 -> 21.1, 960 tiles 4-16 % faster; at 640 and 768 tiles the tile kernels stay ahead,
//    4096 x 320 x 1280 PLAIN 11.2 against 12.1 us).
bool stripe_auto(const vk::GemmParams& p) {
    if (p.e) return false;
    if (cdiv(p.Mreal, STRIPE_BM) >= 2 * NCU / 4 && p.Mreal >= 16384) return true;
    if (p.Mreal >= 1024 && (long long)cdiv(p.Mreal, 64) * cdiv(p.Nreal, 128) >= 15LL * NCU / 4) return true;
    int cs, kper;
    stripe_ranges(p, cs, kper);
    return (long long)cdiv(p.Mreal, STRIPE_BM) * cs <= NCU;
}

constexpr int STRIPE_PRIO_PCT = 55;
void stripe_grid(vk::GemmParams& p) {
    const int mt = cdiv(p.Mreal, STRIPE_BM);
    int cs, kper;
    stripe_ranges(p, cs, kper);
    p.mtiles = mt;
    p.ntiles = cs;
    p.kper = kper;
    p.ksplit = 1;
    // With NCU < blocks <= 2 NCU every block is resident from the start, the first NCU one per CU;
    // on each CU the older block keeps issue priority (oldest wave first) until it ends, and the
    // younger then runs alone. The younger blocks (index >= NCU) raise their priority for their first
    // STRIPE_PRIO_PCT % of chunks, so that the two blocks of a CU end closer together.
    const int nblk = mt * cs;
    p.young0 = nblk > NCU && nblk <= 2 * NCU ? NCU : 0;
    p.prio_chunks = (kper * STRIPE_PRIO_PCT + 50) / 100;
}

// Tile variant and split-K, from measurements over the BASELINE and UNet shapes on MI355X:
//  * 64x128 tiles (three blocks per CU) are fastest for most shapes;
//  * 128x128 tiles win for wide, shallow GEMMs (N >= 960, K <= 1280) with plenty of tiles, where the
//    epilogue dominates and the larger tile halves its fixed per-tile cost;
//  * deep K with few tiles splits K so that all tiles' splits fill one round of blocks (two per CU
//    for 128x128, three for 64x128) with at least 16 K steps per split: few rows (at most 192
//    64x128 tiles, three quarters of the CUs, K >= 4096) run 64x128 tiles in up to six splits (the
//    stride-2 2048x5760x640 conv, 160 tiles: 49.3 -> 35.0 us in three splits), fewer than 256
//    128x128 tiles with K >= 8192 run 128x128 tiles; the int32 partials are reduced in a second pass.
enum SplitRule { SPLIT_NONE, SPLIT_SMALL, SPLIT_DEEP };

SplitRule split_rule(int M, int N, int Kp) {
    const long long tiles0 = (long long)cdiv(M, TILES[0].BM) * cdiv(N, TILES[0].BN);
    const long long tiles1 = (long long)cdiv(M, TILES[1].BM) * cdiv(N, TILES[1].BN);
    if (Kp >= 4096 && tiles1 <= 3 * NCU / 4) return SPLIT_SMALL;
    if (Kp >= 8192 && tiles0 < NCU) return SPLIT_DEEP;
    return SPLIT_NONE;
}

int pick_variant(int M, int N, int Kp) {
    switch (split_rule(M, N, Kp)) {
    case SPLIT_SMALL: return 1;
    case SPLIT_DEEP: return 0;
    default: break;
    }
    const long long tiles1 = (long long)cdiv(M, TILES[1].BM) * cdiv(N, TILES[1].BN);
    if (N >= 960 && Kp <= 1280 && tiles1 > 3LL * NCU) return 0;
    return 1;
}

// Tile of the single-plane int8 GEMM (Gemm::run). It has half the MFMA work per K step of the fused
// two-plane kernel, so deep K wants the 128 x 128 tiles while they give every CU a block, else the
// 128 x 64 ones (one MI355X, 200 launches each: the stacked planes of C3 [16384 x 5760] x 640 112.6 ->
// 84.2 us, of the 2048-row C4 conv [4096 x 11520] x 1280 120.8 -> 79.6 us, of the 512-row one
// [1024 x 11520] x 1280 69.1 -> 52.2 us, [4096 x 1280] x 1280 19.4 -> 17.0 us); shallow K keeps the
// fused kernel's choice.
int pick_variant_raw(int M, int N, int K) {
    if (K < 1024) return pick_variant(M, N, K);
    const long long tiles0 = (long long)cdiv(M, TILES[0].BM) * cdiv(N, TILES[0].BN);
    return tiles0 >= NCU ? 0 : 2;
}

int pick_splitk(int variant, int M, int N, int Kp) {
    const int nK = (Kp + 63) / 64;
    if (g_splitk > 0) return g_splitk < nK ? g_splitk : nK;
    const SplitRule rule = split_rule(M, N, Kp);
    if (rule == SPLIT_NONE) return 1;
    const long long tiles = (long long)cdiv(M, TILES[variant].BM) * cdiv(N, TILES[variant].BN);
    long long s = 2LL * NCU / tiles;   // one round of blocks
    if (rule == SPLIT_SMALL && s > 6) s = 6;
    if (s > nK / 16) s = nK / 16;
    return s < 1 ? 1 : int(s);
}

// Tile order over the XCDs (vk::tile_index), from the bytes each order fetches from beyond the L2s:
// row order reads A once and all of W in every XCD that owns row stripes; column order, with at
// least one (K range, column tile) group per XCD, reads W once and in every XCD the A columns of the
// one or two K ranges it covers (about 1/8 + 1/ksplit of A). Column order is taken only when it
// saves a quarter of the estimate; W-heavy shapes (deep 3x3 convolutions on small images, wide
// GEGLU projections of few rows) are the ones that gain.
double a_operand_bytes(const VgemmASrc* A, const vk::GemmParams& p) {
    switch (A->src) {
    case VGEMM_SRC_I8: return 2.0 * p.Mreal * p.Kp;
    case VGEMM_SRC_I16: return 2.0 * p.Mreal * p.Kp;
    case VGEMM_SRC_X32: return 4.0 * p.Mreal * p.K;
    case VGEMM_SRC_CONV32:
    case VGEMM_SRC_CONV16: {
        const double pix = double(p.Mreal) / (double(p.Ho) * p.Wo) * p.H * p.W;
        return (A->src == VGEMM_SRC_CONV32 ? 4.0 : 2.0) * pix * p.C;
    }
    }
    return 0.0;
}

int pick_tile_order(const vk::GemmParams& p, double a_bytes) {
    if (g_tile_order >= 0) return g_tile_order;
    if ((long long)p.ntiles * p.ksplit < 8) return 0;
    const double w_bytes = double(p.Nreal) * p.Kp;
    const double row = a_bytes + w_bytes * std::min(8, p.mtiles);
    const double col = w_bytes + a_bytes * std::min(8.0, 1.0 + 8.0 / p.ksplit);
    return col < 0.75 * row ? 1 : 0;
}

// Workspace of the int16 view: row maxima [M], masks [G x M] and exponent bytes [G x M], G = the
// output's 32-column groups, each part 256-byte aligned.
struct ViewWs { size_t max_off, mask_off, exp_off, bytes; };
ViewWs view_ws(int M, int nout) {
    const size_t G = size_t(cdiv(nout, 32));
    auto a256 = [](size_t v) { return (v + 255) / 256 * 256; };
    ViewWs w;
    w.max_off = 0;
    w.mask_off = a256(size_t(M) * 4);
    w.exp_off = w.mask_off + a256(size_t(M) * G * 4);
    w.bytes = w.exp_off + a256(size_t(M) * G);
    return w;
}

// Deeper K (the tile kernels): the GEMM's int32 output rows [M x align4(nout)] in the workspace, then
// k_quant_rows' quantisation of them into the view; the GEMM's split-K workspace follows.
constexpr int VIEW_FUSED_KP = 320;
struct ViewWs2 { int ld; size_t bytes; };
ViewWs2 view_ws2(int M, int nout) {
    ViewWs2 w;
    w.ld = (nout + 3) / 4 * 4;
    w.bytes = (size_t(M) * w.ld * 4 + 255) / 256 * 256;
    return w;
}

size_t ws_bytes_for(int variant, int M, int N, int splits) {
    if (splits <= 1) return 0;
    const size_t rows = size_t(cdiv(M, TILES[variant].BM)) * TILES[variant].BM;
    const size_t cols = size_t(cdiv(N, TILES[variant].BN)) * TILES[variant].BN;
    return size_t(splits) * 2 * rows * cols * 4;
}

// The tile the reference's fused GEMM runs for these padded sizes (src/gemm_hl.cu:352-358, automatic
// choice), which is the region its GroupNorm statistics are gathered and flushed over: for
// Kp >= 2048, 64 x 128 when Np % 128 == 0, else 128 x 64 when Mp % 128 == 0 and the A operand is int8
// planes (the int16 rows hold the same planes), else 64 x 64.
Tiles gn_ref_tile(int Mp, int Np, int Kp, int src) {
    int v = 0;
    if (Kp >= 2048) v = Np % 128 == 0 ? 2 : (Mp % 128 == 0 ? 1 : 0);
    const bool planes = src == VGEMM_SRC_I8 || src == VGEMM_SRC_I16;
    if (v == 1 && !planes) v = 0;
    return Tiles{v == 1 ? 128 : 64, v == 2 ? 128 : 64};
}

int launch_src(int src, int variant, int epi, const vk::GemmParams& p, hipStream_t st) {
    hipError_t e;
    switch (src) {
    case VGEMM_SRC_I8: e = vk::launch_gemm_i8(variant, epi, p, 1, st); break;
    case VGEMM_SRC_X32: e = vk::launch_gemm_x32(variant, epi, p, 1, st); break;
    case VGEMM_SRC_CONV32: e = vk::launch_gemm_conv32(variant, epi, p, 1, st); break;
    case VGEMM_SRC_I16: e = vk::launch_gemm_i16(variant, epi, p, 1, st); break;
    case VGEMM_SRC_CONV16: e = vk::launch_gemm_conv16(variant, epi, p, 1, st); break;
    default: return fail(VGEMM_ERR_ARG, "gemm_hl: unknown A source %d", src);
    }
    return hip_status(e, "gemm_hl launch");
}

}  // namespace

extern "C" {

void vgemm_asrc_init(VgemmASrc* a) {
    std::memset(a, 0, sizeof *a);
    a->src = VGEMM_SRC_I8;
    a->stride = 1;
}

void vgemm_aepi_init(VgemmAEpi* e) {
    std::memset(e, 0, sizeof *e);
    e->epi = VGEMM_EPI_PLAIN;
}

int vgemm_supported(int Mp, int Np, int Kp) { return Mp > 0 && Np > 0 && Kp > 0 && Mp % 64 == 0 && Np % 64 == 0 && Kp % 16 == 0; }

void vgemm_set_variant(int v) { g_variant = v; }
int vgemm_get_variant(void) { return g_variant; }
void vgemm_set_splitk(int s) { g_splitk = s < 0 ? 0 : s; }
void vgemm_set_stream_workspaces(int on) { g_sws_on.store(on != 0, std::memory_order_relaxed); }
void vgemm_set_tile_order(int order) { g_tile_order = order < 0 ? -1 : (order ? 1 : 0); }

int vgemm_conv16_halo_rows(int H, int W, int C, int stride, int epi) {
    if (H <= 0 || W <= 0 || C <= 0 || stride <= 0) return 0;
    return vk::conv_halo_bm(epi, H, W, C, stride, (H - 1) / stride + 1, (W - 1) / stride + 1);
}

size_t vgemm_view_workspace_bytes(int Mreal, int Nreal, int Kp, int epi) {
    if (Mreal <= 0 || Nreal <= 0 || Kp <= 0) return 0;
    const int nout = epi == VGEMM_EPI_GEGLU ? Nreal / 2 : Nreal;
    if (Kp <= VIEW_FUSED_KP) return view_ws(Mreal, nout).bytes;
    return view_ws2(Mreal, nout).bytes + vgemm_workspace_bytes(Mreal, Mreal, Nreal, Nreal, Kp, epi);
}

size_t vgemm_workspace_bytes(int Mp, int Mreal, int Np, int Nreal, int Kp, int epi) {
    (void)Mp; (void)Np; (void)epi;
    if (g_variant >= 0 && g_variant < NVARIANT) return ws_bytes_for(g_variant, Mreal, Nreal, pick_splitk(g_variant, Mreal, Nreal, Kp));
    // the automatic choice, or the 128- or 64-row tiles of the halo convolution kernel
    size_t nb = 0;
    for (int v : {pick_variant(Mreal, Nreal, Kp), 0, 1}) nb = std::max(nb, ws_bytes_for(v, Mreal, Nreal, pick_splitk(v, Mreal, Nreal, Kp)));
    return nb;
}

}  // extern "C"

namespace {

// Where the split-K partials of a call go: the caller's workspace (AEpi.ws; a call whose split would
// not fit runs unsplit), the library's static scratch (vgemm_hl2_noalloc: the call is rejected if its
// split would not fit), or, for a call that brings none, its stream's workspace (below).
struct WsPolicy {
    void* ws;
    size_t bytes;
    bool strict;
};

// Split-K workspaces of calls that bring none. The reference's AEpi has no workspace, so its callers
// never pass one; such a call whose shape wants a K split (deep K over fewer tiles than CUs) takes a
// workspace that the library allocates for its (device, stream) on the first such call made outside
// stream capture (the reference engine runs its forward eagerly once before it captures it). When a
// later call needs more, a larger one replaces it for new calls; none is ever freed before the
// process ends, since a graph captured earlier may still refer to it. Calls on one stream run in
// order, so they never use it at the same time; calls on other streams have their own (a graph
// captured with such calls uses its capture stream's workspace, so it is replayed on that stream, as
// the reference replays its forward). Under capture with no workspace yet, or with the workspaces
// turned off (vgemm_set_stream_workspaces(0)), the call runs unsplit.
struct StreamWs {
    void* p = nullptr;
    size_t bytes = 0;
};
std::mutex g_sws_mu;
std::map<std::pair<int, uintptr_t>, StreamWs> g_sws;

void* stream_workspace(hipStream_t st, size_t need, size_t* bytes) {
    if (!g_sws_on.load(std::memory_order_relaxed)) return nullptr;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_sws_mu);
    StreamWs& w = g_sws[{dev, reinterpret_cast<uintptr_t>(st)}];
    if (w.p && w.bytes >= need) {
        *bytes = w.bytes;
        return w.p;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    const size_t grain = size_t(4) << 20;
    const size_t sz = (need + grain - 1) / grain * grain;
    void* np = nullptr;
    if (hipMalloc(&np, sz) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    w.p = np;   // a smaller one it replaces stays allocated (graphs may refer to it)
    w.bytes = sz;
    *bytes = sz;
    return w.p;
}

// The int16 view of the output (vgemm_hl2_view): the row-stationary kernel writes each chunk at its
// running row exponent with correction bits and row maxima in the workspace, then the fix-up pass
// settles every row at its final exponent (stripe_kernel.h, producers.hip: view_fix_kernel).
int hl2_impl(void* stream, const VgemmASrc* A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal, int Kp,
             const int32_t* cst, const VgemmAEpi* E, WsPolicy wsp, const VgemmView* V = nullptr);

int view_impl(void* stream, const VgemmASrc* A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal, int Kp, const int32_t* cst,
              const VgemmAEpi* E, const VgemmView* V, vk::GemmParams& p, const WsPolicy& wsp) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int epi = E->epi;
    if (epi != VGEMM_EPI_PLAIN && epi != VGEMM_EPI_GEGLU && epi != VGEMM_EPI_GELU)
        return fail(VGEMM_ERR_ARG, "gemm_hl int16 view: EPI_PLAIN, EPI_GEGLU or EPI_GELU only");
    if (E->residual || E->rowmax || E->gnstat) return fail(VGEMM_ERR_ARG, "gemm_hl int16 view: no residual, rowmax or statistics");
    if (A->src != VGEMM_SRC_I16 && A->src != VGEMM_SRC_I8) return fail(VGEMM_ERR_UNSUPPORTED, "gemm_hl int16 view: int16 rows or int8 planes only");
    if (epi == VGEMM_EPI_GEGLU && Nreal % 2) return fail(VGEMM_ERR_ARG, "gemm_hl: EPI_GEGLU needs an even Nreal (interleaved a/g columns)");
    if (epi != VGEMM_EPI_PLAIN && !E->Lphi) return fail(VGEMM_ERR_ARG, "gemm_hl: EPI_GEGLU/EPI_GELU need Lphi");
    const int nout = epi == VGEMM_EPI_GEGLU ? Nreal / 2 : Nreal;
    if (nout % 4 || !V->hi || !V->lo || !V->e || V->ld < nout || V->ld % 16 || !aligned16(V->hi) || !aligned16(V->lo))
        return fail(VGEMM_ERR_ARG, "gemm_hl int16 view: output columns %% 4 == 0, hi/lo 16-byte aligned, ld >= output columns, ld %% 16 == 0, and e");
    if ((long long)Mreal * V->ld > MAX_EXTENT) return fail(VGEMM_ERR_UNSUPPORTED, "gemm_hl int16 view: planes larger than 2 GiB");
    if (Kp > VIEW_FUSED_KP) {
        // the GEMM's int32 rows into the workspace (the tile kernels, split-K in the workspace's
        // tail), then their quantisation (k_quant_rows, Mreal rows)
        const ViewWs2 vw = view_ws2(Mreal, nout);
        const size_t need = vgemm_view_workspace_bytes(Mreal, Nreal, Kp, epi);
        if (!wsp.ws || wsp.bytes < need)
            return fail(wsp.strict ? VGEMM_ERR_UNSUPPORTED : VGEMM_ERR_ARG, "gemm_hl int16 view: needs a workspace of %zu bytes (AEpi.ws)", need);
        if (!aligned16(wsp.ws)) return fail(VGEMM_ERR_ARG, "gemm_hl: workspace must be 16-byte aligned");
        int32_t* Yw = static_cast<int32_t*>(wsp.ws);
        VgemmAEpi E2 = *E;
        E2.Y = Yw;
        E2.ldy = vw.ld;
        E2.ws_bytes = wsp.bytes - vw.bytes;
        E2.ws = E2.ws_bytes ? static_cast<char*>(wsp.ws) + vw.bytes : nullptr;
        const int rc = hl2_impl(stream, A, Mp, Mreal, W, ldw, Np, Nreal, Kp, cst, &E2, WsPolicy{E2.ws, E2.ws_bytes, wsp.strict});
        if (rc) return rc;
        return hip_status(vk::launch_quant_rows(st, Yw, Mreal, nout, vw.ld, V->hi, V->lo, V->e, V->ld, Mreal), "gemm_hl int16 view: quantisation");
    }
    const ViewWs vw = view_ws(Mreal, nout);
    if (!wsp.ws || wsp.bytes < vw.bytes)
        return fail(wsp.strict ? VGEMM_ERR_UNSUPPORTED : VGEMM_ERR_ARG, "gemm_hl int16 view: needs a workspace of %zu bytes (AEpi.ws)", vw.bytes);
    if (!aligned16(wsp.ws)) return fail(VGEMM_ERR_ARG, "gemm_hl: workspace must be 16-byte aligned");
    char* ws = static_cast<char*>(wsp.ws);
    p.vhi = V->hi; p.vlo = V->lo; p.vld = V->ld;
    p.v_bytes = unsigned((long long)Mreal * V->ld);
    p.vgroups = cdiv(nout, 32);
    p.vmax = reinterpret_cast<uint32_t*>(ws + vw.max_off);
    p.vmask = reinterpret_cast<uint32_t*>(ws + vw.mask_off);
    p.vexp = reinterpret_cast<uint8_t*>(ws + vw.exp_off);
    p.Y = nullptr; p.y_bytes = 0; p.R = nullptr; p.rowmax = nullptr;
    stripe_grid(p);
    int rc = hip_status(vk::launch_fill_u32(st, p.vmax, size_t(Mreal), 0u), "gemm_hl int16 view: row maxima clear");
    if (rc) return rc;
    rc = hip_status(vk::launch_stripe_view(A->src, epi, p, st), "gemm_hl int16 view launch");
    if (rc) return rc;
    return hip_status(vk::launch_view_fix(st, p.vmax, p.vexp, p.vmask, Mreal, nout, p.vgroups, V->hi, V->lo, V->ld, V->e),
                      "gemm_hl int16 view fix-up");
}

int hl2_impl(void* stream, const VgemmASrc* A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal, int Kp,
             const int32_t* cst, const VgemmAEpi* E, WsPolicy wsp, const VgemmView* V) {
    if (!A || !E) return fail(VGEMM_ERR_ARG, "gemm_hl: null ASrc/AEpi");
    // The fields an epilogue does not read are ignored, as the reference's epilogue ignores them
    // (src/gemm_hl.cu:176-177, 279-296): the GroupNorm statistics outside EPI_PLAIN, the residual
    // outside EPI_PLAIN / EPI_GELU, the row maxima on EPI_SPLIT3 and EPI_QKV.
    VgemmAEpi Eu = *E;
    if (Eu.epi != VGEMM_EPI_PLAIN) Eu.gnstat = nullptr;
    if (Eu.epi == VGEMM_EPI_GEGLU || Eu.epi == VGEMM_EPI_SPLIT3 || Eu.epi == VGEMM_EPI_QKV) Eu.residual = nullptr;
    if (Eu.epi == VGEMM_EPI_SPLIT3 || Eu.epi == VGEMM_EPI_QKV) Eu.rowmax = nullptr;
    E = &Eu;
    if (!vgemm_supported(Mp, Np, Kp)) return fail(VGEMM_ERR_ARG, "gemm_hl: unsupported shape (Mp %d, Np %d, Kp %d)", Mp, Np, Kp);
    if (Mreal < 0 || Mreal > Mp || Nreal < 0 || Nreal > Np) return fail(VGEMM_ERR_ARG, "gemm_hl: Mreal/Nreal outside Mp/Np");
    if (!W || !cst || ldw < Kp || ldw % 16 || !aligned16(W)) return fail(VGEMM_ERR_ARG, "gemm_hl: W must be 16-byte aligned with ldw >= Kp, ldw %% 16 == 0");
    if (E->epi < 0 || E->epi > VGEMM_EPI_QKV) return fail(VGEMM_ERR_ARG, "gemm_hl: unknown epilogue %d", E->epi);
    if (E->epi != VGEMM_EPI_QKV && !E->Y && !V) return fail(VGEMM_ERR_ARG, "gemm_hl: null Y");
    // GroupNorm statistics (src/gemm_hl.h:22, src/engine.h:110): EPI_PLAIN, 32 groups of whole
    // columns, a block's rows in at most two samples
    if (E->gnstat && (Nreal % 32 || E->gnT <= 0 || E->gnT % 64))
        return fail(VGEMM_ERR_ARG, "gemm_hl: GroupNorm statistics need Nreal %% 32 == 0 and gnT %% 64 == 0");
    if (E->epi == VGEMM_EPI_QKV) {
        // src/engine.cu:318-326: N = 3C, C = 64 heads, rows = B*T, Tp >= T
        if (E->heads <= 0 || E->C != 64 * E->heads || Nreal != 3 * E->C || E->T <= 0 || E->TpQ < E->T || E->TpK < E->T)
            return fail(VGEMM_ERR_ARG, "gemm_hl: EPI_QKV needs C = 64*heads, Nreal = 3C, T > 0, TpQ >= T, TpK >= T");
        const void* ptrs[] = {E->Y2, E->qhi, E->qlo, E->khi, E->klo, E->qe, E->ke, E->qhs, E->qls, E->qts, E->khs, E->kls, E->kts};
        for (const void* q : ptrs)
            if (!q) return fail(VGEMM_ERR_ARG, "gemm_hl: EPI_QKV needs Y2 and every q/k output");
        if (!aligned16(E->Y2) || ((uintptr_t)E->qhi | (uintptr_t)E->qlo | (uintptr_t)E->khi | (uintptr_t)E->klo) & 3)
            return fail(VGEMM_ERR_ARG, "gemm_hl: EPI_QKV needs a 16-byte aligned Y2 and 4-byte aligned hi/lo planes");
    }
    if (Mreal == 0 || Nreal == 0) return ok();

    vk::GemmParams p;
    std::memset(&p, 0, sizeof p);
    p.Mreal = Mreal; p.Nreal = Nreal; p.Kp = Kp;
    p.w = W; p.ldw = ldw; p.cst = reinterpret_cast<const int4*>(cst);
    const long long wext = (long long)(Nreal - 1) * ldw + Kp;
    if (wext > MAX_EXTENT) return fail(VGEMM_ERR_UNSUPPORTED, "gemm_hl: W larger than 2 GiB");
    p.w_bytes = unsigned(wext);
    p.e = A->e;
    p.stride = 1;

    long long aext = 0;
    switch (A->src) {
    case VGEMM_SRC_I8:
        if (!A->hi || !A->lo || A->ld8 < Kp || A->ld8 % 16 || !aligned16(A->hi) || !aligned16(A->lo))
            return fail(VGEMM_ERR_ARG, "gemm_hl: SRC_I8 planes must be 16-byte aligned with ld8 >= Kp, ld8 %% 16 == 0");
        p.a0 = A->hi; p.a1 = A->lo; p.lda = A->ld8;
        aext = (long long)(Mreal - 1) * A->ld8 + Kp;
        p.a1_bytes = unsigned(aext > MAX_EXTENT ? 0 : aext);
        break;
    case VGEMM_SRC_I16:
        if (!A->q16 || A->K <= 0 || A->K > Kp || A->K % 8 || A->ld16 < A->K || A->ld16 % 8 || !aligned16(A->q16))
            return fail(VGEMM_ERR_ARG, "gemm_hl: SRC_I16 needs K %% 8 == 0, K <= Kp, ld16 >= K, ld16 %% 8 == 0, 16-byte alignment");
        p.a0 = A->q16; p.lda = A->ld16; p.K = A->K;
        aext = ((long long)(Mreal - 1) * A->ld16 + A->K) * 2;
        break;
    case VGEMM_SRC_X32:
        if (!A->x || !A->rowmax || A->K <= 0 || A->K > Kp || A->K % 4 || A->ldx < A->K || A->ldx % 4 || !aligned16(A->x))
            return fail(VGEMM_ERR_ARG, "gemm_hl: SRC_X32 needs x, rowmax, K %% 4 == 0, K <= Kp, ldx >= K, ldx %% 4 == 0, 16-byte alignment");
        p.a0 = A->x; p.lda = A->ldx; p.K = A->K; p.xrowmax = A->rowmax; p.e = nullptr;
        aext = ((long long)(Mreal - 1) * A->ldx + A->K) * 4;
        break;
    case VGEMM_SRC_CONV32:
    case VGEMM_SRC_CONV16: {
        const void* img = A->src == VGEMM_SRC_CONV32 ? static_cast<const void*>(A->img) : static_cast<const void*>(A->img16);
        if (!img || !aligned16(img)) return fail(VGEMM_ERR_ARG, "gemm_hl conv source: null or unaligned image");
        if (A->src == VGEMM_SRC_CONV32 && (A->C <= 0 || A->C % 16 || A->K != 9 * A->C)) return fail(VGEMM_ERR_ARG, "gemm_hl conv source: C %% 16 or K");
        if (A->src == VGEMM_SRC_CONV16 && (A->C <= 0 || A->C % 8 || A->C > 16384 || A->K != 9 * A->C))
            return fail(VGEMM_ERR_ARG, "gemm_hl conv source: C %% 8, C <= 16384 and K == 9C required for SRC_CONV16");
        if (A->K > Kp || A->H <= 0 || A->W <= 0 || A->stride <= 0) return fail(VGEMM_ERR_ARG, "gemm_hl conv source: H/W/stride/Kp");
        const int Ho = (A->H - 1) / A->stride + 1, Wo = (A->W - 1) / A->stride + 1;
        if (A->Ho != Ho || A->Wo != Wo) return fail(VGEMM_ERR_ARG, "gemm_hl conv source: Ho/Wo must be (H-1)/stride+1, (W-1)/stride+1");
        const long long B = (Mreal + (long long)Ho * Wo - 1) / ((long long)Ho * Wo);
        p.a0 = img; p.K = A->K; p.H = A->H; p.W = A->W; p.C = A->C; p.stride = A->stride; p.Ho = Ho; p.Wo = Wo;
        // without an e vector, rowmax holds the image's per-pixel maxima and the kernels derive e
        p.pm = A->e ? nullptr : A->rowmax;
        aext = B * A->H * A->W * (long long)A->C * (A->src == VGEMM_SRC_CONV32 ? 4 : 2);
        break;
    }
    default:
        return fail(VGEMM_ERR_ARG, "gemm_hl: unknown A source %d", A->src);
    }
    if (aext > MAX_EXTENT) return fail(VGEMM_ERR_UNSUPPORTED, "gemm_hl: A operand larger than 2 GiB");
    p.a0_bytes = unsigned(aext);

    const int epi = E->epi;
    p.Y = E->Y; p.ldy = E->ldy; p.R = E->residual; p.Lphi = E->Lphi; p.rowmax = E->rowmax;
    if (V) return view_impl(stream, A, Mp, Mreal, W, ldw, Np, Nreal, Kp, cst, E, V, p, wsp);
    p.Cs = E->Cs; p.Y1 = E->Y1; p.Y2 = E->Y2;
    p.gnstat = static_cast<vk::GnStat*>(E->gnstat); p.gnT = E->gnT;
    p.heads = E->heads; p.qT = E->T; p.TpQ = E->TpQ; p.TpK = E->TpK; p.qC = E->C;
    p.qhi = E->qhi; p.qlo = E->qlo; p.khi = E->khi; p.klo = E->klo; p.qe = E->qe; p.ke = E->ke;
    p.qhs = reinterpret_cast<long long*>(E->qhs); p.qls = reinterpret_cast<long long*>(E->qls); p.qts = reinterpret_cast<long long*>(E->qts);
    p.khs = reinterpret_cast<long long*>(E->khs); p.kls = reinterpret_cast<long long*>(E->kls); p.kts = reinterpret_cast<long long*>(E->kts);
    bool vec = aligned16(E->Y);
    switch (epi) {
    case VGEMM_EPI_PLAIN:
    case VGEMM_EPI_GELU:
        if (E->ldy < Nreal) return fail(VGEMM_ERR_ARG, "gemm_hl: ldy < Nreal");
        if (epi == VGEMM_EPI_GELU && !E->Lphi) return fail(VGEMM_ERR_ARG, "gemm_hl: EPI_GELU needs Lphi");
        vec = vec && E->ldy % 4 == 0 && (!E->residual || aligned16(E->residual));
        break;
    case VGEMM_EPI_GEGLU:
        if (Nreal % 2) return fail(VGEMM_ERR_ARG, "gemm_hl: EPI_GEGLU needs an even Nreal (interleaved a/g columns)");
        if (!E->Lphi) return fail(VGEMM_ERR_ARG, "gemm_hl: EPI_GEGLU needs Lphi");
        if (E->ldy < Nreal / 2) return fail(VGEMM_ERR_ARG, "gemm_hl: ldy < Nreal/2");
        vec = vec && E->ldy % 4 == 0;
        break;
    case VGEMM_EPI_SPLIT3:
        if (E->Cs <= 0 || E->Cs % 4 || Nreal > 3 * E->Cs) return fail(VGEMM_ERR_ARG, "gemm_hl: EPI_SPLIT3 needs Cs %% 4 == 0 and Nreal <= 3*Cs");
        if ((Nreal > E->Cs && !E->Y1) || (Nreal > 2 * E->Cs && !E->Y2)) return fail(VGEMM_ERR_ARG, "gemm_hl: EPI_SPLIT3 needs Y1/Y2");
        vec = vec && (!E->Y1 || aligned16(E->Y1)) && (!E->Y2 || aligned16(E->Y2));
        break;
    case VGEMM_EPI_QKV:
        vec = true;
        break;
    }
    p.vec_store = vec ? 1 : 0;
    hipStream_t st = static_cast<hipStream_t>(stream);

    // shallow GEMMs with many rows: the row-stationary kernel (forced by variant 4 where it applies)
    if (stripe_applies(A->src, epi, p) && !p.gnstat &&
        (g_variant == VARIANT_STRIPE || g_variant == VARIANT_STRIPE16 || (g_variant < 0 && stripe_auto(p)))) {
        const int nout = epi == VGEMM_EPI_GEGLU ? Nreal / 2 : Nreal;
        p.y_bytes = unsigned(((long long)(Mreal - 1) * E->ldy + nout) * 4);
        stripe_grid(p);
        const bool s16 = !p.R && (g_variant == VARIANT_STRIPE16 || (g_variant < 0 && stripe16_auto(epi)));
        if (s16) return hip_status(vk::launch_stripe16(A->src, epi, p, st), "gemm_hl stripe launch");
        return hip_status(vk::launch_stripe(A->src, epi, p, st), "gemm_hl stripe launch");
    }

    // stride-1 3x3 convolutions of int16 images with C % 64 == 0 run the halo-reuse kernel unless a
    // tile variant is forced; its K steps are 64-channel chunks (each covering all nine taps)
    int halo_bm = A->src == VGEMM_SRC_CONV16 && g_variant < 0 ? vk::conv_halo_bm(epi, p.H, p.W, p.C, p.stride, p.Ho, p.Wo) : 0;
    if (halo_bm) {
        // a halo grid that stays below one block per CU (no K split) against a tile grid that fills
        // the chip: the tile kernel (measured: 2048 x 5760 x 1280, C = 640 at 16 x 16, 72 -> 54 us)
        const int hv = halo_bm == 128 ? 0 : 1;
        const long long htiles = (long long)cdiv(Mreal, TILES[hv].BM) * cdiv(Nreal, TILES[hv].BN);
        const int hsplits = (wsp.ws || g_sws_on) && epi != VGEMM_EPI_QKV && !E->gnstat ? pick_splitk(hv, Mreal, Nreal, Kp) : 1;
        const long long tiles1 = (long long)cdiv(Mreal, TILES[1].BM) * cdiv(Nreal, TILES[1].BN);
        if (htiles * hsplits < NCU && tiles1 >= NCU) halo_bm = 0;
    }
    int variant = halo_bm ? (halo_bm == 128 ? 0 : 1) : g_variant >= 0 && g_variant < NVARIANT ? g_variant : pick_variant(Mreal, Nreal, Kp);
    if (variant >= 3 && (A->src == VGEMM_SRC_X32 || A->src == VGEMM_SRC_CONV32)) variant = 0;
    // int32 images with C % 64 == 0 run 64 x 128 tiles on the DMA kernel, which stages the raw int32
    // rows in LDS and quantises them per fragment (C3 shape: 116 us, 218 us on the register-staged kernel)
    if (A->src == VGEMM_SRC_CONV32 && g_variant < 0 && p.C % 64 == 0) variant = 1;
    // int32 rows likewise (K % 4 == 0)
    if (A->src == VGEMM_SRC_X32 && g_variant < 0 && p.K % 4 == 0) variant = 1;
    if (epi == VGEMM_EPI_QKV) variant = 0;   // whole heads per wave (the reference forces its 64 x 64 tile, src/gemm_hl.cu:358)
    if (p.gnstat) {
        // statistics regions = the reference's tile; the block must hold whole regions (128 x 128
        // holds any of them, as does the halo kernel's 128 x 128)
        const Tiles rt = gn_ref_tile(Mp, Np, Kp, A->src);
        p.gnBM = rt.BM;
        p.gnBN = rt.BN;
        if (!halo_bm && (TILES[variant].BM % rt.BM || TILES[variant].BN % rt.BN)) variant = 0;
    }
    const int BM = TILES[variant].BM, BN = TILES[variant].BN;
    p.mtiles = cdiv(Mreal, BM);
    p.ntiles = cdiv(Nreal, BN);
    const int nK = halo_bm ? p.C / 64 : (Kp + 63) / 64;
    // the split-K epilogue pass carries neither the QKV layout nor the GroupNorm statistics
    int splits = epi != VGEMM_EPI_QKV && !E->gnstat ? pick_splitk(variant, Mreal, Nreal, Kp) : 1;
    if (splits > 1 && !wsp.ws) {
        size_t have = 0;
        if (void* sw = stream_workspace(st, ws_bytes_for(variant, Mreal, Nreal, splits), &have)) wsp = WsPolicy{sw, have, false};
    }
    if (!wsp.ws) splits = 1;
    if (splits > 1 && ws_bytes_for(variant, Mreal, Nreal, splits) > wsp.bytes) {
        if (wsp.strict)
            return fail(VGEMM_ERR_UNSUPPORTED, "gemm_hl_noalloc: the split-K partials of this call need %zu bytes; the static workspace holds %zu",
                        ws_bytes_for(variant, Mreal, Nreal, splits), wsp.bytes);
        splits = 1;
    }
    if (splits > nK) splits = nK;
    // few output tiles over a deep K with no split-K workspace (the reference's own AEpi has none):
    // the K-split-over-waves kernel (forced by variant 5 where it applies)
    if (kwave_applies(A->src, epi, p) && (g_variant == VARIANT_KWAVE || (g_variant < 0 && splits <= 1 && kwave_auto(p)))) {
        p.mtiles = cdiv(Mreal, 64);
        p.ntiles = cdiv(Nreal, 64);
        p.ksplit = 1;
        p.kper = (Kp + 63) / 64;
        p.colmajor = pick_tile_order(p, a_operand_bytes(A, p));
        return hip_status(vk::launch_kwave(A->src, epi, p, st), "gemm_hl kwave launch");
    }
    auto run = [&](int e) {
        if (halo_bm) return hip_status(vk::launch_gemm_conv16_halo(halo_bm, e, p, st), "gemm_hl halo conv launch");
        // more blocks than CUs over many K steps: blocks of a CU keep pace through banded wave
        // priority (C3: 83.2 -> 79.2 us; no gain for short K loops, whose blocks end together)
        p.prio_bands = p.kper >= 32 && p.mtiles * p.ntiles * p.ksplit > NCU ? 4 : 0;
        return launch_src(A->src, variant, e, p, st);
    };
    const double a_bytes = a_operand_bytes(A, p);
    if (splits <= 1) {
        p.ksplit = 1; p.kper = nK;
        p.colmajor = pick_tile_order(p, a_bytes);
        return run(p.gnstat ? vk::EPI_PLAIN_GN : epi);
    }
    if (!aligned16(wsp.ws)) return fail(VGEMM_ERR_ARG, "gemm_hl: workspace must be 16-byte aligned");
    p.ksplit = splits;
    p.kper = (nK + splits - 1) / splits;
    p.ksplit = (nK + p.kper - 1) / p.kper;
    p.colmajor = pick_tile_order(p, a_bytes);
    p.ws = static_cast<int32_t*>(wsp.ws);
    p.ws_rows = p.mtiles * BM;
    p.ws_ld = p.ntiles * BN;
    const int rc = run(vk::EPI_PARTIAL);
    if (rc) return rc;
    return hip_status(vk::launch_splitk_epilogue(epi, p, st), "gemm_hl split-K epilogue");
}

// ---- the allocation-free entry point's workspace
// A file-scope device array serves as the split-K workspace of vgemm_hl2_noalloc. Each GPU the
// library runs on holds its own copy for the life of the process. In host code the name `scratch`
// is not a device address: its address on the current device comes from hipGetSymbolAddress, taken
// once per device (scratch_on_current_device) and used everywhere host code refers to it. The
// partial pass writes every element of its tiles in every K range before the reduction reads them,
// so nothing in it has to start at zero; concurrent calls on one GPU share it and race.
static __device__ __align__(256) unsigned char scratch[VGEMM_NOALLOC_WS_BYTES];

constexpr int SCRATCH_MAX_DEVICES = 64;
std::atomic<void*> g_scratch_dev[SCRATCH_MAX_DEVICES];
std::mutex g_scratch_mu;

int scratch_on_current_device(void** out) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return fail(VGEMM_ERR_UNSUPPORTED, "gemm_hl_noalloc: device %d out of range", dev);
    void* ptr = g_scratch_dev[dev].load(std::memory_order_acquire);
    if (!ptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        ptr = g_scratch_dev[dev].load(std::memory_order_relaxed);
        if (!ptr) {
            const hipError_t ge = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
            if (ge != hipSuccess || !ptr) return fail(VGEMM_ERR_HIP, "gemm_hl_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(ge));
            g_scratch_dev[dev].store(ptr, std::memory_order_release);
        }
    }
    *out = ptr;
    return VGEMM_OK;
}

}  // namespace

extern "C" {

int vgemm_hl2(void* stream, const VgemmASrc* A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal, int Kp,
              const int32_t* cst, const VgemmAEpi* E) {
    return hl2_impl(stream, A, Mp, Mreal, W, ldw, Np, Nreal, Kp, cst, E, WsPolicy{E ? E->ws : nullptr, E ? E->ws_bytes : 0, false});
}

int vgemm_hl2_view(void* stream, const VgemmASrc* A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal, int Kp,
                   const int32_t* cst, const VgemmAEpi* E, const VgemmView* V) {
    if (!V) return fail(VGEMM_ERR_ARG, "gemm_hl int16 view: null view");
    return hl2_impl(stream, A, Mp, Mreal, W, ldw, Np, Nreal, Kp, cst, E, WsPolicy{E ? E->ws : nullptr, E ? E->ws_bytes : 0, false}, V);
}

int vgemm_hl2_noalloc(void* stream, const VgemmASrc* A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal, int Kp,
                      const int32_t* cst, const VgemmAEpi* E) {
    void* ws = nullptr;
    const int rc = scratch_on_current_device(&ws);
    if (rc) return rc;
    return hl2_impl(stream, A, Mp, Mreal, W, ldw, Np, Nreal, Kp, cst, E, WsPolicy{ws, VGEMM_NOALLOC_WS_BYTES, true});
}

int vgemm_hl(void* stream, const int8_t* Ahi, const int8_t* Alo, int lda, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal,
             int Kp, const int32_t* cst, const int32_t* e, int32_t* Y, int ldy, const int32_t* residual, int epi, int Cs, int32_t* Y1,
             int32_t* Y2, const int32_t* Lphi) {
    VgemmASrc A;
    vgemm_asrc_init(&A);
    A.src = VGEMM_SRC_I8; A.hi = Ahi; A.lo = Alo; A.ld8 = lda; A.e = e;
    VgemmAEpi E;
    vgemm_aepi_init(&E);
    E.epi = epi; E.Y = Y; E.ldy = ldy; E.residual = residual; E.Cs = Cs; E.Y1 = Y1; E.Y2 = Y2; E.Lphi = Lphi;
    return vgemm_hl2(stream, &A, Mp, Mreal, W, ldw, Np, Nreal, Kp, cst, &E);
}

int vgemm_conv_e(void* stream, const uint32_t* pm, int B, int H, int W, int stride, int32_t* e) {
    if (!pm || !e || B <= 0 || H <= 0 || W <= 0 || stride <= 0) return fail(VGEMM_ERR_ARG, "conv_e: bad arguments");
    return hip_status(vk::launch_conv_e(static_cast<hipStream_t>(stream), pm, B, H, W, stride, e), "conv_e launch");
}

// ---- meow::Gemm replacement
// The handle owns the workspace its init asks for (the reference's Gemm::init allocates it for
// cuBLASLt, src/gemm.cu:7-11): split-K partial sums of deep-K calls with few tiles. Calls on one
// handle share it and must not overlap (as calls sharing a cuBLASLt workspace must not).
struct VgemmI8Handle {
    size_t ws_bytes;
    void* ws;
};

int vgemm_i8_create(size_t ws_bytes, void** handle) {
    if (!handle) return fail(VGEMM_ERR_ARG, "i8gemm: null handle pointer");
    *handle = nullptr;
    void* ws = nullptr;
    if (ws_bytes) {
        const hipError_t e = hipMalloc(&ws, ws_bytes);
        if (e != hipSuccess) return fail(VGEMM_ERR_HIP, "i8gemm: workspace hipMalloc(%zu): %s", ws_bytes, hipGetErrorString(e));
    }
    *handle = new VgemmI8Handle{ws ? ws_bytes : 0, ws};
    return ok();
}

int vgemm_i8_destroy(void* handle) {
    VgemmI8Handle* h = static_cast<VgemmI8Handle*>(handle);
    if (h && h->ws) (void)hipFree(h->ws);
    delete h;
    return ok();
}

int vgemm_i8_run(void* handle, void* stream, const int8_t* A, int lda, long long strideA, const int8_t* W, int ldw, long long strideW,
                 int32_t* C, int ldc, long long strideC, int M, int N, int K, int batch) {
    if (!handle) return fail(VGEMM_ERR_ARG, "i8gemm: null handle");
    if (!A || !W || !C) return fail(VGEMM_ERR_ARG, "i8gemm: null pointer");
    if (M <= 0 || N <= 0 || K <= 0 || batch <= 0) return fail(VGEMM_ERR_ARG, "i8gemm: no int8 GEMM for M=%d N=%d K=%d batch=%d", M, N, K, batch);
    if (K % 16 || N % 4) return fail(VGEMM_ERR_ARG, "i8gemm: K %% 16 == 0 and N %% 4 == 0 required (M=%d N=%d K=%d)", M, N, K);
    if (lda < K || ldw < K || ldc < N || lda % 16 || ldw % 16 || !aligned16(A) || !aligned16(W) || !aligned16(C))
        return fail(VGEMM_ERR_ARG, "i8gemm: leading dimensions must cover K/N, be multiples of 16 bytes, pointers 16-byte aligned");
    if (batch > 1 && (strideA % 16 || strideW % 16 || strideC % 4)) return fail(VGEMM_ERR_ARG, "i8gemm: batch strides must keep 16-byte alignment");
    const long long aext = (long long)(M - 1) * lda + K, wext = (long long)(N - 1) * ldw + K;
    if (aext > MAX_EXTENT || wext > MAX_EXTENT) return fail(VGEMM_ERR_UNSUPPORTED, "i8gemm: operand larger than 2 GiB");
    if (batch > 65535) return fail(VGEMM_ERR_UNSUPPORTED, "i8gemm: batch > 65535");
    vk::GemmParams p;
    std::memset(&p, 0, sizeof p);
    p.a0 = A; p.a0_bytes = unsigned(aext); p.lda = lda;
    p.w = W; p.w_bytes = unsigned(wext); p.ldw = ldw;
    p.Y = C; p.ldy = ldc; p.vec_store = ldc % 4 == 0 ? 1 : 0;
    p.Mreal = M; p.Nreal = N; p.Kp = K; p.K = K;
    p.sA = strideA; p.sW = strideW; p.sC = strideC;
    const int variant = g_variant >= 0 && g_variant < NVARIANT ? g_variant : pick_variant_raw(M, N, K);
    p.mtiles = cdiv(M, TILES[variant].BM);
    p.ntiles = cdiv(N, TILES[variant].BN);
    const int nK = (K + 63) / 64;
    p.ksplit = 1; p.kper = nK;
    p.stride = 1;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // deep K over fewer tiles than CUs: split K into the handle's workspace, then sum the ranges
    const VgemmI8Handle* h = static_cast<const VgemmI8Handle*>(handle);
    const long long tiles = (long long)p.mtiles * p.ntiles;
    if (batch == 1 && h->ws && tiles < NCU && nK >= 32 && ldc % 4 == 0 && g_splitk != 1) {
        const long long rows = (long long)p.mtiles * TILES[variant].BM, cols = (long long)p.ntiles * TILES[variant].BN;
        const long long plane = rows * cols * 4;
        long long s = g_splitk > 1 ? g_splitk : std::min<long long>(2LL * NCU / tiles, nK / 16);
        s = std::min<long long>(s, (long long)(h->ws_bytes / size_t(plane)));
        if (s * plane > MAX_EXTENT) s = MAX_EXTENT / plane;
        if (s >= 2) {
            p.kper = (nK + int(s) - 1) / int(s);
            p.ksplit = (nK + p.kper - 1) / p.kper;
            p.Y = static_cast<int32_t*>(h->ws); p.ldy = int(cols); p.sC = rows * cols; p.vec_store = 1;
            p.colmajor = pick_tile_order(p, double(M) * K);
            if (int rc = hip_status(vk::launch_gemm_raw(variant, p, 1, st), "i8gemm split launch")) return rc;
            return hip_status(vk::launch_raw_reduce(static_cast<const int32_t*>(h->ws), p.ksplit, plane, int(cols), M, N, C, ldc, st),
                              "i8gemm split reduce");
        }
    }
    p.colmajor = pick_tile_order(p, double(M) * K);
    return hip_status(vk::launch_gemm_raw(variant, p, batch, st), "i8gemm launch");
}

// ---- producers
int vgemm_quant_rows(void* stream, const int32_t* X, int M, int K, int ldx, int8_t* hi, int8_t* lo, int32_t* e, int Kp) {
    if (!X || !hi || !lo || !e || M <= 0 || K <= 0 || Kp < K || Kp % 4 || ldx < K) return fail(VGEMM_ERR_ARG, "quant_rows: bad arguments");
    return hip_status(vk::launch_quant_rows(static_cast<hipStream_t>(stream), X, M, K, ldx, hi, lo, e, Kp, (M + 31) / 32 * 32), "quant_rows launch");
}

int vgemm_epilogue(void* stream, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int32_t* cst, const int32_t* e, int32_t* Y,
                   int ldy, const int32_t* residual, void* gs, int T) {
    if (N % 4 || ldc % 4 || ldy % 4) return fail(VGEMM_ERR_ARG, "epilogue: N/ld must be multiples of 4");
    if (!Chi || !Clo || !cst || !e || !Y || M <= 0 || N <= 0) return fail(VGEMM_ERR_ARG, "epilogue: bad arguments");
    if (!aligned16(Chi) || !aligned16(Clo) || !aligned16(Y) || (residual && !aligned16(residual))) return fail(VGEMM_ERR_ARG, "epilogue: pointers must be 16-byte aligned");
    // src/kernels.h:16: 32 groups of whole columns, a block's 1024 elements in one sample
    if (gs && (N % 32 || T <= 0 || ((long long)T * N) % 1024 || ldy != N)) return fail(VGEMM_ERR_ARG, "epilogue GN stats: shape (N %% 32 == 0, (T*N) %% 1024 == 0 and ldy == N required)");
    return hip_status(vk::launch_epilogue(static_cast<hipStream_t>(stream), Chi, Clo, M, N, ldc, reinterpret_cast<const int4*>(cst), e, Y, ldy, residual,
                                          static_cast<vk::GnStat*>(gs), T),
                      "epilogue launch");
}

int vgemm_pixmax(void* stream, const int32_t* X, int rows, int C, uint32_t* pm) {
    if (!X || !pm || rows <= 0 || C <= 0) return fail(VGEMM_ERR_ARG, "pixmax: bad arguments");
    return hip_status(vk::launch_pixmax(static_cast<hipStream_t>(stream), X, rows, C, pm), "pixmax launch");
}

int vgemm_im2col3(void* stream, const int32_t* X, const uint32_t* pm, int B, int H, int W, int C, int stride, int8_t* hi, int8_t* lo, int32_t* e,
                  int Kp) {
    if (!X || !pm || !hi || !lo || !e || B <= 0 || H <= 0 || W <= 0 || stride <= 0) return fail(VGEMM_ERR_ARG, "im2col3: bad arguments");
    if (C <= 0 || C % 4 || Kp < 9 * C || Kp % 4 || !aligned16(X)) return fail(VGEMM_ERR_ARG, "im2col3: C %% 4 == 0, Kp >= 9C, Kp %% 4 == 0, aligned X required");
    return hip_status(vk::launch_im2col3(static_cast<hipStream_t>(stream), X, pm, B, H, W, C, stride, hi, lo, e, Kp), "im2col3 launch");
}

int vgemm_epilogue_split(void* stream, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int32_t* cst, const int32_t* e, int Cs,
                         int32_t* Y0, int32_t* Y1, int32_t* Y2) {
    if (!Chi || !Clo || !cst || !e || !Y0 || M <= 0 || N <= 0 || Cs <= 0 || N > 3 * Cs || (N > Cs && !Y1) || (N > 2 * Cs && !Y2))
        return fail(VGEMM_ERR_ARG, "epilogue_split: bad arguments");
    return hip_status(vk::launch_epilogue_split(static_cast<hipStream_t>(stream), Chi, Clo, M, N, ldc, reinterpret_cast<const int4*>(cst), e, Cs, Y0, Y1, Y2),
                      "epilogue_split launch");
}

int vgemm_epilogue_geglu_q(void* stream, const int32_t* Chi, const int32_t* Clo, int M, int F, int ldc, const int32_t* cst, const int32_t* e,
                           const int32_t* Lphi, int8_t* hi, int8_t* lo, int32_t* eo, int Kp) {
    if (!Chi || !Clo || !cst || !e || !Lphi || !hi || !lo || !eo || M <= 0 || F <= 0 || Kp < F) return fail(VGEMM_ERR_ARG, "epilogue_geglu_q: bad arguments");
    if (F > 5120) return fail(VGEMM_ERR_ARG, "epilogue_geglu_q: F too large");
    return hip_status(vk::launch_epilogue_geglu_q(static_cast<hipStream_t>(stream), Chi, Clo, M, F, ldc, reinterpret_cast<const int4*>(cst), e, Lphi, hi, lo,
                                                  eo, Kp),
                      "epilogue_geglu_q launch");
}

// ---- graphs
int vgemm_graph_begin(void* stream) {
    if (!stream) return fail(VGEMM_ERR_ARG, "graph_begin: the null stream cannot be captured");
    return hip_status(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}

int vgemm_graph_end(void* stream, void** exec) {
    if (!stream || !exec) return fail(VGEMM_ERR_ARG, "graph_end: bad arguments");
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(stream), &g);
    if (e != hipSuccess) return hip_status(e, "hipStreamEndCapture");
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_status(e, "hipGraphInstantiate");
    *exec = x;
    return ok();
}

int vgemm_graph_launch(void* exec, void* stream) {
    if (!exec) return fail(VGEMM_ERR_ARG, "graph_launch: null graph");
    return hip_status(hipGraphLaunch(static_cast<hipGraphExec_t>(exec), static_cast<hipStream_t>(stream)), "hipGraphLaunch");
}

int vgemm_graph_destroy(void* exec) {
    if (!exec) return ok();
    return hip_status(hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec)), "hipGraphExecDestroy");
}

int vgemm_fill_u32(void* stream, uint32_t* p, size_t count, uint32_t value) {
    if (!p && count) return fail(VGEMM_ERR_ARG, "fill_u32: null pointer");
    if (!count) return ok();
    return hip_status(vk::launch_fill_u32(static_cast<hipStream_t>(stream), p, count, value), "fill_u32 launch");
}

// ---- elementwise kernels (src/kernels.cu:537-566, 767-771)
int vgemm_act(void* stream, int32_t* X, size_t n, const int32_t* L) {
    if (!n) return ok();
    if (!X || !L) return fail(VGEMM_ERR_ARG, "act: null pointer");
    return hip_status(vk::launch_act(static_cast<hipStream_t>(stream), X, n, L), "act launch");
}

int vgemm_geglu(void* stream, int32_t* A, const int32_t* G, size_t n, const int32_t* L) {
    if (!n) return ok();
    if (!A || !G || !L) return fail(VGEMM_ERR_ARG, "geglu: null pointer");
    return hip_status(vk::launch_geglu(static_cast<hipStream_t>(stream), A, G, n, L), "geglu launch");
}

int vgemm_add(void* stream, int32_t* X, const int32_t* Y, size_t n) {
    if (!n) return ok();
    if (!X || !Y) return fail(VGEMM_ERR_ARG, "add: null pointer");
    return hip_status(vk::launch_add(static_cast<hipStream_t>(stream), X, Y, n), "add launch");
}

int vgemm_concat(void* stream, const int32_t* A, int Ca, const int32_t* B, int Cb, int rows, int32_t* out, void* gs, int T) {
    if (Ca < 0 || Cb < 0 || rows < 0 || (Ca && !A) || (Cb && !B)) return fail(VGEMM_ERR_ARG, "concat: bad arguments");
    const int Co = Ca + Cb;
    if (gs && (Co % 32 || T <= 0 || ((long long)T * Co) % 256)) return fail(VGEMM_ERR_ARG, "concat GN stats: shape");   // src/kernels.cu:768
    if (!rows || !Co) return ok();
    if (!out) return fail(VGEMM_ERR_ARG, "concat: bad arguments");
    return hip_status(vk::launch_concat(static_cast<hipStream_t>(stream), A, Ca, B, Cb, rows, out, static_cast<vk::GnStat*>(gs), T), "concat launch");
}

int vgemm_upsample2(void* stream, const int32_t* X, int B, int H, int W, int C, int32_t* out) {
    if (B < 0 || H < 0 || W < 0 || C < 0) return fail(VGEMM_ERR_ARG, "upsample2: bad arguments");
    if (!B || !H || !W || !C) return ok();
    if (!X || !out) return fail(VGEMM_ERR_ARG, "upsample2: null pointer");
    return hip_status(vk::launch_upsample2(static_cast<hipStream_t>(stream), X, B, H, W, C, out), "upsample2 launch");
}

int vgemm_gn_init(void* stream, void* gs, int count) {
    if (!gs || count <= 0) return fail(VGEMM_ERR_ARG, "gn_init: bad arguments");
    return hip_status(vk::launch_gn_init(static_cast<hipStream_t>(stream), static_cast<vk::GnStat*>(gs), count), "gn_init launch");
}

// ---- integer normalisations (src/kernels.cu:172-305,349-420, 745-762,820-830)
namespace {
int norm_shape(const char* what, const int32_t* X, long long rows, int C) {
    if (!X || rows <= 0 || C <= 0) return fail(VGEMM_ERR_ARG, "%s: bad arguments", what);
    if (C % 4 || C > 2560) return fail(VGEMM_ERR_ARG, "%s: C must be a multiple of 4 and at most 2560", what);
    if (!aligned16(X)) return fail(VGEMM_ERR_ARG, "%s: X must be 16-byte aligned", what);
    if (rows * C > (1LL << 40)) return fail(VGEMM_ERR_UNSUPPORTED, "%s: too many elements", what);
    return VGEMM_OK;
}
int gn_shape(const char* what, const int32_t* X, int B, int T, int C, int groups, const void* gs) {
    if (B <= 0 || T <= 0 || !gs) return fail(VGEMM_ERR_ARG, "%s: bad arguments", what);
    if (int rc = norm_shape(what, X, (long long)B * T, C)) return rc;
    if (groups <= 0 || groups > 64 || C % groups) return fail(VGEMM_ERR_ARG, "%s: groups must divide C and be at most 64", what);
    return VGEMM_OK;
}
int view_planes(const char* what, int C, const int8_t* hi, const int8_t* lo, const int32_t* e, int Kp) {
    if (!lo || !e || Kp < C || Kp % 4 || ((uintptr_t)hi | (uintptr_t)lo) & 3) return fail(VGEMM_ERR_ARG, "%s: hi/lo/e with Kp >= C, Kp %% 4 == 0, 4-byte aligned planes", what);
    return VGEMM_OK;
}
}  // namespace

int vgemm_gn_stats1(void* stream, const int32_t* X, int B, int T, int C, int groups, void* gs) {
    if (int rc = gn_shape("gn_stats1", X, B, T, C, groups, gs)) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    vk::GnStat* g = static_cast<vk::GnStat*>(gs);
    const int cnt = B * groups;
    if (int rc = hip_status(vk::launch_gn_init(st, g, cnt), "gn_stats1 init")) return rc;
    if (int rc = hip_status(vk::launch_gn_reduce(st, false, X, B, T, C, groups, g), "gn_stats1 reduce")) return rc;
    return hip_status(vk::launch_gn_fin1(st, g, cnt, (long long)T * (C / groups)), "gn_stats1 fin1");
}

int vgemm_gn_fin1(void* stream, void* gs, int cnt, int64_t n) {
    if (!gs || cnt <= 0 || n <= 0) return fail(VGEMM_ERR_ARG, "gn_fin1: bad arguments");
    return hip_status(vk::launch_gn_fin1(static_cast<hipStream_t>(stream), static_cast<vk::GnStat*>(gs), cnt, n), "gn_fin1 launch");
}

int vgemm_gn_stats2(void* stream, const int32_t* X, int B, int T, int C, int groups, int64_t den, void* gs) {
    if (int rc = gn_shape("gn_stats2", X, B, T, C, groups, gs)) return rc;
    if (den <= 0) return fail(VGEMM_ERR_ARG, "gn_stats2: den must be positive");
    hipStream_t st = static_cast<hipStream_t>(stream);
    vk::GnStat* g = static_cast<vk::GnStat*>(gs);
    if (int rc = hip_status(vk::launch_gn_reduce(st, true, X, B, T, C, groups, g), "gn_stats2 reduce")) return rc;
    return hip_status(vk::launch_gn_fin2(st, g, B * groups, (long long)T * (C / groups), den), "gn_stats2 fin2");
}

int vgemm_gn_apply(void* stream, const int32_t* X, int B, int T, int C, int groups, const void* gs, const int64_t* g, const int64_t* beta, int32_t* Y) {
    if (int rc = gn_shape("gn_apply", X, B, T, C, groups, gs)) return rc;
    if (!g || !beta || !Y) return fail(VGEMM_ERR_ARG, "gn_apply: bad arguments");
    return hip_status(vk::launch_gn_apply(static_cast<hipStream_t>(stream), X, B, T, C, groups, static_cast<const vk::GnStat*>(gs), reinterpret_cast<const long long*>(g), reinterpret_cast<const long long*>(beta), Y),
                      "gn_apply launch");
}

int vgemm_gn_apply_row(void* stream, const int32_t* X, int B, int T, int C, int groups, const void* gs, const int32_t* g, const int32_t* beta,
                       const int32_t* Lsig, int32_t* Y, uint32_t* pm, int8_t* hi, int8_t* lo, int32_t* e, int Kp) {
    if (int rc = gn_shape("gn_apply_row", X, B, T, C, groups, gs)) return rc;
    // the reference's row kernel caches 32 records per row (src/kernels.cu:287-305)
    if (groups > 32) return fail(VGEMM_ERR_ARG, "gn_apply_row: at most 32 groups");
    if (!g || !beta || !aligned16(g) || !aligned16(beta)) return fail(VGEMM_ERR_ARG, "gn_apply_row: g/beta must be 16-byte aligned");
    if (hi) {
        if (int rc = view_planes("gn_apply_row", C, hi, lo, e, Kp)) return rc;
    } else if (!Y || !aligned16(Y)) {
        return fail(VGEMM_ERR_ARG, "gn_apply_row: Y (16-byte aligned) or hi/lo/e required");
    }
    return hip_status(vk::launch_gn_apply_row(static_cast<hipStream_t>(stream), X, B * T, T, C, groups, static_cast<const vk::GnStat*>(gs), g, beta, Lsig,
                                              Y, pm, hi, lo, e, Kp),
                      "gn_apply_row launch");
}

int vgemm_lnorm(void* stream, const int32_t* X, int M, int C, const int64_t* g, const int64_t* beta, int64_t den, int32_t* Y) {
    if (int rc = norm_shape("lnorm", X, M, C)) return rc;
    if (!g || !beta || !Y || !aligned16(Y) || den <= 0) return fail(VGEMM_ERR_ARG, "lnorm: bad arguments");
    return hip_status(vk::launch_lnorm(static_cast<hipStream_t>(stream), false, X, M, C, g, beta, den, Y, nullptr, nullptr, nullptr, 0), "lnorm launch");
}

int vgemm_lnorm_q(void* stream, const int32_t* X, int M, int C, const int32_t* g, const int32_t* beta, int64_t den, int8_t* hi, int8_t* lo, int32_t* e,
                  int Kp) {
    if (int rc = norm_shape("lnorm_q", X, M, C)) return rc;
    if (!g || !beta || !aligned16(g) || !aligned16(beta) || !hi || den <= 0) return fail(VGEMM_ERR_ARG, "lnorm_q: bad arguments");
    if (int rc = view_planes("lnorm_q", C, hi, lo, e, Kp)) return rc;
    return hip_status(vk::launch_lnorm(static_cast<hipStream_t>(stream), true, X, M, C, g, beta, den, nullptr, hi, lo, e, Kp), "lnorm_q launch");
}

// ---- attention (src/kernels.h:42-50,61,73-77)

int vgemm_quant_heads(void* stream, const int32_t* X, int B, int T, int C, int heads, int Tp, int8_t* hi, int8_t* lo, int32_t* e, int64_t* hs,
                      int64_t* ls, int64_t* tsum) {
    if (!X || !hi || !lo || !e || !hs || !ls || !tsum || B <= 0 || heads <= 0 || T <= 0 || Tp < T || C < 64 * heads)
        return fail(VGEMM_ERR_ARG, "quant_heads: bad arguments");
    return hip_status(vk::launch_quant_heads(static_cast<hipStream_t>(stream), X, B, T, C, heads, Tp, hi, lo, e, reinterpret_cast<long long*>(hs),
                                             reinterpret_cast<long long*>(ls), reinterpret_cast<long long*>(tsum)),
                      "quant_heads launch");
}

int vgemm_quant_heads_pad(void* stream, int G, int T, int Tp, int8_t* hi, int8_t* lo, int32_t* e, int64_t* hs, int64_t* ls, int64_t* tsum) {
    if (G <= 0 || T < 0) return fail(VGEMM_ERR_ARG, "quant_heads_pad: bad arguments");
    if (Tp <= T) return VGEMM_OK;   // nothing to pad (src/kernels.cu:807)
    if (!hi || !lo || !e || !hs || !ls || !tsum) return fail(VGEMM_ERR_ARG, "quant_heads_pad: bad arguments");
    return hip_status(vk::launch_quant_heads_pad(static_cast<hipStream_t>(stream), G, T, Tp, hi, lo, e, reinterpret_cast<long long*>(hs),
                                                 reinterpret_cast<long long*>(ls), reinterpret_cast<long long*>(tsum)),
                      "quant_heads_pad launch");
}

int vgemm_quant_v(void* stream, const int32_t* X, int B, int Tk, int C, int heads, int Tkp, int8_t* vthi, int8_t* vtlo, int32_t* ev, int64_t* vsum,
                  uint32_t* scratch) {
    (void)scratch;   // the column maxima stay inside one block per group here
    if (!X || !vthi || !vtlo || !ev || !vsum || B <= 0 || heads <= 0 || Tk <= 0 || Tkp < Tk || C < 64 * heads)
        return fail(VGEMM_ERR_ARG, "quant_v: bad arguments");
    if (Tkp % 64 || !aligned16(vthi) || !aligned16(vtlo)) return fail(VGEMM_ERR_ARG, "quant_v: Tkp %% 64 == 0 and 16-byte aligned planes required");
    return hip_status(vk::launch_quant_v(static_cast<hipStream_t>(stream), X, B, Tk, C, heads, Tkp, vthi, vtlo, ev, reinterpret_cast<long long*>(vsum)),
                      "quant_v launch");
}

int vgemm_fused_attention(void* stream, const int8_t* qhi, const int8_t* qlo, const int32_t* eq, const int64_t* qhs, const int64_t* qls,
                          const int8_t* khi, const int8_t* klo, const int32_t* ek, const int64_t* ksum, const int8_t* vthi, const int8_t* vtlo,
                          const int32_t* ev, const int64_t* vsum, int B, int heads, int Tq, int Tqp, int Tk, int Tkp, int causal, const int64_t* Lexp,
                          int C, int32_t* gmx, int64_t* gr, int32_t* out, uint32_t* rowmax) {
    (void)vsum; (void)gmx; (void)gr;   // one launch: the row statistics never leave the kernel
    if (Tqp % 64 || Tkp % 64) return fail(VGEMM_ERR_ARG, "fused attention: Tqp/Tkp alignment");   // src/attn.cu:554
    if (!qhi || !qlo || !eq || !qhs || !qls || !khi || !klo || !ek || !ksum || !vthi || !vtlo || !ev || !Lexp || !out || B <= 0 || heads <= 0 ||
        Tq <= 0 || Tq > Tqp || Tk <= 0 || Tk > Tkp || C < 64 * heads || C % 4)
        return fail(VGEMM_ERR_ARG, "fused attention: bad arguments");
    if (!aligned16(qhi) || !aligned16(qlo) || !aligned16(khi) || !aligned16(klo) || !aligned16(vthi) || !aligned16(vtlo) || !aligned16(out))
        return fail(VGEMM_ERR_ARG, "fused attention: operands must be 16-byte aligned");
    if ((long long)B * heads > 65535) return fail(VGEMM_ERR_UNSUPPORTED, "fused attention: at most 65535 groups");
    const vk::AttnArgs a{qhi, qlo, eq, reinterpret_cast<const long long*>(qhs), reinterpret_cast<const long long*>(qls), khi, klo, ek,
                         reinterpret_cast<const long long*>(ksum), vthi, vtlo, ev, heads, Tq, Tqp, Tk, Tkp, causal ? 1 : 0,
                         reinterpret_cast<const long long*>(Lexp), C, out, rowmax};
    return hip_status(vk::launch_attention(static_cast<hipStream_t>(stream), a, B * heads), "fused attention launch");
}

const char* vgemm_last_error(void) { return g_err.c_str(); }
const char* vgemm_version(void) { return "vgemm 0.1 gfx950"; }

}  // extern "C"

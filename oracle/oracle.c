/*
 * TEST INFRASTRUCTURE ONLY -- CPU restatement of the reference's W8A16 hi/lo integer GEMM path
 * (emanwrxsti/vela: src/intops.cuh, src/gemm_hl.cu, src/kernels.cu, src/engine.cu).
 *
 * Used as the correctness oracle by tests/ and __graft_entry__.smoke(), and timed by bench.py's
 * cpu_baseline leg ("port": the reference has no CPU GEMM of its own). The MI355X product path in
 * vela_amd/ never calls into this file.
 *
 * Structure deliberately follows the reference's arithmetic, not the GPU kernel's: the A operand is
 * materialised as int8 hi/lo planes per row, each plane is dotted with W in int32, and the exact
 * int64 epilogue epi1 reconstructs acc = 256*Chi + Clo + 128*wsum (src/gemm_hl.cu:40-43).
 *
 * How each function is pinned (tests/test_oracle_*.py): closed forms and brute force for the
 * primitives, the reference's own edge lists (src/test_attn_score.cu:14, src/test_im2col.cu:13-20),
 * an independent int64 q.W matmul with exact rational rounding for the GEMM, the m=1,s=0,b=0
 * special case (a plain integer matmul), and hand-computed fixtures in tests/golden/.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0;
void orc_set_threads(int n) { g_threads = n; }
int orc_get_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ primitives: src/intops.cuh */

/* src/intops.cuh:9 */
int64_t orc_sat32(int64_t v) { return v < INT64_C(-2147483648) ? INT64_C(-2147483648) : (v > INT64_C(2147483647) ? INT64_C(2147483647) : v); }

/* src/intops.cuh:11-17. The rounding add wraps on overflow (as the device's 64-bit add does). */
int64_t orc_rshr(int64_t v, int64_t s) {
    if (s >= 0) {
        const int p = s > 62 ? 62 : (int)s;
        const int64_t half = (INT64_C(1) << p) >> 1;
        const int64_t t = (int64_t)((uint64_t)v + (uint64_t)half);
        return orc_sat32(t >> p);
    }
    const int neg = -s > 31 ? 31 : (int)(-s);
    const int64_t lim = INT64_C(1) << (62 - neg);
    const int64_t r = v < -lim ? -lim : (v > lim ? lim : v);
    return orc_sat32(r * (INT64_C(1) << neg));
}

/* src/intops.cuh:37-38: e = #{k in [15,32): m >= 2^k} */
int orc_row_exp(int64_t m) {
    int e = 0;
    for (int k = 15; k < 32; ++k) e += (m >= (INT64_C(1) << k));
    return e;
}

/* src/intops.cuh:39 */
int64_t orc_quant16(int64_t v, int e) {
    const int64_t q = orc_rshr(v, e);
    return q < -32767 ? -32767 : (q > 32767 ? 32767 : q);
}

/* src/intops.cuh:40-41 (e in [0,17]) */
int32_t orc_quant16_32(int32_t v, int e) {
    const int32_t q = e ? ((v >> e) + ((v >> (e - 1)) & 1)) : v;
    return q < -32767 ? -32767 : (q > 32767 ? 32767 : q);
}

/* src/intops.cuh:42-50; the int32 interpolation wraps like the device's 32-bit arithmetic */
int32_t orc_lut16i(int64_t x, const int32_t* L) {
    const int64_t z = x + (INT64_C(16) << 16);
    if (z < 0) return 0;
    if (z >= (INT64_C(32) << 16)) return 65536;
    const int i = (int)(z >> 10), f = (int)(z & 1023);
    const int32_t a = L[i], b = L[i + 1];
    const int32_t prod = (int32_t)(((uint32_t)b - (uint32_t)a) * (uint32_t)f);
    return (int32_t)((uint32_t)a + (uint32_t)(prod >> 10));
}

/* src/intops.cuh:65-66 */
void orc_split16(int64_t a, int8_t* hi, int8_t* lo) {
    *hi = (int8_t)(a >> 8);
    *lo = (int8_t)((a & 255) - 128);
}

/* src/gemm_hl.cu:40-43 (== src/kernels.cu:36-39, 59-62); c4 = {m, s, b, wsum}. acc*m wraps. */
int32_t orc_epi1(int32_t chi, int32_t clo, const int32_t* c4, int32_t er) {
    const int64_t acc = 256 * (int64_t)chi + (int64_t)clo + 128 * (int64_t)c4[3];
    const int64_t v = (int64_t)((uint64_t)acc * (uint64_t)(int64_t)c4[0]);
    return (int32_t)orc_sat32(orc_rshr(v, (int64_t)c4[1] - (int64_t)er) + c4[2]);
}

/* GEGLU of one interleaved pair: src/gemm_hl.cu:292-293 (== src/kernels.cu:510-513) */
int32_t orc_geglu(int32_t a, int32_t g, const int32_t* L) {
    const int64_t ge = orc_sat32(orc_rshr((int64_t)g * orc_lut16i(g, L), 16));
    return (int32_t)orc_sat32(orc_rshr((int64_t)a * ge, 16));
}

/* GELU epilogue: src/gemm_hl.cu:280 */
int32_t orc_gelu(int32_t y, const int32_t* L) { return (int32_t)orc_sat32(orc_rshr((int64_t)y * orc_lut16i(y, L), 16)); }

void orc_rshr_n(const int64_t* v, const int64_t* s, int64_t* out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = orc_rshr(v[i], s[i]); }
void orc_row_exp_n(const int64_t* m, int32_t* out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = orc_row_exp(m[i]); }
void orc_quant16_32_n(const int32_t* v, const int32_t* e, int32_t* out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = orc_quant16_32(v[i], e[i]); }
void orc_lut16i_n(const int64_t* x, const int32_t* L, int32_t* out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = orc_lut16i(x[i], L); }
void orc_epi1_n(const int32_t* chi, const int32_t* clo, const int32_t* c4, const int32_t* er, int32_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_epi1(chi[i], clo[i], c4 + 4 * i, er[i]);
}

static inline uint32_t uabs32(int32_t v) { return v < 0 ? (uint32_t)(-(int64_t)v) : (uint32_t)v; }
static inline int8_t qhi(int32_t q) { return (int8_t)(q >> 8); }
static inline int8_t qlo(int32_t q) { return (int8_t)((q & 255) - 128); }

/* ------------------------------------------------------------------ producers: src/kernels.cu */

/* k_quant_rows: src/kernels.cu:42-57, 488-497, 727-731. Rows [M, align32(M)) become the pad value
 * 0 = (hi 0, lo -128); their e is left untouched. */
void orc_quant_rows(const int32_t* X, int M, int K, int ldx, int8_t* hi, int8_t* lo, int32_t* e, int Kp) {
    const int Mp = (M + 31) / 32 * 32;
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (int r = 0; r < Mp; ++r) {
        int8_t* h = hi + (size_t)r * Kp;
        int8_t* l = lo + (size_t)r * Kp;
        if (r >= M) {
            for (int k = 0; k < Kp; ++k) { h[k] = 0; l[k] = -128; }
            continue;
        }
        const int32_t* x = X + (size_t)r * ldx;
        uint32_t m = 0;
        for (int k = 0; k < K; ++k) { const uint32_t a = uabs32(x[k]); m = a > m ? a : m; }
        const int ee = orc_row_exp(m);
        e[r] = ee;
        for (int k = 0; k < Kp; ++k) {
            const int32_t q = k < K ? orc_quant16_32(x[k], ee) : 0;
            h[k] = qhi(q); l[k] = qlo(q);
        }
    }
}

/* k_pixmax: src/kernels.cu:106-115 */
void orc_pixmax(const int32_t* X, int rows, int C, uint32_t* pm) {
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (int r = 0; r < rows; ++r) {
        uint32_t m = 0;
        for (int c = 0; c < C; ++c) { const uint32_t a = uabs32(X[(size_t)r * C + c]); m = a > m ? a : m; }
        pm[r] = m;
    }
}

static inline uint32_t window_max(const uint32_t* pm, int b, int H, int W, int stride, int oy, int ox) {
    uint32_t m = 0;
    for (int ky = 0; ky < 3; ++ky)
        for (int kx = 0; kx < 3; ++kx) {
            const int iy = oy * stride - 1 + ky, ix = ox * stride - 1 + kx;
            if (iy >= 0 && iy < H && ix >= 0 && ix < W) {
                const uint32_t v = pm[((size_t)b * H + iy) * W + ix];
                m = v > m ? v : m;
            }
        }
    return m;
}

/* k_im2col3: src/kernels.cu:117-170, 740-744. K index is tap-major (k = tap*C + c, tap = 3*ky + kx);
 * pad columns [9C, Kp) hold the value 0 = (0,-128); pad rows [rows, align32(rows)) are memset to
 * hi 0x00 / lo 0x80. */
void orc_im2col3(const int32_t* X, const uint32_t* pm, int B, int H, int W, int C, int stride,
                 int8_t* hi, int8_t* lo, int32_t* e, int Kp) {
    const int Ho = (H - 1) / stride + 1, Wo = (W - 1) / stride + 1, rows = B * Ho * Wo;
    const int Mp = (rows + 31) / 32 * 32, K = 9 * C;
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (int r = 0; r < Mp; ++r) {
        int8_t* h = hi + (size_t)r * Kp;
        int8_t* l = lo + (size_t)r * Kp;
        if (r >= rows) { memset(h, 0, (size_t)Kp); memset(l, 0x80, (size_t)Kp); continue; }
        const int b = r / (Ho * Wo), p = r % (Ho * Wo), oy = p / Wo, ox = p % Wo;
        const int ee = orc_row_exp(window_max(pm, b, H, W, stride, oy, ox));
        e[r] = ee;
        for (int tap = 0; tap < 9; ++tap) {
            const int iy = oy * stride - 1 + tap / 3, ix = ox * stride - 1 + tap % 3;
            const int in = iy >= 0 && iy < H && ix >= 0 && ix < W;
            const int32_t* xp = in ? X + (((size_t)b * H + iy) * W + ix) * C : NULL;
            for (int c = 0; c < C; ++c) {
                const int32_t q = in ? orc_quant16_32(xp[c], ee) : 0;
                h[tap * C + c] = qhi(q); l[tap * C + c] = qlo(q);
            }
        }
        for (int k = K; k < Kp; ++k) { h[k] = 0; l[k] = -128; }
    }
}

/* k_conv_e: src/gemm_hl.cu:335-341, 346-349 */
void orc_conv_e(const uint32_t* pm, int B, int H, int W, int stride, int32_t* e) {
    const int Ho = (H - 1) / stride + 1, Wo = (W - 1) / stride + 1, rows = B * Ho * Wo;
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (int r = 0; r < rows; ++r) {
        const int b = r / (Ho * Wo), p = r % (Ho * Wo), oy = p / Wo, ox = p % Wo;
        e[r] = orc_row_exp(window_max(pm, b, H, W, stride, oy, ox));
    }
}

/* k_epilogue (without GroupNorm statistics): src/kernels.cu:70-95 */
void orc_epilogue(const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int32_t* cst,
                  const int32_t* e, int32_t* Y, int ldy, const int32_t* R) {
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (int r = 0; r < M; ++r)
        for (int n = 0; n < N; ++n) {
            int32_t y = orc_epi1(Chi[(size_t)r * ldc + n], Clo[(size_t)r * ldc + n], cst + 4 * n, e[r]);
            if (R) y = (int32_t)orc_sat32((int64_t)y + R[(size_t)r * ldy + n]);
            Y[(size_t)r * ldy + n] = y;
        }
}

/* k_epilogue_split: src/kernels.cu:97-104 */
void orc_epilogue_split(const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int32_t* cst,
                        const int32_t* e, int Cs, int32_t* Y0, int32_t* Y1, int32_t* Y2) {
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (int r = 0; r < M; ++r)
        for (int n = 0; n < N; ++n) {
            const int part = n >= 2 * Cs ? 2 : (n >= Cs ? 1 : 0);
            int32_t* Y = part == 0 ? Y0 : (part == 1 ? Y1 : Y2);
            Y[(size_t)r * Cs + (n - part * Cs)] = orc_epi1(Chi[(size_t)r * ldc + n], Clo[(size_t)r * ldc + n], cst + 4 * n, e[r]);
        }
}

/* k_epilogue_geglu_q: src/kernels.cu:499-534 + quant_row_out (:250-259). Columns [0,F) are a,
 * [F,2F) are g; output row-quantised to hi/lo [*, Kp] + e, pad columns (0,-128). */
void orc_epilogue_geglu_q(const int32_t* Chi, const int32_t* Clo, int M, int F, int ldc, const int32_t* cst,
                          const int32_t* e, const int32_t* L, int8_t* hi, int8_t* lo, int32_t* eo, int Kp) {
#pragma omp parallel num_threads(orc_get_threads())
    {
        int32_t* v = (int32_t*)malloc(sizeof(int32_t) * (size_t)(F > 0 ? F : 1));
#pragma omp for schedule(static)
        for (int r = 0; r < M; ++r) {
            const size_t base = (size_t)r * ldc;
            uint32_t m = 0;
            for (int c = 0; c < F; ++c) {
                const int32_t a = orc_epi1(Chi[base + c], Clo[base + c], cst + 4 * c, e[r]);
                const int32_t g = orc_epi1(Chi[base + F + c], Clo[base + F + c], cst + 4 * (F + c), e[r]);
                v[c] = orc_geglu(a, g, L);
                const uint32_t u = uabs32(v[c]);
                m = u > m ? u : m;
            }
            const int ee = orc_row_exp(m);
            eo[r] = ee;
            int8_t* h = hi + (size_t)r * Kp;
            int8_t* l = lo + (size_t)r * Kp;
            for (int c = 0; c < F; ++c) { const int32_t q = orc_quant16_32(v[c], ee); h[c] = qhi(q); l[c] = qlo(q); }
            for (int c = F; c < Kp; ++c) { h[c] = 0; l[c] = -128; }
        }
        free(v);
    }
}

/* Exact GroupNorm statistics of an output (no flush rule): every y[r][n] is added to record
 * (r / T) * 32 + n / (N / 32): sum += y, mn = min(mn, y), mx = max(mx, y). The records are
 * accumulated into, as the reference's atomics do after k_gn_init. This is what the reference's
 * statistics reduce to when no tile's group is saturated through (see orc_gn_tiles). */
void orc_gn_accumulate(const int32_t* Y, int M, int N, int ldy, int T, int64_t* sum, int32_t* mn, int32_t* mx) {
    const int cg = N / 32;
    for (int r = 0; r < M; ++r) {
        const int b = r / T;
        for (int n = 0; n < N; ++n) {
            const int32_t y = Y[(size_t)r * ldy + n];
            const int k = b * 32 + n / cg;
            sum[k] += y;
            if (y < mn[k]) mn[k] = y;
            if (y > mx[k]) mx[k] = y;
        }
    }
}

/* Fold the statistics of one region (a tile or a block) into a record by the reference's flush
 * rule: the region's (sum, min, max) of a group are added only when its min is not INT_MAX, so a
 * region whose values of that group are all INT_MAX (or that holds none) adds nothing
 * (src/gemm_hl.cu:306-309, src/kernels.cu:67-68). */
static void gn_flush_region(int64_t rsum, int32_t rmn, int32_t rmx, int64_t* sum, int32_t* mn, int32_t* mx) {
    if (rmn == INT32_MAX) return;
    *sum += rsum;
    if (rmn < *mn) *mn = rmn;
    if (rmx > *mx) *mx = rmx;
}

/* The tile the reference's fused GEMM runs for these padded sizes, which is the region its
 * GroupNorm statistics are flushed by (src/gemm_hl.cu:352-358 with g_gemm_hl_variant = -1): for
 * Kp >= 2048 the 64x128 tile when Np % 128 == 0, else the 128x64 tile when Mp % 128 == 0 and the
 * source is the int8 planes; otherwise 64x64. src8 = 1 for int8-plane sources (SRC_I8, and the int16
 * rows that hold the same bytes), 0 for the sources quantised on load (SRC_X32, SRC_CONV32). */
void orc_gn_ref_tile(int Mp, int Np, int Kp, int src8, int* BMr, int* BNr) {
    int v = 0;
    if (Kp >= 2048) v = Np % 128 == 0 ? 2 : (Mp % 128 == 0 ? 1 : 0);
    if (v == 1 && Mp % 128) v = 0;
    if (v == 2 && Np % 128) v = 0;
    if (!src8 && v == 1) v = 0;
    *BMr = v == 1 ? 128 : 64;
    *BNr = v == 2 ? 128 : 64;
}

/* GroupNorm statistics of the fused GEMM's EPI_PLAIN output (src/gemm_hl.cu:175-177, 285-287,
 * 306-309): each BMr x BNr tile (rows m0 = i*BMr, columns n0 = j*BNr) gathers, per group
 * n / (N / 32), the sum, min and max of its outputs with r < M, n < N, and flushes them into record
 * (m0 / T) * 32 + group by the rule above. The whole tile goes to the sample of its first row, as
 * in the reference. */
void orc_gn_tiles(const int32_t* Y, int M, int N, int ldy, int T, int BMr, int BNr, int64_t* sum, int32_t* mn, int32_t* mx) {
    const int cg = N / 32;
    for (int m0 = 0; m0 < M; m0 += BMr) {
        const int b = m0 / T;
        for (int n0 = 0; n0 < N; n0 += BNr) {
            int64_t s[32];
            int32_t lo[32], hi[32];
            for (int g = 0; g < 32; ++g) { s[g] = 0; lo[g] = INT32_MAX; hi[g] = INT32_MIN; }
            for (int r = m0; r < m0 + BMr && r < M; ++r)
                for (int n = n0; n < n0 + BNr && n < N; ++n) {
                    const int32_t y = Y[(size_t)r * ldy + n];
                    const int g = n / cg;
                    s[g] += y;
                    if (y < lo[g]) lo[g] = y;
                    if (y > hi[g]) hi[g] = y;
                }
            for (int g = 0; g < 32; ++g) gn_flush_region(s[g], lo[g], hi[g], sum + b * 32 + g, mn + b * 32 + g, mx + b * 32 + g);
        }
    }
}

/* GroupNorm statistics of the planar epilogue k_epilogue (src/kernels.cu:70-95, 732-736): the output
 * [M x N] (N % 4 == 0) is cut into blocks of 1024 consecutive elements in row-major order (element
 * r * N + n); each block gathers per group n / (N / 32) the sum, min and max of its elements and
 * flushes them by the rule above into record (first row of the block / T) * 32 + group. With
 * (T * N) % 1024 == 0 no block holds two samples. */
void orc_gn_blocks(const int32_t* Y, int M, int N, int ldy, int T, int64_t* sum, int32_t* mn, int32_t* mx) {
    const int cg = N / 32;
    const int64_t total = (int64_t)M * N;
    for (int64_t e0 = 0; e0 < total; e0 += 1024) {
        const int b = (int)((e0 / N) / T);
        int64_t s[32];
        int32_t lo[32], hi[32];
        for (int g = 0; g < 32; ++g) { s[g] = 0; lo[g] = INT32_MAX; hi[g] = INT32_MIN; }
        for (int64_t i = e0; i < e0 + 1024 && i < total; ++i) {
            const int r = (int)(i / N), n = (int)(i % N);
            const int32_t y = Y[(size_t)r * ldy + n];
            const int g = n / cg;
            s[g] += y;
            if (y < lo[g]) lo[g] = y;
            if (y > hi[g]) hi[g] = y;
        }
        for (int g = 0; g < 32; ++g) gn_flush_region(s[g], lo[g], hi[g], sum + b * 32 + g, mn + b * 32 + g, mx + b * 32 + g);
    }
}

/* The EPI_QKV outputs from the plain output Y [M x 3C] (src/gemm_hl.cu:179-241): columns
 * [0, C) are q, [C, 2C) k, [2C, 3C) v, C = 64 * heads, row r = b * T + t. v is copied to V [M x C].
 * q and k are quantised per (row, head): e = row_exp(max |y| over the head's 64 values),
 * q16 = quant16_32(y, e), hi = q16 >> 8, lo = (q16 & 255) - 128, stored at row
 * (b * heads + head) * Tp + t of the [*, 64] planes, with e and the sums of hi, lo and q16 over the 64
 * values (the k_quant_heads layout, src/kernels.cu:611-631). Rows t >= T of the planes are not
 * written. */
void orc_qkv_heads(const int32_t* Y, int M, int ldy, int C, int heads, int T, int TpQ, int TpK,
                   int8_t* qhi, int8_t* qlo, int32_t* qe, int64_t* qhs, int64_t* qls, int64_t* qts,
                   int8_t* khi, int8_t* klo, int32_t* ke, int64_t* khs, int64_t* kls, int64_t* kts, int32_t* V) {
    for (int r = 0; r < M; ++r) {
        const int32_t* y = Y + (size_t)r * ldy;
        for (int c = 0; c < C; ++c) V[(size_t)r * C + c] = y[2 * C + c];
        const int b = r / T, t = r % T;
        for (int part = 0; part < 2; ++part) {
            const int Tp = part ? TpK : TpQ;
            int8_t* hp = part ? khi : qhi;
            int8_t* lp = part ? klo : qlo;
            for (int h = 0; h < heads; ++h) {
                const int32_t* v = y + part * C + 64 * h;
                int64_t m = 0;
                for (int d = 0; d < 64; ++d) {
                    const int64_t av = v[d] < 0 ? -(int64_t)v[d] : v[d];
                    if (av > m) m = av;
                }
                const int ee = orc_row_exp(m);
                const size_t gt = (size_t)(b * heads + h) * Tp + t;
                int64_t hs = 0, ls = 0, ts = 0;
                for (int d = 0; d < 64; ++d) {
                    const int32_t q = orc_quant16_32(v[d], ee);
                    int8_t hb, lb;
                    orc_split16(q, &hb, &lb);
                    hp[gt * 64 + d] = hb;
                    lp[gt * 64 + d] = lb;
                    hs += hb; ls += lb; ts += q;
                }
                (part ? ke : qe)[gt] = ee;
                (part ? khs : qhs)[gt] = hs;
                (part ? kls : qls)[gt] = ls;
                (part ? kts : qts)[gt] = ts;
            }
        }
    }
}

/* ------------------------------------------------------------------ the GEMMs */

/* One row of A as hi/lo planes. SRC_I8: src/gemm_hl.cu:87-97. SRC_X32: src/gemm_hl.cu:99-121
 * (e = row_exp(rowmax), q = quant16_32). SRC_CONV32: src/gemm_hl.cu:104-114 (implicit 3x3/pad-1
 * im2col, tap-major K, outside the image -> 0). SRC_I16 holds q = 256*hi + lo + 128 directly;
 * SRC_CONV16 is SRC_CONV32 on an int16 image. Columns k >= K are the value 0. */
int orc_a_row(const OrcGemm* g, int r, int8_t* hi, int8_t* lo, int32_t* e) {
    const int Kp = g->Kp;
    switch (g->src) {
    case ORC_SRC_I8:
        memcpy(hi, g->hi + (size_t)r * g->ld8, (size_t)Kp);
        memcpy(lo, g->lo + (size_t)r * g->ld8, (size_t)Kp);
        *e = g->e ? g->e[r] : 0;
        return 0;
    case ORC_SRC_I16: {
        const int16_t* q = g->q16 + (size_t)r * g->ld16;
        for (int k = 0; k < Kp; ++k) { const int32_t v = k < g->K ? q[k] : 0; hi[k] = qhi(v); lo[k] = qlo(v); }
        *e = g->e ? g->e[r] : 0;
        return 0;
    }
    case ORC_SRC_X32: {
        const int ee = orc_row_exp(g->xrowmax[r]);
        const int32_t* x = g->x + (size_t)r * g->ldx;
        for (int k = 0; k < Kp; ++k) { const int32_t q = k < g->K ? orc_quant16_32(x[k], ee) : 0; hi[k] = qhi(q); lo[k] = qlo(q); }
        *e = ee;
        return 0;
    }
    case ORC_SRC_CONV32:
    case ORC_SRC_CONV16: {
        const int C = g->C, HoWo = g->Ho * g->Wo;
        const int b = r / HoWo, p = r % HoWo, oy = p / g->Wo, ox = p % g->Wo;
        const int ee = g->e ? g->e[r] : 0;
        for (int k = 0; k < Kp; ++k) {
            int32_t q = 0;
            if (k < g->K) {
                const int tap = k / C, c = k % C;
                const int iy = oy * g->stride - 1 + tap / 3, ix = ox * g->stride - 1 + tap % 3;
                if (iy >= 0 && iy < g->H && ix >= 0 && ix < g->W) {
                    const size_t at = (((size_t)b * g->H + iy) * g->W + ix) * C + c;
                    const int32_t x = g->src == ORC_SRC_CONV32 ? g->img[at] : (int32_t)g->img16[at];
                    q = orc_quant16_32(x, ee);
                }
            }
            hi[k] = qhi(q); lo[k] = qlo(q);
        }
        *e = ee;
        return 0;
    }
    default:
        return -1;
    }
}

/* Per-plane int32 dot products of one materialised row against columns [n0, n1) of W. |Chi|,|Clo|
 * <= 2^14 * Kp, exact in int32 for Kp < 2^17 (src/gemm_hl.cu:138-161 computes the same sums). */
static void row_planes(const int8_t* hi, const int8_t* lo, const int8_t* W, int ldw, int Kp, int n0, int n1,
                       int32_t* chi, int32_t* clo) {
    int n = n0;
    for (; n + 4 <= n1; n += 4) {
        const int8_t* w0 = W + (size_t)n * ldw;
        const int8_t* w1 = w0 + ldw;
        const int8_t* w2 = w1 + ldw;
        const int8_t* w3 = w2 + ldw;
        int32_t h0 = 0, h1 = 0, h2 = 0, h3 = 0, l0 = 0, l1 = 0, l2 = 0, l3 = 0;
        for (int k = 0; k < Kp; ++k) {
            const int32_t a = hi[k], b = lo[k];
            h0 += a * w0[k]; h1 += a * w1[k]; h2 += a * w2[k]; h3 += a * w3[k];
            l0 += b * w0[k]; l1 += b * w1[k]; l2 += b * w2[k]; l3 += b * w3[k];
        }
        chi[n] = h0; chi[n + 1] = h1; chi[n + 2] = h2; chi[n + 3] = h3;
        clo[n] = l0; clo[n + 1] = l1; clo[n + 2] = l2; clo[n + 3] = l3;
    }
    for (; n < n1; ++n) {
        const int8_t* w = W + (size_t)n * ldw;
        int32_t h = 0, l = 0;
        for (int k = 0; k < Kp; ++k) { h += hi[k] * w[k]; l += lo[k] * w[k]; }
        chi[n] = h; clo[n] = l;
    }
}

static int check_gemm(const OrcGemm* g) {
    if (g->Kp <= 0 || g->Mreal < 0 || g->Nreal < 0) return -1;
    if (g->epi == ORC_EPI_GEGLU && (g->Nreal & 1)) return -1;
    if (g->src < 0 || g->src > ORC_SRC_CONV16) return -1;
    return 0;
}

/* The fused-epilogue GEMM of src/gemm_hl.cu:65-310 for EPI_PLAIN (+residual, +rowmax), EPI_GELU,
 * EPI_SPLIT3 and EPI_GEGLU (+rowmax), for output rows [r0, r1). Column pairs follow :269-297. */
int orc_gemm_hl_rows(const OrcGemm* g, int r0, int r1) {
    if (check_gemm(g)) return -1;
    if (r1 <= 0 || r1 > g->Mreal) r1 = g->Mreal;
    if (r0 < 0) r0 = 0;
    const int Kp = g->Kp, N = g->Nreal;
    int bad = 0;
#pragma omp parallel num_threads(orc_get_threads()) reduction(| : bad)
    {
        int8_t* hi = (int8_t*)malloc((size_t)Kp);
        int8_t* lo = (int8_t*)malloc((size_t)Kp);
        int32_t* chi = (int32_t*)malloc(sizeof(int32_t) * (size_t)(N > 0 ? N : 1));
        int32_t* clo = (int32_t*)malloc(sizeof(int32_t) * (size_t)(N > 0 ? N : 1));
#pragma omp for schedule(dynamic, 16)
        for (int r = r0; r < r1; ++r) {
            int32_t er = 0;
            if (orc_a_row(g, r, hi, lo, &er)) { bad = 1; continue; }
            row_planes(hi, lo, g->w, g->ldw, Kp, 0, N, chi, clo);
            uint32_t mx = 0;
            if (g->epi == ORC_EPI_GEGLU) {
                for (int n = 0; n + 1 < N; n += 2) {
                    const int32_t a = orc_epi1(chi[n], clo[n], g->cst + 4 * n, er);
                    const int32_t gg = orc_epi1(chi[n + 1], clo[n + 1], g->cst + 4 * (n + 1), er);
                    const int32_t v = orc_geglu(a, gg, g->Lphi);
                    g->Y[(size_t)r * g->ldy + (n >> 1)] = v;
                    const uint32_t u = uabs32(v); mx = u > mx ? u : mx;
                }
            } else if (g->epi == ORC_EPI_SPLIT3) {
                for (int n = 0; n < N; ++n) {
                    const int part = n >= 2 * g->Cs ? 2 : (n >= g->Cs ? 1 : 0);
                    int32_t* Y = part == 0 ? g->Y : (part == 1 ? g->Y1 : g->Y2);
                    Y[(size_t)r * g->Cs + (n - part * g->Cs)] = orc_epi1(chi[n], clo[n], g->cst + 4 * n, er);
                }
            } else {
                for (int n = 0; n < N; ++n) {
                    int32_t y = orc_epi1(chi[n], clo[n], g->cst + 4 * n, er);
                    if (g->epi == ORC_EPI_GELU) y = orc_gelu(y, g->Lphi);
                    if (g->residual) y = (int32_t)orc_sat32((int64_t)y + g->residual[(size_t)r * g->ldy + n]);
                    g->Y[(size_t)r * g->ldy + n] = y;
                    const uint32_t u = uabs32(y); mx = u > mx ? u : mx;
                }
            }
            if (g->rowmax && g->epi != ORC_EPI_SPLIT3 && mx > g->rowmax[r]) g->rowmax[r] = mx;
        }
        free(hi); free(lo); free(chi); free(clo);
    }
    return bad ? -1 : 0;
}

int orc_gemm_hl(const OrcGemm* g) { return orc_gemm_hl_rows(g, 0, g->Mreal); }

int orc_gemm_planes(const OrcGemm* g, int32_t* Chi, int32_t* Clo, int ldc) {
    if (check_gemm(g)) return -1;
    const int Kp = g->Kp;
    int bad = 0;
#pragma omp parallel num_threads(orc_get_threads()) reduction(| : bad)
    {
        int8_t* hi = (int8_t*)malloc((size_t)Kp);
        int8_t* lo = (int8_t*)malloc((size_t)Kp);
#pragma omp for schedule(dynamic, 16)
        for (int r = 0; r < g->Mreal; ++r) {
            int32_t er;
            if (orc_a_row(g, r, hi, lo, &er)) { bad = 1; continue; }
            row_planes(hi, lo, g->w, g->ldw, Kp, 0, g->Nreal, Chi + (size_t)r * ldc, Clo + (size_t)r * ldc);
        }
        free(hi); free(lo);
    }
    return bad ? -1 : 0;
}

/* Gemm::run: C[M,N] = A[M,K] * W[N,K]^T, int32 accumulate (src/gemm.cu:22-29), strided batch (:30-35) */
void orc_i8gemm(const int8_t* A, int lda, long long sA, const int8_t* W, int ldw, long long sW,
                int32_t* C, int ldc, long long sC, int M, int N, int K, int batch) {
    for (int bt = 0; bt < batch; ++bt) {
        const int8_t* Ab = A + bt * sA;
        const int8_t* Wb = W + bt * sW;
        int32_t* Cb = C + bt * sC;
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
        for (int m = 0; m < M; ++m) {
            const int8_t* a = Ab + (size_t)m * lda;
            for (int n = 0; n < N; ++n) {
                const int8_t* w = Wb + (size_t)n * ldw;
                int32_t s = 0;
                for (int k = 0; k < K; ++k) s += a[k] * w[k];
                Cb[(size_t)m * ldc + n] = s;
            }
        }
    }
}

/* ------------------------------------------------------------------ weight preparation */

/* DevModel::load: src/engine.cu:26-44. W [N x K] (K = 9C for a 3x3 conv in PyTorch's c-major
 * order) -> wout [Np x Kp] zero padded, tap-major for convs (kk = (k%9)*C + k/9), cst[n] = {m, s, b,
 * wsum over the real K}; pad columns get {1, 0, 0, 0} (src/engine.cu:29). */
void orc_prep_weight(const int8_t* w, int N, int K, int conv3, const int32_t* m, const int32_t* s,
                     const int32_t* b, int Np, int Kp, int8_t* wout, int32_t* cst_out) {
    const int C = conv3 ? K / 9 : 0;
    memset(wout, 0, (size_t)Np * Kp);
    for (int n = 0; n < Np; ++n) {
        int32_t* c = cst_out + 4 * n;
        if (n >= N) { c[0] = 1; c[1] = 0; c[2] = 0; c[3] = 0; continue; }
        int64_t sum = 0;
        for (int k = 0; k < K; ++k) {
            const int kk = conv3 ? (k % 9) * C + k / 9 : k;
            wout[(size_t)n * Kp + kk] = w[(size_t)n * K + k];
            sum += w[(size_t)n * K + k];
        }
        c[0] = m[n]; c[1] = s[n]; c[2] = b[n]; c[3] = (int32_t)sum;
    }
}

/* mergeLins(interleave = true) with two parts: src/engine.cu:71-101. wa, wg [N x Kp] (first N rows
 * used), ca, cg [4N]. wout [Np x Kp] with Np = align64(2N); row 2i = a_i, 2i+1 = g_i. */
void orc_interleave2(const int8_t* wa, const int32_t* ca, const int8_t* wg, const int32_t* cg, int N, int Kp,
                     int8_t* wout, int32_t* cout) {
    const int Np = (2 * N + 63) / 64 * 64;
    memset(wout, 0, (size_t)Np * Kp);
    for (int n = 0; n < Np; ++n) { cout[4 * n] = 1; cout[4 * n + 1] = 0; cout[4 * n + 2] = 0; cout[4 * n + 3] = 0; }
    for (int i = 0; i < N; ++i) {
        memcpy(wout + (size_t)(2 * i) * Kp, wa + (size_t)i * Kp, (size_t)Kp);
        memcpy(wout + (size_t)(2 * i + 1) * Kp, wg + (size_t)i * Kp, (size_t)Kp);
        memcpy(cout + 8 * i, ca + 4 * i, 16);
        memcpy(cout + 8 * i + 4, cg + 4 * i, 16);
    }
}

/* ------------------------------------------------------------------ integer normalisations */

/* src/intops.cuh:18 */
int64_t orc_floor_div(int64_t a, int64_t b) {
    int64_t q = a / b;
    if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
    return q;
}

/* src/intops.cuh:51-56: floor(sqrt(v)) by a double estimate and integer corrections */
int64_t orc_isqrt(int64_t v) {
    if (v <= 0) return 0;
    int64_t s = (int64_t)sqrt((double)v);
    while (s > 0 && s * s > v) --s;
    while ((s + 1) * (s + 1) <= v) ++s;
    return s;
}

/* src/kernels.cu:173 */
void orc_gn_init(OrcGnStat* gs, int cnt) {
    for (int i = 0; i < cnt; ++i) { gs[i].sum = 0; gs[i].mn = INT32_MAX; gs[i].mx = INT32_MIN; gs[i].ss = 0; }
}

/* src/kernels.cu:175-183: sum, min and max over rows t < T and channels [g cg, (g + 1) cg) of sample b */
void orc_gn_stats1(const int32_t* X, int B, int T, int C, int groups, OrcGnStat* gs) {
    const int cg = C / groups;
    for (int b = 0; b < B; ++b)
        for (int g = 0; g < groups; ++g) {
            OrcGnStat* s = gs + b * groups + g;
            for (int t = 0; t < T; ++t)
                for (int j = 0; j < cg; ++j) {
                    const int32_t v = X[((size_t)b * T + t) * C + g * cg + j];
                    s->sum += v;
                    if (v < s->mn) s->mn = v;
                    if (v > s->mx) s->mx = v;
                }
        }
}

/* src/kernels.cu:185-192 */
void orc_gn_fin1(OrcGnStat* gs, int cnt, int64_t n) {
    for (int i = 0; i < cnt; ++i) {
        OrcGnStat* s = gs + i;
        s->mean = orc_floor_div(s->sum + n / 2, n);
        const int64_t a = (int64_t)s->mx - s->mean, b = s->mean - (int64_t)s->mn;
        const int e = orc_row_exp(a > b ? a : b) - 5;
        s->e = e > 0 ? e : 0;
    }
}

/* src/kernels.cu:193-201: ss += dd^2 with dd the rounding shift of x - mean by e (no saturation) */
void orc_gn_stats2(const int32_t* X, int B, int T, int C, int groups, OrcGnStat* gs) {
    const int cg = C / groups;
    for (int b = 0; b < B; ++b)
        for (int g = 0; g < groups; ++g) {
            OrcGnStat* s = gs + b * groups + g;
            const int e = s->e;
            for (int t = 0; t < T; ++t)
                for (int j = 0; j < cg; ++j) {
                    const int64_t d = (int64_t)X[((size_t)b * T + t) * C + g * cg + j] - s->mean;
                    const int64_t dd = e ? ((d >> e) + ((d >> (e - 1)) & 1)) : d;
                    s->ss += dd * dd;
                }
        }
}

/* src/kernels.cu:203-210 */
void orc_gn_fin2(OrcGnStat* gs, int cnt, int64_t n, int64_t den) {
    for (int i = 0; i < cnt; ++i) {
        OrcGnStat* s = gs + i;
        const int64_t var = orc_floor_div(s->ss, n);
        const int sh = 32 - 2 * s->e;
        const int64_t one = sh >= 0 ? (INT64_C(1) << sh) : 0;
        const int64_t eps = orc_floor_div(one + den / 2, den);
        s->sd = orc_isqrt((int64_t)((uint64_t)(var + eps) << 16));
    }
}

/* the normalised Q16 value floor(((x - mean) 2^(25 - e) + sd) / (2 sd)) (src/kernels.cu:217,296); 0 for sd = 0 */
static int64_t orc_gn_norm(int32_t x, const OrcGnStat* s) {
    if (s->sd == 0) return 0;
    const int64_t d = (int64_t)x - s->mean;
    return orc_floor_div((int64_t)((uint64_t)d << (25 - s->e)) + s->sd, 2 * s->sd);
}

/* src/kernels.cu:211-219 */
void orc_gn_apply(const int32_t* X, int B, int T, int C, int groups, const OrcGnStat* gs, const int64_t* g, const int64_t* beta, int32_t* Y) {
    const int cg = C / groups;
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t)
            for (int c = 0; c < C; ++c) {
                const size_t i = ((size_t)b * T + t) * C + c;
                const int64_t yy = orc_gn_norm(X[i], gs + b * groups + c / cg);
                Y[i] = (int32_t)orc_sat32(orc_rshr((int64_t)((uint64_t)yy * (uint64_t)g[c]), 16) + beta[c]);
            }
}

/* quant_row_out of one row (src/kernels.cu:317-331): e = row_exp(max |v|), q = quant16_32, pads (0, -128) */
static void orc_row_view(const int32_t* v, int C, int8_t* h, int8_t* l, int32_t* e, int Kp) {
    uint32_t m = 0;
    for (int c = 0; c < C; ++c) {
        const uint32_t a = v[c] < 0 ? (uint32_t)(-(int64_t)v[c]) : (uint32_t)v[c];
        if (a > m) m = a;
    }
    const int ee = orc_row_exp(m);
    *e = ee;
    for (int c = 0; c < Kp; ++c) {
        const int32_t q = c < C ? orc_quant16_32(v[c], ee) : 0;
        h[c] = (int8_t)(q >> 8);
        l[c] = (int8_t)((q & 255) - 128);
    }
}

/* src/kernels.cu:287-305 */
void orc_gn_apply_row(const int32_t* X, int B, int T, int C, int groups, const OrcGnStat* gs, const int32_t* g, const int32_t* beta,
                      const int32_t* Lsig, int32_t* Y, uint32_t* pm, int8_t* hi, int8_t* lo, int32_t* e, int Kp) {
    const int cg = C / groups;
    int32_t* v = (int32_t*)malloc((size_t)C * sizeof(int32_t));
    for (int row = 0; row < B * T; ++row) {
        const int b = row / T;
        uint32_t m = 0;
        for (int c = 0; c < C; ++c) {
            const int64_t yy = orc_gn_norm(X[(size_t)row * C + c], gs + b * groups + c / cg);
            int64_t y = orc_sat32(orc_rshr((int64_t)((uint64_t)yy * (uint64_t)(int64_t)g[c]), 16) + beta[c]);
            if (Lsig) y = orc_sat32(orc_rshr(y * orc_lut16i(y, Lsig), 16));
            v[c] = (int32_t)y;
            const uint32_t a = y < 0 ? (uint32_t)(-y) : (uint32_t)y;
            if (a > m) m = a;
        }
        if (hi) {
            orc_row_view(v, C, hi + (size_t)row * Kp, lo + (size_t)row * Kp, e + row, Kp);
        } else {
            memcpy(Y + (size_t)row * C, v, (size_t)C * sizeof(int32_t));
            if (pm) pm[row] = m;
        }
    }
    free(v);
}

/* the LayerNorm statistics of one row (src/kernels.cu:224-238): mean, the shift ex, sd */
static void orc_lnorm_stats(const int32_t* x, int C, int64_t den, int64_t* mean, int* ex, int64_t* sd) {
    int64_t sum = 0;
    int32_t mn = INT32_MAX, mx = INT32_MIN;
    for (int c = 0; c < C; ++c) { sum += x[c]; if (x[c] < mn) mn = x[c]; if (x[c] > mx) mx = x[c]; }
    const int64_t n = C;
    *mean = orc_floor_div(sum + n / 2, n);
    const int64_t a = (int64_t)mx - *mean, b = *mean - (int64_t)mn;
    const int e = orc_row_exp(a > b ? a : b) - 5;
    *ex = e > 0 ? e : 0;
    int64_t ss = 0;
    for (int c = 0; c < C; ++c) {
        const int64_t dd = orc_rshr((int64_t)x[c] - *mean, *ex);
        ss += dd * dd;
    }
    const int64_t var = orc_floor_div(ss, n);
    const int shb = 32 - 2 * *ex;
    const int64_t one = shb >= 0 ? (INT64_C(1) << shb) : 0;
    const int64_t eps = orc_floor_div(one + den / 2, den);
    *sd = orc_isqrt((int64_t)((uint64_t)(var + eps) << 16));
}

static int64_t orc_lnorm_value(int32_t x, int64_t mean, int ex, int64_t sd, int64_t g, int64_t beta) {
    const int64_t yy = sd ? orc_floor_div((int64_t)((uint64_t)((int64_t)x - mean) << (25 - ex)) + sd, 2 * sd) : 0;
    return orc_sat32(orc_rshr((int64_t)((uint64_t)yy * (uint64_t)g), 16) + beta);
}

/* src/kernels.cu:221-246 */
void orc_lnorm(const int32_t* X, int M, int C, const int64_t* g, const int64_t* beta, int64_t den, int32_t* Y) {
    for (int row = 0; row < M; ++row) {
        const int32_t* x = X + (size_t)row * C;
        int64_t mean, sd;
        int ex;
        orc_lnorm_stats(x, C, den, &mean, &ex, &sd);
        for (int c = 0; c < C; ++c) Y[(size_t)row * C + c] = (int32_t)orc_lnorm_value(x[c], mean, ex, sd, g[c], beta[c]);
    }
}

/* src/kernels.cu:349-390 */
void orc_lnorm_q(const int32_t* X, int M, int C, const int32_t* g, const int32_t* beta, int64_t den, int8_t* hi, int8_t* lo,
                 int32_t* e, int Kp) {
    int32_t* v = (int32_t*)malloc((size_t)C * sizeof(int32_t));
    for (int row = 0; row < M; ++row) {
        const int32_t* x = X + (size_t)row * C;
        int64_t mean, sd;
        int ex;
        orc_lnorm_stats(x, C, den, &mean, &ex, &sd);
        for (int c = 0; c < C; ++c) v[c] = (int32_t)orc_lnorm_value(x[c], mean, ex, sd, g[c], beta[c]);
        orc_row_view(v, C, hi + (size_t)row * Kp, lo + (size_t)row * Kp, e + row, Kp);
    }
    free(v);
}

/* ------------------------------------------------------------------ attention */

/* ---------------------------------------------------------------- elementwise (src/kernels.cu:536-561)
 * One element at a time in the reference's order, with its primitives: act_k, geglu_k, add_k,
 * concat_k (+ the gnacc per-block records) and upsample2_k. */

/* :537 act_k: x = sat32(rshr(x lut16i(x, L), 16)) */
void orc_act(int32_t* X, size_t n, const int32_t* L) {
    for (size_t i = 0; i < n; ++i) {
        const int64_t x = X[i];
        X[i] = (int32_t)orc_sat32(orc_rshr(x * orc_lut16i(x, L), 16));
    }
}

/* :538-542 geglu_k: a = sat32(rshr(a sat32(rshr(g lut16i(g, L), 16)), 16)) */
void orc_geglu_n(int32_t* A, const int32_t* G, size_t n, const int32_t* L) {
    for (size_t i = 0; i < n; ++i) A[i] = orc_geglu(A[i], G[i], L);
}

/* :543 add_k: x = sat32(x + y) */
void orc_add(int32_t* X, const int32_t* Y, size_t n) {
    for (size_t i = 0; i < n; ++i) X[i] = (int32_t)orc_sat32((int64_t)X[i] + Y[i]);
}

/* :544-556 concat_k: element i of out (row i / Co, column i % Co) from A or B. With gs, the block of
 * 256 consecutive elements i (blockDim = NT = 256, :9) gathers per group c / (Co / 32) the sum, min
 * and max of its live elements (gnacc_add, :66) and flushes each group whose min is not INT_MAX to
 * record (first element's row / T) * 32 + group (gnacc_flush, :67-69). */
void orc_concat(const int32_t* A, int Ca, const int32_t* B, int Cb, int rows, int32_t* out, OrcGnStat* gs, int T) {
    const int Co = Ca + Cb;
    const size_t tot = (size_t)rows * Co;
    for (size_t i = 0; i < tot; ++i) {
        const size_t r = i / Co;
        const int c = (int)(i % Co);
        out[i] = c < Ca ? A[r * Ca + c] : B[r * Cb + (c - Ca)];
    }
    if (!gs) return;
    const int cg = Co >> 5;
    for (size_t b0 = 0; b0 < tot; b0 += 256) {
        int64_t sum[32];
        int32_t mn[32], mx[32];
        for (int g = 0; g < 32; ++g) { sum[g] = 0; mn[g] = INT32_MAX; mx[g] = INT32_MIN; }
        for (size_t i = b0; i < b0 + 256 && i < tot; ++i) {
            const int g = (int)(i % Co) / cg;
            sum[g] += out[i];
            if (out[i] < mn[g]) mn[g] = out[i];
            if (out[i] > mx[g]) mx[g] = out[i];
        }
        const int sample = (int)(b0 / Co / T);
        for (int g = 0; g < 32; ++g) {
            OrcGnStat* s = gs + sample * 32 + g;
            gn_flush_region(sum[g], mn[g], mx[g], &s->sum, &s->mn, &s->mx);
        }
    }
}

/* :557-561 upsample2_k: out[b, y, x, c] = X[b, y / 2, x / 2, c] over the 2H x 2W image */
void orc_upsample2(const int32_t* X, int B, int H, int W, int C, int32_t* out) {
    const size_t tot = (size_t)B * 4 * H * W * C;
    for (size_t i = 0; i < tot; ++i) {
        const int c = (int)(i % C);
        size_t p = i / C;
        const int x = (int)(p % (2 * W));
        p /= 2 * W;
        const int y = (int)(p % (2 * H));
        const size_t b = p / (2 * H);
        out[i] = X[((b * H + (y >> 1)) * W + (x >> 1)) * C + c];
    }
}

/* src/kernels.cu:611-631 (quant_heads_k): each (g, t) row of 64 values, e = row_exp(max |x|),
 * quant16, split16, and the sums of hi, lo and q; rows t >= T are the value 0 = (0, -128) */
void orc_quant_heads(const int32_t* X, int B, int T, int C, int heads, int Tp, int8_t* hi, int8_t* lo, int32_t* e, int64_t* hs,
                     int64_t* ls, int64_t* tsum) {
    const int G = B * heads;
    for (int g = 0; g < G; ++g)
        for (int t = 0; t < Tp; ++t) {
            const size_t w = (size_t)g * Tp + t;
            if (t >= T) {
                for (int d = 0; d < 64; ++d) { hi[w * 64 + d] = 0; lo[w * 64 + d] = -128; }
                e[w] = 0; hs[w] = 0; ls[w] = -128 * 64; tsum[w] = 0;
                continue;
            }
            const int b = g / heads, h = g % heads;
            const int32_t* x = X + ((size_t)b * T + t) * C + h * 64;
            uint32_t m = 0;
            for (int d = 0; d < 64; ++d) {
                const uint32_t a = x[d] < 0 ? (uint32_t)(-(int64_t)x[d]) : (uint32_t)x[d];
                if (a > m) m = a;
            }
            const int ee = orc_row_exp(m);
            int64_t sh = 0, sl = 0, st = 0;
            for (int d = 0; d < 64; ++d) {
                const int64_t q = orc_quant16(x[d], ee);
                int8_t a, c;
                orc_split16(q, &a, &c);
                hi[w * 64 + d] = a; lo[w * 64 + d] = c;
                sh += a; sl += c; st += q;
            }
            e[w] = ee; hs[w] = sh; ls[w] = sl; tsum[w] = st;
        }
}

/* src/kernels.cu:799-805 */
void orc_quant_heads_pad(int G, int T, int Tp, int8_t* hi, int8_t* lo, int32_t* e, int64_t* hs, int64_t* ls, int64_t* tsum) {
    for (int g = 0; g < G; ++g)
        for (int t = T; t < Tp; ++t) {
            const size_t w = (size_t)g * Tp + t;
            for (int d = 0; d < 64; ++d) { hi[w * 64 + d] = 0; lo[w * 64 + d] = -128; }
            e[w] = 0; hs[w] = 0; ls[w] = -128 * 64; tsum[w] = 0;
        }
}

/* src/kernels.cu:632-672 (quant_v_max_k, quant_v_sum_k, quant_v_write_k): per (g, d) column of the
 * Tk rows: ev = row_exp(max |x|), vsum = sum of quant16; the transposed planes [g * 64 + d][t], the
 * value 0 for t >= Tk */
void orc_quant_v(const int32_t* X, int B, int Tk, int C, int heads, int Tkp, int8_t* vth, int8_t* vtl, int32_t* ev, int64_t* vsum) {
    const int G = B * heads;
    for (int g = 0; g < G; ++g) {
        const int b = g / heads, h = g % heads;
        for (int d = 0; d < 64; ++d) {
            uint32_t m = 0;
            for (int t = 0; t < Tk; ++t) {
                const int32_t v = X[((size_t)b * Tk + t) * C + h * 64 + d];
                const uint32_t a = v < 0 ? (uint32_t)(-(int64_t)v) : (uint32_t)v;
                if (a > m) m = a;
            }
            const int e = orc_row_exp(m);
            int64_t s = 0;
            for (int t = 0; t < Tkp; ++t) {
                const int64_t q = t < Tk ? orc_quant16(X[((size_t)b * Tk + t) * C + h * 64 + d], e) : 0;
                int8_t a, c;
                orc_split16(q, &a, &c);
                vth[((size_t)g * 64 + d) * Tkp + t] = a;
                vtl[((size_t)g * 64 + d) * Tkp + t] = c;
                s += q;
            }
            ev[g * 64 + d] = e;
            vsum[g * 64 + d] = s;
        }
    }
}

/* exp table lookup (src/attn.cu:85-91, src/kernels.cu:692-693): 0 for z >= 2^20, else the linear
 * interpolation between entries z >> 10 and (z >> 10) + 1 with fraction z & 1023 (floor shift) */
static int64_t orc_lutexp(uint32_t z, const int64_t* L) {
    if (z >= (16u << 16)) return 0;
    const int64_t i = z >> 10, f = z & 1023;
    return L[i] + (((L[i + 1] - L[i]) * f) >> 10);
}

/* The exact attention of src/attn.cu:1-6 and src/kernels.cu:673-722 from the int16 values of the
 * planes (q = 256 hi + lo + 128): per query row, S = sum_d Q_d K_d over the valid keys (k < Tk, and
 * k <= q when causal), s = rshr(S, 19 - eq - ek), mx = max s, E = lutexp(mx - s), sumE = sum E,
 * r = floor(2^62 / sumE) (0 for sumE <= 0), P = min(32767, (E r + 2^46) >> 47) (mod 2^64; 0 for
 * E <= 0), O_d = sum_k P_k V_kd, out = rshr(O, 15 - ev[d]). */
void orc_attention(const int8_t* qh, const int8_t* ql, const int32_t* eq, const int8_t* kh, const int8_t* kl, const int32_t* ek,
                   const int8_t* vth, const int8_t* vtl, const int32_t* ev, int B, int heads, int Tq, int Tqp, int Tk, int Tkp,
                   int causal, const int64_t* Lexp, int C, int32_t* out, uint32_t* rowmax) {
    const int G = B * heads;
    #pragma omp parallel for schedule(dynamic) collapse(2)
    for (int g = 0; g < G; ++g) {
        for (int q = 0; q < Tq; ++q) {
            const int b = g / heads, h = g % heads;
            int32_t* s = (int32_t*)malloc(sizeof(int32_t) * (size_t)(Tk > 0 ? Tk : 1));
            int64_t* E = (int64_t*)malloc(sizeof(int64_t) * (size_t)(Tk > 0 ? Tk : 1));
            const size_t rq = (size_t)g * Tqp + q;
            int32_t mx = INT32_MIN;
            int nk = 0;
            for (int k = 0; k < Tk; ++k) {
                if (causal && k > q) break;
                const size_t rk = (size_t)g * Tkp + k;
                int64_t S = 0;
                for (int d = 0; d < 64; ++d) {
                    const int64_t qv = 256 * (int64_t)qh[rq * 64 + d] + ql[rq * 64 + d] + 128;
                    const int64_t kv = 256 * (int64_t)kh[rk * 64 + d] + kl[rk * 64 + d] + 128;
                    S += qv * kv;
                }
                s[k] = (int32_t)orc_rshr(S, 19 - (int64_t)eq[rq] - ek[rk]);
                if (s[k] > mx) mx = s[k];
                nk = k + 1;
            }
            int64_t sumE = 0;
            for (int k = 0; k < nk; ++k) { E[k] = orc_lutexp((uint32_t)mx - (uint32_t)s[k], Lexp); sumE += E[k]; }
            const uint64_t r = sumE > 0 ? (uint64_t)orc_floor_div(INT64_C(1) << 62, sumE) : 0;
            uint32_t am = 0;
            for (int d = 0; d < 64; ++d) {
                int64_t O = 0;
                for (int k = 0; k < nk; ++k) {
                    int64_t P = 0;
                    if (E[k] > 0) {
                        const uint64_t pp = ((uint64_t)E[k] * r + (UINT64_C(1) << 46)) >> 47;
                        P = pp > 32767 ? 32767 : (int64_t)pp;
                    }
                    const size_t iv = ((size_t)g * 64 + d) * Tkp + k;
                    O += P * (256 * (int64_t)vth[iv] + vtl[iv] + 128);
                }
                const int32_t o = (int32_t)orc_rshr(O, 15 - (int64_t)ev[g * 64 + d]);
                out[((size_t)b * Tq + q) * C + h * 64 + d] = o;
                const uint32_t a = o < 0 ? (uint32_t)(-(int64_t)o) : (uint32_t)o;
                if (a > am) am = a;
            }
            /* rows of one (b, q) come from `heads` groups: the max is taken under a lock */
            if (rowmax) {
                #pragma omp critical(orc_attention_rowmax)
                if (am > rowmax[(size_t)b * Tq + q]) rowmax[(size_t)b * Tq + q] = am;
            }
            free(s);
            free(E);
        }
    }
}

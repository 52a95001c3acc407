// The producers and epilogues of the reference's src/kernels.h (emanwrxsti/vela) that feed and
// finish the GEMM path, the integer GroupNorm / LayerNorm around it, and the exact attention with its
// operand producers, as drop-in meow:: functions over libvgemm.so (include/vgemm.h). The rest of
// src/kernels.h is not part of this library. Errors throw std::runtime_error.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "../vgemm.h"

namespace meow {

namespace detail {
inline void kcheck(int rc) {
    if (rc != VGEMM_OK) throw std::runtime_error(std::string(vgemm_last_error()));
}
}  // namespace detail

typedef int64_t i64;   // src/kernels.h:8
typedef unsigned int u32;

// src/kernels.h:9: the GroupNorm statistics record (same fields and layout as VgemmGnStat)
struct GnStat {
    int64_t sum;
    int mn, mx;
    int64_t mean;
    int e;
    int64_t ss, sd;
};
static_assert(sizeof(GnStat) == sizeof(VgemmGnStat), "GnStat layout");

// src/kernels.h:11-12
inline void k_quant_rows(hipStream_t st, const int32_t* X, int M, int K, int ldx, int8_t* hi, int8_t* lo, int32_t* e, int Kp) {
    detail::kcheck(vgemm_quant_rows(st, X, M, K, ldx, hi, lo, e, Kp));
}

// src/kernels.h:13-16 (gs: per-(sample, group) sum/min/max of Y, 32 groups, N % 32 == 0, (T*N) % 1024 == 0)
inline void k_epilogue(hipStream_t st, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int4* cst, const int32_t* e,
                       int32_t* Y, int ldy, const int32_t* residual = nullptr, GnStat* gs = nullptr, int T = 0) {
    detail::kcheck(vgemm_epilogue(st, Chi, Clo, M, N, ldc, reinterpret_cast<const int32_t*>(cst), e, Y, ldy, residual, gs, T));
}

// src/kernels.h:25 (src/kernels.cu:173)
inline void k_gn_init(hipStream_t st, GnStat* gs, int cnt) { detail::kcheck(vgemm_gn_init(st, gs, cnt)); }

// src/kernels.h:17-18
inline void k_pixmax(hipStream_t st, const int32_t* X, int rows, int C, uint32_t* pm) { detail::kcheck(vgemm_pixmax(st, X, rows, C, pm)); }

// src/kernels.h:19-21 (K index tap-major: tap*C + c, tap = 3*ky + kx, as src/test_im2col.cu:41 checks)
inline void k_im2col3(hipStream_t st, const int32_t* X, const uint32_t* pm, int B, int H, int W, int C, int stride, int8_t* hi, int8_t* lo,
                      int32_t* e, int Kp) {
    detail::kcheck(vgemm_im2col3(st, X, pm, B, H, W, C, stride, hi, lo, e, Kp));
}

// src/kernels.h:67-68
inline void k_epilogue_split(hipStream_t st, const int32_t* Chi, const int32_t* Clo, int M, int N, int ldc, const int4* cst, const int32_t* e,
                             int Cs, int32_t* Y0, int32_t* Y1, int32_t* Y2) {
    detail::kcheck(vgemm_epilogue_split(st, Chi, Clo, M, N, ldc, reinterpret_cast<const int32_t*>(cst), e, Cs, Y0, Y1, Y2));
}

// src/kernels.h:69-70
inline void k_epilogue_geglu_q(hipStream_t st, const int32_t* Chi, const int32_t* Clo, int M, int F, int ldc, const int4* cst,
                               const int32_t* e, const int32_t* Lphi, int8_t* hi, int8_t* lo, int32_t* eo, int Kp) {
    detail::kcheck(vgemm_epilogue_geglu_q(st, Chi, Clo, M, F, ldc, reinterpret_cast<const int32_t*>(cst), e, Lphi, hi, lo, eo, Kp));
}

// ---- integer normalisations (src/kernels.h:21-24,59-63,66-67); C % 4 == 0, C <= 2560
inline void k_gn_stats1(hipStream_t st, const int32_t* X, int B, int T, int C, int groups, GnStat* gs) {
    detail::kcheck(vgemm_gn_stats1(st, X, B, T, C, groups, gs));
}
inline void k_gn_fin1(hipStream_t st, GnStat* gs, int cnt, i64 n) { detail::kcheck(vgemm_gn_fin1(st, gs, cnt, n)); }
inline void k_gn_stats2(hipStream_t st, const int32_t* X, int B, int T, int C, int groups, i64 den, GnStat* gs) {
    detail::kcheck(vgemm_gn_stats2(st, X, B, T, C, groups, den, gs));
}
inline void k_gn_apply(hipStream_t st, const int32_t* X, int B, int T, int C, int groups, const GnStat* gs, const i64* g, const i64* beta, int32_t* Y) {
    detail::kcheck(vgemm_gn_apply(st, X, B, T, C, groups, gs, reinterpret_cast<const int64_t*>(g), reinterpret_cast<const int64_t*>(beta), Y));
}
inline void k_lnorm(hipStream_t st, const int32_t* X, int M, int C, const i64* g, const i64* beta, i64 den, int32_t* Y) {
    detail::kcheck(vgemm_lnorm(st, X, M, C, reinterpret_cast<const int64_t*>(g), reinterpret_cast<const int64_t*>(beta), den, Y));
}
inline void k_lnorm_q(hipStream_t st, const int32_t* X, int M, int C, const int32_t* g, const int32_t* beta, i64 den, int8_t* hi, int8_t* lo,
                      int32_t* e, int Kp) {
    detail::kcheck(vgemm_lnorm_q(st, X, M, C, g, beta, den, hi, lo, e, Kp));
}
inline void k_gn_apply_row(hipStream_t st, const int32_t* X, int B, int T, int C, int groups, const GnStat* gs, const int32_t* g, const int32_t* beta,
                           const int32_t* Lsig, int32_t* Y, uint32_t* pm, int8_t* hi, int8_t* lo, int32_t* e, int Kp) {
    detail::kcheck(vgemm_gn_apply_row(st, X, B, T, C, groups, gs, g, beta, Lsig, Y, pm, hi, lo, e, Kp));
}

// ---- attention (src/kernels.h:42-50,61,73-77)
inline void k_quant_heads(hipStream_t st, const int32_t* X, int B, int T, int C, int heads, int Tp, int8_t* hi, int8_t* lo, int32_t* e, i64* hs,
                          i64* ls, i64* tsum) {
    detail::kcheck(vgemm_quant_heads(st, X, B, T, C, heads, Tp, hi, lo, e, reinterpret_cast<int64_t*>(hs), reinterpret_cast<int64_t*>(ls),
                                     reinterpret_cast<int64_t*>(tsum)));
}
inline void k_quant_heads_pad(hipStream_t st, int G, int T, int Tp, int8_t* hi, int8_t* lo, int32_t* e, i64* hs, i64* ls, i64* tsum) {
    detail::kcheck(vgemm_quant_heads_pad(st, G, T, Tp, hi, lo, e, reinterpret_cast<int64_t*>(hs), reinterpret_cast<int64_t*>(ls),
                                         reinterpret_cast<int64_t*>(tsum)));
}
inline void k_quant_v(hipStream_t st, const int32_t* X, int B, int Tk, int C, int heads, int Tkp, int8_t* vt_hi, int8_t* vt_lo, int32_t* ev, i64* vsum,
                      uint32_t* scratch) {
    detail::kcheck(vgemm_quant_v(st, X, B, Tk, C, heads, Tkp, vt_hi, vt_lo, ev, reinterpret_cast<int64_t*>(vsum), scratch));
}
inline void k_fused_attention(hipStream_t st, const int8_t* qhi, const int8_t* qlo, const int32_t* eq, const i64* qhs, const i64* qls, const int8_t* khi,
                              const int8_t* klo, const int32_t* ek, const i64* ksum, const int8_t* vthi, const int8_t* vtlo, const int32_t* ev,
                              const i64* vsum, int B, int heads, int Tq, int Tqp, int Tk, int Tkp, bool causal, const i64* Lexp, int C, int32_t* gmx,
                              i64* gr, int32_t* out, uint32_t* rowmax = nullptr) {
    detail::kcheck(vgemm_fused_attention(st, qhi, qlo, eq, reinterpret_cast<const int64_t*>(qhs), reinterpret_cast<const int64_t*>(qls), khi, klo, ek,
                                         reinterpret_cast<const int64_t*>(ksum), vthi, vtlo, ev, reinterpret_cast<const int64_t*>(vsum), B, heads, Tq,
                                         Tqp, Tk, Tkp, causal ? 1 : 0, reinterpret_cast<const int64_t*>(Lexp), C, gmx, reinterpret_cast<int64_t*>(gr),
                                         out, rowmax));
}

// src/kernels.h:31-35: the elementwise kernels between the GEMMs
inline void k_act(hipStream_t st, int32_t* X, size_t n, const int32_t* L) { detail::kcheck(vgemm_act(st, X, n, L)); }
inline void k_geglu(hipStream_t st, int32_t* A, const int32_t* G, size_t n, const int32_t* Lphi) { detail::kcheck(vgemm_geglu(st, A, G, n, Lphi)); }
inline void k_add(hipStream_t st, int32_t* X, const int32_t* Y, size_t n) { detail::kcheck(vgemm_add(st, X, Y, n)); }
inline void k_concat(hipStream_t st, const int32_t* A, int Ca, const int32_t* B, int Cb, int rows, int32_t* out, GnStat* gs = nullptr, int T = 0) {
    detail::kcheck(vgemm_concat(st, A, Ca, B, Cb, rows, out, gs, T));
}
inline void k_upsample2(hipStream_t st, const int32_t* X, int B, int H, int W, int C, int32_t* out) {
    detail::kcheck(vgemm_upsample2(st, X, B, H, W, C, out));
}

}  // namespace meow

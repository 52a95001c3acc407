// The producers and epilogues of the reference's src/kernels.h (emanwrxsti/vela) that feed and
// finish the GEMM path, and the integer GroupNorm / LayerNorm around it, as drop-in meow:: functions
// over libvgemm.so (include/vgemm.h). Attention and the rest of src/kernels.h are not part of this
// library. Errors throw std::runtime_error.
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

}  // namespace meow

// Drop-in replacement for the reference's src/gemm_hl.h (emanwrxsti/vela): the meow:: hi/lo GEMM
// surface, implemented over the C ABI of libvgemm.so (include/vgemm.h). Same names, argument
// order and meaning, with CUDA types replaced by HIP ones (hipStream_t, HIP's int4). Errors throw
// std::runtime_error with the library's message, as src/gemm_hl.cu:331,351,357 throw.
//
//   Y[r, n] = sat32(rshr((256*Ahi[r].W[n] + Alo[r].W[n] + 128*wsum[n]) * m[n], s[n] - e[r]) + b[n])
//             (+ residual, saturated)                                        (src/gemm_hl.h:1-3)
// A planes [Mp rows, ld lda] (Mp % 64 == 0), W [Np rows, ld ldw] (Np % 64 == 0), K = Kp (% 16 == 0).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "../vgemm.h"

namespace meow {

// src/gemm_hl.h:8-9 (plus the two int16 sources of this library)
enum GemmEpi { EPI_PLAIN = VGEMM_EPI_PLAIN, EPI_SPLIT3 = VGEMM_EPI_SPLIT3, EPI_GEGLU = VGEMM_EPI_GEGLU, EPI_GELU = VGEMM_EPI_GELU,
               EPI_QKV = VGEMM_EPI_QKV };
enum GemmSrc { SRC_I8 = VGEMM_SRC_I8, SRC_X32 = VGEMM_SRC_X32, SRC_CONV32 = VGEMM_SRC_CONV32, SRC_I16 = VGEMM_SRC_I16,
               SRC_CONV16 = VGEMM_SRC_CONV16 };

namespace detail {
inline void check(int rc) {
    if (rc != VGEMM_OK) throw std::runtime_error(std::string(vgemm_last_error()));
}
}  // namespace detail

// src/gemm_hl.h:12-17: the A operand, with the reference's default member values.
struct ASrc {
    int src = SRC_I8;
    const int8_t* hi = nullptr; const int8_t* lo = nullptr; int ld8 = 0; const int32_t* e = nullptr;
    const int32_t* x = nullptr; int ldx = 0; const uint32_t* rowmax = nullptr; int K = 0;
    const int32_t* img = nullptr; int H = 0, W = 0, C = 0, stride = 1, Ho = 0, Wo = 0;
    const int16_t* q16 = nullptr; int ld16 = 0;   // SRC_I16
    const int16_t* img16 = nullptr;               // SRC_CONV16
};

// src/gemm_hl.h:18-26: the epilogue (gnstat points at GnStat records of include/vela/kernels.h);
// ws/ws_bytes add an optional split-K workspace.
struct AEpi {
    int epi = EPI_PLAIN; int32_t* Y = nullptr; int ldy = 0; const int32_t* residual = nullptr;
    int Cs = 0; int32_t* Y1 = nullptr; int32_t* Y2 = nullptr; const int32_t* Lphi = nullptr;
    uint32_t* rowmax = nullptr;
    void* gnstat = nullptr; int gnT = 0;
    int heads = 0, T = 0, TpQ = 0, TpK = 0, C = 0;
    int8_t *qhi = nullptr, *qlo = nullptr, *khi = nullptr, *klo = nullptr; int32_t *qe = nullptr, *ke = nullptr;
    int64_t *qhs = nullptr, *qls = nullptr, *qts = nullptr, *khs = nullptr, *kls = nullptr, *kts = nullptr;
    void* ws = nullptr; size_t ws_bytes = 0;
};

// The int16 view of the output (vgemm_hl2_view; no counterpart in the reference's fused GEMM).
struct View {
    int8_t* hi = nullptr; int8_t* lo = nullptr; int32_t* e = nullptr; int ld = 0;
};

namespace detail {
inline VgemmASrc to_c(const ASrc& a) {
    VgemmASrc c;
    vgemm_asrc_init(&c);
    c.src = a.src; c.hi = a.hi; c.lo = a.lo; c.ld8 = a.ld8; c.e = a.e;
    c.x = a.x; c.ldx = a.ldx; c.rowmax = a.rowmax; c.K = a.K;
    c.img = a.img; c.H = a.H; c.W = a.W; c.C = a.C; c.stride = a.stride; c.Ho = a.Ho; c.Wo = a.Wo;
    c.q16 = a.q16; c.ld16 = a.ld16; c.img16 = a.img16;
    return c;
}
inline VgemmAEpi to_c(const AEpi& e) {
    VgemmAEpi c;
    vgemm_aepi_init(&c);
    c.epi = e.epi; c.Y = e.Y; c.ldy = e.ldy; c.residual = e.residual;
    c.Cs = e.Cs; c.Y1 = e.Y1; c.Y2 = e.Y2; c.Lphi = e.Lphi; c.rowmax = e.rowmax;
    c.gnstat = e.gnstat; c.gnT = e.gnT;
    c.heads = e.heads; c.T = e.T; c.TpQ = e.TpQ; c.TpK = e.TpK; c.C = e.C;
    c.qhi = e.qhi; c.qlo = e.qlo; c.khi = e.khi; c.klo = e.klo; c.qe = e.qe; c.ke = e.ke;
    c.qhs = e.qhs; c.qls = e.qls; c.qts = e.qts; c.khs = e.khs; c.kls = e.kls; c.kts = e.kts;
    c.ws = e.ws; c.ws_bytes = e.ws_bytes;
    return c;
}
}  // namespace detail

// src/gemm_hl.h:27 / src/gemm_hl.cu:350-370
inline void k_gemm_hl2(hipStream_t st, const ASrc& A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal, int Kp,
                       const int4* cst, const AEpi& E) {
    const VgemmASrc a = detail::to_c(A);
    const VgemmAEpi e = detail::to_c(E);
    detail::check(vgemm_hl2(st, &a, Mp, Mreal, W, ldw, Np, Nreal, Kp, reinterpret_cast<const int32_t*>(cst), &e));
}

// k_gemm_hl2 writing the int16 view of its output instead of Y (this library's extension)
inline void k_gemm_hl2_view(hipStream_t st, const ASrc& A, int Mp, int Mreal, const int8_t* W, int ldw, int Np, int Nreal, int Kp,
                            const int4* cst, const AEpi& E, const View& V) {
    const VgemmASrc a = detail::to_c(A);
    const VgemmAEpi e = detail::to_c(E);
    const VgemmView v{V.hi, V.lo, V.e, V.ld};
    detail::check(vgemm_hl2_view(st, &a, Mp, Mreal, W, ldw, Np, Nreal, Kp, reinterpret_cast<const int32_t*>(cst), &e, &v));
}

// src/gemm_hl.h:29 / src/gemm_hl.cu:335-349
inline void k_conv_e(hipStream_t st, const uint32_t* pm, int B, int H, int W, int stride, int32_t* e) {
    detail::check(vgemm_conv_e(st, pm, B, H, W, stride, e));
}

// src/gemm_hl.h:30-33 / src/gemm_hl.cu:371-376 (default arguments as the reference's)
inline void k_gemm_hl(hipStream_t st, const int8_t* Ahi, const int8_t* Alo, int lda, int Mp, int Mreal, const int8_t* W, int ldw, int Np,
                      int Nreal, int Kp, const int4* cst, const int32_t* e, int32_t* Y, int ldy, const int32_t* residual,
                      int epi = EPI_PLAIN, int Cs = 0, int32_t* Y1 = nullptr, int32_t* Y2 = nullptr, const int32_t* Lphi = nullptr) {
    detail::check(vgemm_hl(st, Ahi, Alo, lda, Mp, Mreal, W, ldw, Np, Nreal, Kp, reinterpret_cast<const int32_t*>(cst), e, Y, ldy, residual,
                           epi, Cs, Y1, Y2, Lphi));
}

// src/gemm_hl.h:34 / src/gemm_hl.cu:344
inline bool gemm_hl_supported(int Mp, int Np, int Kp) { return vgemm_supported(Mp, Np, Kp) != 0; }

// src/gemm_hl.h:35 / src/gemm_hl.cu:345: the process-wide tile override (-1 = automatic). Written
// by tests only. Values select this library's tiles: 0 = 128x128, 1 = 64x128, 2 = 128x64 (rows x
// columns); every value gives the same bytes.
struct GemmHlVariant {
    GemmHlVariant& operator=(int v) { vgemm_set_variant(v); return *this; }
    operator int() const { return vgemm_get_variant(); }
};
inline GemmHlVariant g_gemm_hl_variant;

}  // namespace meow

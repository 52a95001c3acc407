// Drop-in replacement for the reference's src/gemm.h (emanwrxsti/vela): meow::Gemm, the int8 x int8
// -> int32 GEMM that the reference runs through cuBLASLt (src/gemm.cu), here a gfx950 MFMA kernel of
// libvgemm.so (include/vgemm.h: vgemm_i8_*).
//   Row-major view: C[M, N] = A[M, K] * W[N, K]^T, strided batch (src/gemm.h:1-3, src/gemm.cu:22-35).
//   K % 16 == 0, N % 4 == 0, 16-byte aligned pointers.
// The reference's plan cache and eager autotune (src/gemm.cu:50-68) have no counterpart: the
// kernel is chosen per call from the shape, with nothing to warm up before graph capture.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "../vgemm.h"

namespace meow {

class Gemm {
public:
    Gemm() = default;
    Gemm(const Gemm&) = delete;
    Gemm& operator=(const Gemm&) = delete;

    // src/gemm.cu:7-12 (the workspace size is accepted; the kernel needs none)
    void init(int wsBytes) {
        if (h_) return;
        if (vgemm_i8_create(size_t(wsBytes > 0 ? wsBytes : 0), &h_) != VGEMM_OK) throw std::runtime_error(vgemm_last_error());
    }
    ~Gemm() {
        if (h_) vgemm_i8_destroy(h_);
    }
    // src/gemm.cu:41-70: throws where the reference throws ("no int8 GEMM for ...")
    void run(hipStream_t st, const int8_t* A, int lda, long long strideA, const int8_t* W, int ldw, long long strideW, int32_t* C, int ldc,
             long long strideC, int M, int N, int K, int batch = 1) {
        if (!h_) init(0);
        if (vgemm_i8_run(h_, st, A, lda, strideA, W, ldw, strideW, C, ldc, strideC, M, N, K, batch) != VGEMM_OK)
            throw std::runtime_error(vgemm_last_error());
    }

private:
    void* h_ = nullptr;
};

}  // namespace meow

// Device-side helpers shared by the vgemm kernels: exact integer primitives (restating
// src/intops.cuh:9-66 of the reference), buffer-resource loads and the parameter block.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef short s2 __attribute__((ext_vector_type(2)));
typedef long long i64;
typedef unsigned long long u64;

enum { SRC_I8 = 0, SRC_X32 = 1, SRC_CONV32 = 2, SRC_I16 = 3, SRC_CONV16 = 4 };
// EPI_PLAIN_GN: EPI_PLAIN that also accumulates GroupNorm statistics (a kernel instantiation of its
// own, so that the plain kernels carry none of its registers or code)
enum { EPI_PLAIN = 0, EPI_SPLIT3 = 1, EPI_GEGLU = 2, EPI_GELU = 3, EPI_QKV = 4, EPI_PLAIN_GN = 5, EPI_PARTIAL = 8, EPI_RAW = 9 };

// Per-(sample, group) GroupNorm statistics (src/kernels.h:9, same layout): the GEMM epilogue accumulates
// sum, mn and mx; the other fields belong to the normalisation that follows.
struct GnStat {
    long long sum;
    int mn, mx;
    long long mean;
    int e;
    long long ss, sd;
};

// A buffer offset that is outside every buffer this library builds (extents are checked < 2^31 on
// the host): a load from it returns zeros (the hardware range check of raw buffer loads).
constexpr unsigned OOB = 0x80000000u;
// Third descriptor word of a raw (untyped) buffer resource on gfx9-family GPUs.
constexpr int RSRC_WORD3 = 0x00020000;

struct GemmParams {
    // A operand
    const void* a0;            // hi plane / q16 / x / img / img16
    const void* a1;            // lo plane (SRC_I8)
    unsigned a0_bytes, a1_bytes;
    int lda;                   // row stride in elements (ld8 / ld16 / ldx)
    const int32_t* e;          // per-row shift (SRC_I8, SRC_I16, SRC_CONV*); may be null
    const uint32_t* xrowmax;   // SRC_X32
    const uint32_t* pm;        // convolution sources without e: per-pixel max |x| of the image (shift computed in-kernel)
    int K;                     // real K of the source (X32 / I16 / CONV)
    int H, W, C, stride, Ho, Wo;
    // weights
    const int8_t* w; unsigned w_bytes; int ldw;
    int Mreal, Nreal, Kp;
    const int4* cst;
    // epilogue
    int32_t* Y; int ldy; const int32_t* R;
    int Cs; int32_t* Y1; int32_t* Y2;
    const int32_t* Lphi; uint32_t* rowmax;
    int vec_store;             // output rows/pointers allow 16-byte stores
    unsigned y_bytes;          // byte extent of Y (and of the residual) from row 0 to the last output element
    // split-K partials: ws[(split * 2 + plane) * ws_rows + row][col], row stride ws_ld
    int ksplit, kper;
    int32_t* ws; int ws_rows, ws_ld;
    // tiling; colmajor: tile order over the XCDs (0: each XCD takes whole row stripes, every column
    // tile and K range of them; 1: each XCD takes (K range, column tile) groups, every row tile of them)
    int mtiles, ntiles, colmajor;
    // row-stationary kernel: blocks from index young0 on (0: none) raise their wave priority for their
    // first prio_chunks chunks (the blocks dispatched second to a CU, which otherwise yield issue
    // slots to the older block until it ends)
    int young0, prio_chunks;
    // wave priority by progress in prio_bands bands (0 or 1: off; tile and row-stationary kernels)
    int prio_bands;
    // strided batch (EPI_RAW)
    long long sA, sW, sC;
    // GroupNorm statistics of the output (EPI_PLAIN_GN): GnStat[sample * 32 + group], gnT rows per
    // sample, gathered and flushed per gnBM x gnBN region (the reference's tile, 64 or 128 each)
    GnStat* gnstat; int gnT, gnBM, gnBN;
    // EPI_QKV (src/gemm_hl.h:23-25): N = 3C, C = 64 heads; q/k head-quantised, v int32 into Y2
    int heads, qT, TpQ, TpK, qC;
    int8_t *qhi, *qlo, *khi, *klo;
    int32_t *qe, *ke;
    long long *qhs, *qls, *qts, *khs, *kls, *kts;
    // int16 view of the output (row-stationary kernel): hi/lo planes [rows x vld] written at each
    // chunk's running row exponent, with per-(32-column group, row) exponents vexp and correction
    // bits vmask (group-major) for the fix-up pass, and the row maxima vmax (all in the workspace)
    int8_t *vhi, *vlo; int vld; unsigned v_bytes;
    uint32_t* vmax; uint8_t* vexp; uint32_t* vmask; int vgroups;
};

// ---------------------------------------------------------------- exact integer primitives

__device__ __forceinline__ i64 sat32(i64 v) { return v < -2147483648LL ? -2147483648LL : (v > 2147483647LL ? 2147483647LL : v); }

// rshr: rounding right shift for s >= 0, saturating left shift for s < 0, result saturated to int32
// (src/intops.cuh:11-17). The rounding add wraps in 64 bits.
__device__ __forceinline__ i64 rshr(i64 v, i64 s) {
    if (s >= 0) {
        const int p = s > 62 ? 62 : int(s);
        const i64 t = i64(u64(v) + u64((1LL << p) >> 1));
        return sat32(t >> p);
    }
    const int neg = -s > 31 ? 31 : int(-s);
    const i64 lim = 1LL << (62 - neg);
    const i64 r = v < -lim ? -lim : (v > lim ? lim : v);
    return sat32(r * (1LL << neg));
}

// e = max(0, bitlen(m) - 15) (src/intops.cuh:37-38 for m < 2^32)
__device__ __forceinline__ int rowexp_u32(uint32_t m) { return m ? max(0, 32 - __clz(m) - 15) : 0; }

// quant16 of an int32 with e in [0,17] (src/intops.cuh:40-41)
__device__ __forceinline__ int quant16_32(int v, int e) {
    const int q = e ? ((v >> e) + ((v >> (e - 1)) & 1)) : v;
    return min(max(q, -32767), 32767);
}

// Interpolated Q16 table over [-16,16) (src/intops.cuh:42-50); 32-bit arithmetic wraps.
__device__ __forceinline__ int lut16i(i64 x, const int32_t* __restrict__ L) {
    const i64 z = x + (16LL << 16);
    if (z < 0) return 0;
    if (z >= (32LL << 16)) return 65536;
    const int i = int(z >> 10), f = int(z & 1023);
    const int a = L[i], b = L[i + 1];
    const int prod = int((unsigned(b) - unsigned(a)) * unsigned(f));
    return int(unsigned(a) + unsigned(prod >> 10));
}

// The exact epilogue of one element (src/gemm_hl.cu:40-43); acc * m wraps in 64 bits.
__device__ __forceinline__ int epi1_exact(int chi, int clo, int m, int s, int b, int wsum, int er) {
    const i64 acc = 256LL * chi + clo + 128LL * wsum;
    const i64 v = i64(u64(acc) * u64(i64(m)));
    return int(sat32(rshr(v, i64(s) - er) + b));
}

__device__ __forceinline__ int geglu_exact(int a, int g, const int32_t* __restrict__ L) {
    const i64 ge = sat32(rshr(i64(g) * lut16i(g, L), 16));
    return int(sat32(rshr(i64(a) * ge, 16)));
}

__device__ __forceinline__ int gelu_exact(int y, const int32_t* __restrict__ L) { return int(sat32(rshr(i64(y) * lut16i(y, L), 16))); }

__device__ __forceinline__ uint32_t uabs(int v) { return v < 0 ? uint32_t(-i64(v)) : uint32_t(v); }

// ---------------------------------------------------------------- fast exact epilogue pieces

// double -> int32 with saturation (v_cvt_i32_f64 clamps out-of-range values; the argument is
// always an integer-valued double here). Not volatile: the result depends on the operand alone.
// Inline asm still limits the scheduler around it, so code that overlaps MFMA latency with this
// conversion (the attention scores) clamps and converts in C++ instead.
__device__ __forceinline__ int cvt_sat(double x) {
    int r;
    asm("v_cvt_i32_f64 %0, %1" : "=v"(r) : "v"(x));
    return r;
}

__device__ __forceinline__ int add_sat(int a, int b) { return __builtin_elementwise_add_sat(a, b); }

// ---------------------------------------------------------------- buffer loads

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, RSRC_WORD3);
}

__device__ __forceinline__ v4i bload16(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// The same raw buffer resource as four words, for the asm DMA loads below.
__device__ __forceinline__ v4i make_rsrc_words(const void* base, unsigned bytes) {
    const unsigned long long a = reinterpret_cast<unsigned long long>(base);
    return v4i{int(unsigned(a)), int(unsigned(a >> 32) & 0xffffu), int(bytes), RSRC_WORD3};
}

// HBM -> LDS without registers: each lane's 16 bytes at buffer offset `off` + `soff` land at LDS
// byte address lds + 16 * lane (buffer_load_dwordx4 ... lds, M0 = LDS base). Lanes whose `off` is
// at or above 2^31 read zeros. Issued from asm so that the compiler does not wait for it before
// every barrier and LDS read: completion is awaited explicitly with vm_wait<N>() before the barrier
// that publishes the stage.
__device__ __forceinline__ void dma16(v4i rsrc, unsigned off, unsigned soff, unsigned lds) {
    // both are wave-uniform by construction; readfirstlane states it where the compiler cannot prove it
    soff = __builtin_amdgcn_readfirstlane(soff);
    lds = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" : : "v"(off), "s"(rsrc), "s"(soff), "s"(lds) : "memory");
}

template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// workgroup barrier that orders memory accesses in the compiler (no implicit waits)
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" : : : "memory"); }

// Wave priority by progress. Blocks resident on one CU start together, and the sequencer issues from
// the oldest wave first, so the block dispatched first runs ahead and the last one finishes alone.
// With PrioBands a block's steps [0, n) fall into `bands` equal bands, band b running at priority
// bands - 1 - b: a block that falls a band behind the others on its CU takes issue priority until it
// has caught up, so that the blocks of a CU end close together. The priority is back to 0 in the
// last band.
struct PrioBands {
    int b, next, n, bands;
    __device__ __forceinline__ static void set(int pr) {
        if (pr >= 3) __builtin_amdgcn_s_setprio(3);
        else if (pr == 2) __builtin_amdgcn_s_setprio(2);
        else if (pr == 1) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
    }
    __device__ __forceinline__ void init(int n_, int bands_) {
        n = n_;
        bands = min(bands_, 4);
        b = 0;
        next = bands > 1 ? (n + bands - 1) / bands : 0x7fffffff;
        if (bands > 1) set(bands - 1);
    }
    // at the start of step s (called for every s in order)
    __device__ __forceinline__ void step(int s) {
        if (s == next) {
            ++b;
            set(bands - 1 - b);
            next = b + 1 >= bands ? 0x7fffffff : ((b + 1) * n + bands - 1) / bands;
        }
    }
};

// LDS byte address of a pointer into __shared__ memory (generic -> local address-space cast)
__device__ __forceinline__ unsigned lds_addr(const void* p) {
    typedef const __attribute__((address_space(3))) char* lds_ptr;
    return unsigned(uintptr_t((lds_ptr)(p)));
}

}  // namespace vk

/*
 * Seeded synthetic inputs for the W8A16 GEMM configurations (host side, shared by tests and bench).
 *
 * Generator: splitmix64 seeds one xoshiro256** stream per 65536-element chunk (chunk j of a call with
 * seed S is seeded from S ^ (j * 0x9E3779B97F4A7C15)), so the output depends only on (seed, n) and
 * not on the number of threads. Distributions: Box-Muller Gaussian rounded to nearest, inverse-CDF
 * Laplace, and uniform integers by 64x64->128 multiply-shift. Values are clipped to [lo, hi].
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define CHUNK 65536

static uint64_t splitmix64(uint64_t* x) {
    uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

typedef struct { uint64_t s[4]; } xo256;

static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static inline uint64_t xo_next(xo256* g) {
    uint64_t* s = g->s;
    const uint64_t r = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
}

static void xo_seed(xo256* g, uint64_t seed, uint64_t chunk) {
    uint64_t x = seed ^ (chunk * 0x9E3779B97F4A7C15ull);
    for (int i = 0; i < 4; ++i) g->s[i] = splitmix64(&x);
}

/* uniform double in (0, 1] */
static inline double u01(xo256* g) { return ((double)(xo_next(g) >> 11) + 1.0) * (1.0 / 9007199254740992.0); }

static inline int64_t clampi(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

static inline int64_t uniform_int(xo256* g, int64_t lo, int64_t hi) {
    const uint64_t range = (uint64_t)(hi - lo) + 1;
    const unsigned __int128 p = (unsigned __int128)xo_next(g) * range;
    return lo + (int64_t)(uint64_t)(p >> 64);
}

static inline double gauss(xo256* g) {
    const double u1 = u01(g), u2 = u01(g);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static inline double laplace(xo256* g, double b) {
    const double u = u01(g) - 0.5;             /* (-0.5, 0.5] */
    const double a = fabs(u) * 2.0;            /* (0, 1] */
    const double mag = a >= 1.0 ? 0.0 : -b * log(1.0 - a);
    return u < 0 ? -mag : mag;
}

#define DEFINE_FILL(NAME, T, EXPR, ...)                                                         \
    void NAME(T* out, size_t n, uint64_t seed, __VA_ARGS__) {                                           \
        const int64_t nchunks = (int64_t)((n + CHUNK - 1) / CHUNK);                             \
        _Pragma("omp parallel for schedule(static)")                                            \
        for (int64_t j = 0; j < nchunks; ++j) {                                                 \
            xo256 g; xo_seed(&g, seed, (uint64_t)j);                                             \
            const size_t i0 = (size_t)j * CHUNK, i1 = i0 + CHUNK < n ? i0 + CHUNK : n;          \
            for (size_t i = i0; i < i1; ++i) out[i] = (T)(EXPR);                                  \
        }                                                                                       \
    }

/* Gaussian(sigma), rounded to nearest, clipped */
DEFINE_FILL(vdg_i16_gauss, int16_t, clampi(llround(sigma * gauss(&g)), lo, hi), double sigma, int lo, int hi)
DEFINE_FILL(vdg_i8_gauss, int8_t, clampi(llround(sigma * gauss(&g)), lo, hi), double sigma, int lo, int hi)
DEFINE_FILL(vdg_i32_gauss, int32_t, clampi(llround(sigma * gauss(&g)), lo, hi), double sigma, int64_t lo, int64_t hi)
/* Laplace(b), rounded to nearest, clipped */
DEFINE_FILL(vdg_i16_laplace, int16_t, clampi(llround(laplace(&g, b)), lo, hi), double b, int lo, int hi)
/* uniform integers in [lo, hi] */
DEFINE_FILL(vdg_i8_uniform, int8_t, uniform_int(&g, lo, hi), int lo, int hi)
DEFINE_FILL(vdg_i16_uniform, int16_t, uniform_int(&g, lo, hi), int lo, int hi)
DEFINE_FILL(vdg_i32_uniform, int32_t, uniform_int(&g, lo, hi), int64_t lo, int64_t hi)
/* signed values of a random bit width in [1, maxbits] (as src/test_gemm_hl.cu:16 draws its X) */
DEFINE_FILL(vdg_i32_bits, int32_t,
            (int32_t)({ const int bits = 1 + (int)uniform_int(&g, 0, maxbits - 1);
                        const uint64_t r = xo_next(&g);
                        (int64_t)(r & ((1ull << bits) - 1)) - (int64_t)(1ull << (bits - 1)); }),
            int maxbits)

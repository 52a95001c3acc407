// The C++ drop-in surface (include/vela/*.h) used the way the reference's own code uses
// src/gemm_hl.h, src/gemm.h and src/kernels.h: the structure of src/test_gemm_hl.cu:10-86 (the
// fused hi/lo GEMM against the planar path -- Gemm::run over the stacked [hi; lo] planes plus
// k_epilogue -- for every tile variant; SRC_X32 against k_quant_rows + SRC_I8; SRC_CONV32 against
// k_pixmax + k_conv_e + k_im2col3 + SRC_I8), plus an int64 host check of the planar path, a graph
// capture and replay (src/engine.cu:610-631), GroupNorm statistics (fused and planar, with
// k_gn_init), the EPI_QKV head layout, and the throwing error paths (src/gemm_hl.cu:351,357).
// With a model file as argv[1] (tests/golden/tiny_model.poisd), also meow::Poisd + meow::DevModel
// (src/poisd.h, src/engine.h) and GEMMs on the loaded linears. Needs a GPU; run by
// tests/test_gpu_dropin.py. Prints one line per check and exits non-zero on the
// first mismatch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "vela/gemm.h"
#include "vela/gemm_hl.h"
#include "vela/kernels.h"
#include "vela/model.h"
#include "vela/poisd.h"

#define HIP_OK(x)                                                                          \
    do {                                                                                   \
        hipError_t err_ = (x);                                                             \
        if (err_ != hipSuccess) {                                                          \
            std::fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(err_)); \
            std::exit(3);                                                                  \
        }                                                                                  \
    } while (0)

namespace {

template <class T>
struct Dev {
    T* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { HIP_OK(hipMalloc(&p, (count ? count : 1) * sizeof(T))); }
    Dev(const std::vector<T>& h) : Dev(h.size()) { put(h); }
    ~Dev() { (void)hipFree(p); }
    void put(const std::vector<T>& h) { HIP_OK(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice)); }
    std::vector<T> get() const {
        std::vector<T> h(n);
        HIP_OK(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
        return h;
    }
};

int fails = 0;
void expect(bool ok, const std::string& what) {
    std::printf("%s %s\n", ok ? "PASS" : "FAIL", what.c_str());
    std::fflush(stdout);
    if (!ok) ++fails;
}

int64_t sat32(int64_t v) { return v < INT32_MIN ? INT32_MIN : (v > INT32_MAX ? INT32_MAX : v); }
int64_t rshr(int64_t v, int64_t s) {
    if (s >= 0) {
        const int p = s > 62 ? 62 : int(s);
        return sat32(int64_t(uint64_t(v) + uint64_t((int64_t(1) << p) >> 1)) >> p);
    }
    const int n = -s > 31 ? 31 : int(-s);
    const int64_t lim = int64_t(1) << (62 - n);
    return sat32((v < -lim ? -lim : (v > lim ? lim : v)) * (int64_t(1) << n));
}

struct Problem {
    int Mp, M, Np, N, Kp;
    std::vector<int8_t> hi, lo, w;
    std::vector<int32_t> cst, e, res;
};

Problem make(std::mt19937& rng, int M, int N, int K) {
    Problem p;
    p.M = M; p.N = N; p.Mp = (M + 63) / 64 * 64; p.Np = (N + 63) / 64 * 64; p.Kp = (K + 15) / 16 * 16;
    p.hi.resize(size_t(p.Mp) * p.Kp); p.lo.resize(p.hi.size());
    for (auto& v : p.hi) v = int8_t(int(rng() % 256) - 128);
    for (auto& v : p.lo) v = int8_t(int(rng() % 256) - 128);
    p.w.assign(size_t(p.Np) * p.Kp, 0);
    p.cst.assign(size_t(p.Np) * 4, 0);
    for (int n = 0; n < p.Np; ++n) {
        int64_t ws = 0;
        if (n < N)
            for (int k = 0; k < p.Kp; ++k) {
                const int8_t v = int8_t(int(rng() % 255) - 127);
                p.w[size_t(n) * p.Kp + k] = v;
                ws += v;
            }
        // src/test_gemm_hl.cu:63: m in [2^14, 2^15), s in [20, 30), b in [-50000, 50000)
        p.cst[4 * n] = n < N ? int((1 << 14) + rng() % (1 << 14)) : 1;
        p.cst[4 * n + 1] = n < N ? int(20 + rng() % 10) : 0;
        p.cst[4 * n + 2] = n < N ? int(rng() % 100000) - 50000 : 0;
        p.cst[4 * n + 3] = int(ws);
    }
    p.e.resize(p.Mp);
    for (auto& v : p.e) v = int(rng() % 12);
    p.res.resize(size_t(M) * N);
    for (auto& v : p.res) v = int32_t(rng());
    return p;
}

// int64 host restatement of the planar path: acc = sum_k q*w with q = 256 hi + lo + 128
std::vector<int32_t> host_ref(const Problem& p, bool residual) {
    std::vector<int32_t> Y(size_t(p.M) * p.N);
    for (int r = 0; r < p.M; ++r)
        for (int n = 0; n < p.N; ++n) {
            int64_t acc = 0;
            for (int k = 0; k < p.Kp; ++k) {
                const int64_t q = 256 * int64_t(p.hi[size_t(r) * p.Kp + k]) + p.lo[size_t(r) * p.Kp + k] + 128;
                acc += q * p.w[size_t(n) * p.Kp + k];
            }
            const int32_t* c = &p.cst[4 * n];
            int64_t y = sat32(rshr(int64_t(uint64_t(acc) * uint64_t(int64_t(c[0]))), int64_t(c[1]) - p.e[r]) + c[2]);
            if (residual) y = sat32(y + p.res[size_t(r) * p.N + n]);
            Y[size_t(r) * p.N + n] = int32_t(y);
        }
    return Y;
}

void test_fused_vs_planar(hipStream_t st, std::mt19937& rng, int M, int N, int K) {
    Problem p = make(rng, M, N, K);
    // stacked [hi; lo] planes, as src/engine.cu:144 allocates them
    std::vector<int8_t> planes(p.hi);
    planes.insert(planes.end(), p.lo.begin(), p.lo.end());
    Dev<int8_t> A(planes), W(p.w);
    Dev<int32_t> cst(p.cst), e(p.e);
    const int8_t* dhi = A.p;
    const int8_t* dlo = A.p + size_t(p.Mp) * p.Kp;
    // planar path: Gemm::run over 2Mp rows, then k_epilogue with the residual aliasing Y
    meow::Gemm lt;
    lt.init(32 << 20);
    Dev<int32_t> C(size_t(2) * p.Mp * p.Np), Yp(p.res);
    lt.run(st, A.p, p.Kp, 0, W.p, p.Kp, 0, C.p, p.Np, 0, 2 * p.Mp, p.Np, p.Kp);
    meow::k_epilogue(st, C.p, C.p + size_t(p.Mp) * p.Np, p.M, p.N, p.Np, reinterpret_cast<const int4*>(cst.p), e.p, Yp.p, p.N, Yp.p);
    HIP_OK(hipStreamSynchronize(st));
    const std::vector<int32_t> planar = Yp.get();
    const std::string shape = std::to_string(M) + "x" + std::to_string(N) + "x" + std::to_string(K);
    expect(planar == host_ref(p, true), "planar Gemm::run + k_epilogue == int64 host " + shape);
    for (int v = -1; v < 3; ++v) {
        meow::g_gemm_hl_variant = v;
        Dev<int32_t> Y(p.res);
        meow::k_gemm_hl(st, dhi, dlo, p.Kp, p.Mp, p.M, W.p, p.Kp, p.Np, p.N, p.Kp, reinterpret_cast<const int4*>(cst.p), e.p, Y.p, p.N,
                        Y.p);
        HIP_OK(hipStreamSynchronize(st));
        expect(Y.get() == planar, "k_gemm_hl variant " + std::to_string(v) + " == planar " + shape);
    }
    meow::g_gemm_hl_variant = -1;
}

void test_x32(hipStream_t st, std::mt19937& rng) {
    const int M = 96, N = 64, K = 1024;   // src/test_gemm_hl.cu:16 shape class, random bit widths 1..31
    std::vector<int32_t> x(size_t(M) * K);
    std::vector<uint32_t> rmax(M, 0);
    for (int r = 0; r < M; ++r) {
        const int bits = 1 + int(rng() % 31);
        for (int k = 0; k < K; ++k) {
            const int64_t v = int64_t(rng() & ((1u << (bits - 1)) * 2 - 1)) - (int64_t(1) << (bits - 1));
            x[size_t(r) * K + k] = int32_t(v);
            const uint32_t a = uint32_t(v < 0 ? -v : v);
            if (a > rmax[r]) rmax[r] = a;
        }
    }
    Problem p = make(rng, M, N, K);
    Dev<int32_t> X(x), cst(p.cst), Y1(size_t(M) * N), Y2(size_t(M) * N), e(p.Mp);
    Dev<uint32_t> R(rmax);
    Dev<int8_t> W(p.w), hi(size_t(p.Mp) * p.Kp), lo(size_t(p.Mp) * p.Kp);
    meow::ASrc a;
    a.src = meow::SRC_X32; a.x = X.p; a.ldx = K; a.rowmax = R.p; a.K = K;
    meow::AEpi ep;
    ep.Y = Y1.p; ep.ldy = N;
    meow::k_gemm_hl2(st, a, p.Mp, M, W.p, p.Kp, p.Np, N, p.Kp, reinterpret_cast<const int4*>(cst.p), ep);
    meow::k_quant_rows(st, X.p, M, K, K, hi.p, lo.p, e.p, p.Kp);
    meow::k_gemm_hl(st, hi.p, lo.p, p.Kp, p.Mp, M, W.p, p.Kp, p.Np, N, p.Kp, reinterpret_cast<const int4*>(cst.p), e.p, Y2.p, N, nullptr);
    HIP_OK(hipStreamSynchronize(st));
    expect(Y1.get() == Y2.get(), "SRC_X32 == k_quant_rows + SRC_I8");
}

void test_conv32(hipStream_t st, std::mt19937& rng) {
    const int B = 2, H = 9, Wd = 7, C = 32, stride = 2;   // src/test_gemm_hl.cu:12 class, scaled down
    const int Ho = (H - 1) / stride + 1, Wo = (Wd - 1) / stride + 1, M = B * Ho * Wo, N = 128, K = 9 * C;
    std::vector<int32_t> img(size_t(B) * H * Wd * C);
    for (auto& v : img) v = int32_t(rng()) >> int(rng() % 24);
    Problem p = make(rng, M, N, K);
    Dev<int32_t> X(img), cst(p.cst), e(p.Mp), e2(p.Mp), Y1(size_t(M) * N), Y2(size_t(M) * N);
    Dev<uint32_t> pm(size_t(B) * H * Wd);
    Dev<int8_t> W(p.w), hi(size_t(p.Mp) * p.Kp), lo(size_t(p.Mp) * p.Kp);
    meow::k_pixmax(st, X.p, B * H * Wd, C, pm.p);
    meow::k_conv_e(st, pm.p, B, H, Wd, stride, e.p);
    meow::ASrc a;
    a.src = meow::SRC_CONV32; a.img = X.p; a.H = H; a.W = Wd; a.C = C; a.stride = stride; a.Ho = Ho; a.Wo = Wo; a.K = K; a.e = e.p;
    meow::AEpi ep;
    ep.Y = Y1.p; ep.ldy = N;
    meow::k_gemm_hl2(st, a, p.Mp, M, W.p, p.Kp, p.Np, N, p.Kp, reinterpret_cast<const int4*>(cst.p), ep);
    meow::k_im2col3(st, X.p, pm.p, B, H, Wd, C, stride, hi.p, lo.p, e2.p, p.Kp);
    meow::k_gemm_hl(st, hi.p, lo.p, p.Kp, p.Mp, M, W.p, p.Kp, p.Np, N, p.Kp, reinterpret_cast<const int4*>(cst.p), e2.p, Y2.p, N, nullptr);
    HIP_OK(hipStreamSynchronize(st));
    std::vector<int32_t> ea = e.get(), eb = e2.get();
    ea.resize(M); eb.resize(M);
    expect(ea == eb, "k_conv_e == k_im2col3 e");
    expect(Y1.get() == Y2.get(), "SRC_CONV32 == k_pixmax + k_im2col3 + SRC_I8");
}

void test_graph(hipStream_t st, std::mt19937& rng) {
    Problem p = make(rng, 200, 128, 320);
    Dev<int8_t> hi(p.hi), lo(p.lo), W(p.w);
    Dev<int32_t> cst(p.cst), e(p.e), Y(size_t(p.M) * p.N);
    HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    meow::k_gemm_hl(st, hi.p, lo.p, p.Kp, p.Mp, p.M, W.p, p.Kp, p.Np, p.N, p.Kp, reinterpret_cast<const int4*>(cst.p), e.p, Y.p, p.N, nullptr);
    hipGraph_t g;
    HIP_OK(hipStreamEndCapture(st, &g));
    hipGraphExec_t x;
    HIP_OK(hipGraphInstantiate(&x, g, nullptr, nullptr, 0));
    const std::vector<int32_t> want = host_ref(p, false);
    for (int i = 0; i < 3; ++i) {
        HIP_OK(hipMemset(Y.p, 0x5a, Y.n * sizeof(int32_t)));
        HIP_OK(hipGraphLaunch(x, st));
        HIP_OK(hipStreamSynchronize(st));
        expect(Y.get() == want, "graph replay " + std::to_string(i));
    }
    HIP_OK(hipGraphExecDestroy(x));
    HIP_OK(hipGraphDestroy(g));
}

// GroupNorm statistics (src/engine.cu:170-172, src/kernels.cu:63-95): the fused GEMM with gnstat and
// the planar Gemm::run + k_epilogue(..., gs, T) fill the same records, equal to a host reduction
void test_gnstat(hipStream_t st, std::mt19937& rng) {
    const int T = 64, B = 3, M = B * T, N = 320;
    Problem p = make(rng, M, N, 320);
    std::vector<int8_t> planes(p.hi);
    planes.insert(planes.end(), p.lo.begin(), p.lo.end());
    Dev<int8_t> A(planes), W(p.w);
    Dev<int32_t> cst(p.cst), e(p.e), Yf(p.res), Yp(p.res), C(size_t(2) * p.Mp * p.Np);
    Dev<meow::GnStat> gf(size_t(B) * 32), gp(size_t(B) * 32);
    meow::k_gn_init(st, gf.p, B * 32);
    meow::k_gn_init(st, gp.p, B * 32);
    meow::ASrc a;
    a.src = meow::SRC_I8; a.hi = A.p; a.lo = A.p + size_t(p.Mp) * p.Kp; a.ld8 = p.Kp; a.e = e.p;
    meow::AEpi ep;
    ep.Y = Yf.p; ep.ldy = N; ep.residual = Yf.p; ep.gnstat = gf.p; ep.gnT = T;
    meow::k_gemm_hl2(st, a, p.Mp, M, W.p, p.Kp, p.Np, N, p.Kp, reinterpret_cast<const int4*>(cst.p), ep);
    meow::Gemm lt;
    lt.init(0);
    lt.run(st, A.p, p.Kp, 0, W.p, p.Kp, 0, C.p, p.Np, 0, 2 * p.Mp, p.Np, p.Kp);
    meow::k_epilogue(st, C.p, C.p + size_t(p.Mp) * p.Np, M, N, p.Np, reinterpret_cast<const int4*>(cst.p), e.p, Yp.p, N, Yp.p, gp.p, T);
    HIP_OK(hipStreamSynchronize(st));
    const std::vector<int32_t> want = host_ref(p, true);
    expect(Yf.get() == want && Yp.get() == want, "GroupNorm GEMMs: Y == int64 host");
    const std::vector<meow::GnStat> sf = gf.get(), sp = gp.get();
    bool ok = true;
    for (int b = 0; b < B; ++b)
        for (int g = 0; g < 32; ++g) {
            int64_t sum = 0;
            int mn = INT32_MAX, mx = INT32_MIN;
            for (int r = b * T; r < (b + 1) * T; ++r)
                for (int n = g * (N / 32); n < (g + 1) * (N / 32); ++n) {
                    const int v = want[size_t(r) * N + n];
                    sum += v;
                    mn = v < mn ? v : mn;
                    mx = v > mx ? v : mx;
                }
            for (const auto* s : {&sf[b * 32 + g], &sp[b * 32 + g]}) ok = ok && s->sum == sum && s->mn == mn && s->mx == mx;
        }
    expect(ok, "GroupNorm records: fused gnstat == k_epilogue(gs) == host reduction");
}

// EPI_QKV (src/engine.cu:318-330): v and the head-quantised q/k against a host restatement of the
// k_quant_heads layout (src/kernels.cu:611-631) over the plain GEMM output
void test_qkv(hipStream_t st, std::mt19937& rng) {
    const int heads = 2, C = 64 * heads, T = 77, B = 2, M = B * T, TpQ = 128, TpK = 128;
    Problem p = make(rng, M, 3 * C, 320);
    Dev<int8_t> hi(p.hi), lo(p.lo), W(p.w);
    Dev<int32_t> cst(p.cst), e(p.e), V(size_t(M) * C);
    const size_t G = size_t(B) * heads * TpQ;
    Dev<int8_t> qhi(G * 64), qlo(G * 64), khi(G * 64), klo(G * 64);
    Dev<int32_t> qe(G), ke(G);
    Dev<int64_t> qhs(G), qls(G), qts(G), khs(G), kls(G), kts(G);
    meow::ASrc a;
    a.src = meow::SRC_I8; a.hi = hi.p; a.lo = lo.p; a.ld8 = p.Kp; a.e = e.p;
    meow::AEpi ep;
    ep.epi = meow::EPI_QKV; ep.Y2 = V.p; ep.heads = heads; ep.T = T; ep.TpQ = TpQ; ep.TpK = TpK; ep.C = C;
    ep.qhi = qhi.p; ep.qlo = qlo.p; ep.khi = khi.p; ep.klo = klo.p; ep.qe = qe.p; ep.ke = ke.p;
    ep.qhs = qhs.p; ep.qls = qls.p; ep.qts = qts.p; ep.khs = khs.p; ep.kls = kls.p; ep.kts = kts.p;
    meow::k_gemm_hl2(st, a, p.Mp, M, W.p, p.Kp, p.Np, 3 * C, p.Kp, reinterpret_cast<const int4*>(cst.p), ep);
    HIP_OK(hipStreamSynchronize(st));
    const std::vector<int32_t> y = host_ref(p, false);
    bool vok = true;
    const std::vector<int32_t> vg = V.get();
    for (int r = 0; r < M; ++r)
        for (int c = 0; c < C; ++c) vok = vok && vg[size_t(r) * C + c] == y[size_t(r) * 3 * C + 2 * C + c];
    expect(vok, "EPI_QKV v == plain GEMM columns [2C, 3C)");
    bool qok = true;
    for (int part = 0; part < 2; ++part) {
        const std::vector<int8_t> H = (part ? khi : qhi).get(), L = (part ? klo : qlo).get();
        const std::vector<int32_t> E = (part ? ke : qe).get();
        const std::vector<int64_t> HS = (part ? khs : qhs).get(), LS = (part ? kls : qls).get(), TS = (part ? kts : qts).get();
        for (int r = 0; r < M; ++r)
            for (int h = 0; h < heads; ++h) {
                const int32_t* v = &y[size_t(r) * 3 * C + part * C + 64 * h];
                int64_t m = 0;
                for (int d = 0; d < 64; ++d) m = std::max<int64_t>(m, v[d] < 0 ? -int64_t(v[d]) : v[d]);
                int ee = 0;
                for (int k = 15; k < 32; ++k) ee += m >= (int64_t(1) << k);
                const size_t gt = size_t((r / T) * heads + h) * (part ? TpK : TpQ) + r % T;
                int64_t hs = 0, ls = 0, ts = 0;
                for (int d = 0; d < 64; ++d) {
                    int q = ee ? (v[d] >> ee) + ((v[d] >> (ee - 1)) & 1) : v[d];
                    q = q < -32767 ? -32767 : (q > 32767 ? 32767 : q);
                    const int hb = q >> 8, lb = (q & 255) - 128;
                    qok = qok && H[gt * 64 + d] == hb && L[gt * 64 + d] == lb;
                    hs += hb; ls += lb; ts += q;
                }
                qok = qok && E[gt] == ee && HS[gt] == hs && LS[gt] == ls && TS[gt] == ts;
            }
    }
    expect(qok, "EPI_QKV q/k planes, e and sums == host k_quant_heads restatement");
}

void test_errors(hipStream_t st) {
    expect(!meow::gemm_hl_supported(100, 64, 16) && meow::gemm_hl_supported(128, 64, 16), "gemm_hl_supported");
    bool threw = false;
    try {
        meow::ASrc a;
        meow::AEpi ep;
        meow::k_gemm_hl2(st, a, 100, 100, nullptr, 16, 64, 64, 16, nullptr, ep);
    } catch (const std::runtime_error& ex) {
        threw = std::strstr(ex.what(), "unsupported shape") != nullptr;
    }
    expect(threw, "k_gemm_hl2 throws on an unsupported shape");
    threw = false;
    try {
        meow::Gemm lt;
        lt.init(0);
        lt.run(st, nullptr, 16, 0, nullptr, 16, 0, nullptr, 16, 0, 0, 16, 16);
    } catch (const std::runtime_error& ex) {
        threw = true;
    }
    expect(threw, "Gemm::run throws on a bad call");
}

// A model file through meow::Poisd / meow::DevModel, and GEMMs on its prepared linears: the merged
// to_qkv against to_q, to_k and to_v run alone, and a linear off the padding grid against an int64
// host restatement computed from the file's own tensors.
void test_model(hipStream_t st, std::mt19937& rng, const char* path) {
    meow::Poisd bad;
    std::string err;
    expect(!bad.load(std::string(path) + ".missing", err) && err.find("cannot open") == 0, "Poisd::load reports a missing file");
    meow::Poisd model;
    expect(model.load(path, err), "Poisd::load " + std::string(path) + (err.empty() ? "" : ": " + err));
    expect(model.has("lut.phi") && model.get("lut.phi").count == 2049 && model.i32s("c.cin") == -77, "Poisd accessors");
    meow::DevModel dm;
    dm.load(0, model);
    expect(dm.bytes > 0 && dm.lutPhi32 != nullptr && dm.hasLin("unet.conv_in") && !dm.hasLin("te.tok"), "DevModel::load");
    const std::string blk = "unet.down_blocks.0.attentions.0.transformer_blocks.0.attn1.";
    const meow::Lin& qkv = dm.lin(blk + "to_qkv");
    expect(qkv.N == 192 && qkv.K == 64 && qkv.Np == 192 && qkv.Kp == 64 && !qkv.conv3, "merged to_qkv geometry");
    const int M = 150, Mp = 192;
    std::vector<int16_t> q(size_t(Mp) * 64);
    for (auto& v : q) v = int16_t(int(rng() % 65535) - 32767);
    Dev<int16_t> dq(q);
    auto run = [&](const meow::Lin& L, int ld16) {
        Dev<int32_t> Y(size_t(M) * L.N);
        meow::ASrc a;
        a.src = meow::SRC_I16; a.q16 = dq.p; a.ld16 = ld16; a.K = L.K;
        meow::AEpi ep;
        ep.Y = Y.p; ep.ldy = L.N;
        meow::k_gemm_hl2(st, a, Mp, M, L.w, L.Kp, L.Np, L.N, L.Kp, L.cst, ep);
        HIP_OK(hipStreamSynchronize(st));
        return Y.get();
    };
    const std::vector<int32_t> all = run(qkv, 64);
    bool same = true;
    int part = 0;
    for (const char* p : {"to_q", "to_k", "to_v"}) {
        const std::vector<int32_t> one = run(dm.lin(blk + p), 64);
        for (int r = 0; r < M; ++r)
            for (int n = 0; n < 64; ++n) same = same && all[size_t(r) * 192 + 64 * part + n] == one[size_t(r) * 64 + n];
        ++part;
    }
    expect(same, "merged to_qkv product == to_q | to_k | to_v products");
    // 70 x 40 linear (Np 128, Kp 48): the int16 rows are read at ld16 = 64 with K = 40 real columns
    const std::string te = "unet.time_embedding.linear_1";
    const meow::Lin& L = dm.lin(te);
    const std::vector<int32_t> y = run(L, 64);
    const int8_t* w = model.i8(te + ".w");
    const std::vector<int64_t> m = model.i32v(te + ".m"), s = model.i32v(te + ".s"), b = model.i32v(te + ".b");
    bool ok = L.Np == 128 && L.Kp == 48;
    for (int r = 0; r < M; ++r)
        for (int n = 0; n < 70; ++n) {
            int64_t acc = 0;
            for (int k = 0; k < 40; ++k) acc += int64_t(q[size_t(r) * 64 + k]) * w[n * 40 + k];
            const int64_t want = sat32(rshr(int64_t(uint64_t(acc) * uint64_t(m[n])), s[n]) + b[n]);
            ok = ok && y[size_t(r) * 70 + n] == want;
        }
    expect(ok, "loaded 70x40 linear == int64 host restatement from the file's tensors");
}

}  // namespace

int main(int argc, char** argv) {
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    std::mt19937 rng(1);
    try {
        for (int K : {64, 320, 1280}) test_fused_vs_planar(st, rng, 300, 200, K);
        test_fused_vs_planar(st, rng, 64, 64, 16);
        test_x32(st, rng);
        test_conv32(st, rng);
        test_graph(st, rng);
        test_gnstat(st, rng);
        test_qkv(st, rng);
        test_errors(st);
        if (argc > 1) test_model(st, rng, argv[1]);
    } catch (const std::exception& ex) {
        std::printf("FAIL exception: %s\n", ex.what());
        return 2;
    }
    HIP_OK(hipStreamDestroy(st));
    std::printf("%s: %d failure(s)\n", fails ? "FAILED" : "ALL PASS", fails);
    return fails ? 1 : 0;
}

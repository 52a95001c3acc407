// The reference engine's resnet and transformer blocks (src/engine.cu:140-454) on this library's
// kernels: host code only, every step one call of the C ABI of include/vgemm.h on the caller's
// stream, intermediates from an arena allocated once. The step sequence, the buffers each step
// reads and writes and the engine configuration's choices (fusedLoader, fusedAttention, gnFuse,
// customGemmMaxK) follow the reference, so that the blocks produce its bytes; the GEMMs themselves
// are the fused kernels of this library whatever the reference would route to cuBLASLt (the same
// bytes: the planar route and the fused one agree by construction, tests/test_gpu_gemm.py).
#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/vgemm.h"
#include "../../include/vgemm_engine.h"
#include "../../include/vgemm_model.h"

namespace vk {
int set_error(int code, const std::string& msg);
void clear_error();
}  // namespace vk

namespace {

typedef long long i64;

struct Fail : std::runtime_error {
    int code;
    Fail(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

// a C ABI call of this library: a failure carries its message out of the block
void call(int rc) {
    if (rc != VGEMM_OK) throw Fail(rc, vgemm_last_error());
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Tensor {   // meow::Tensor (src/engine.h:36)
    int32_t* d = nullptr;
    int B = 0, T = 0, C = 0;
    uint32_t* rowmax = nullptr;
    VgemmGnStat* gnst = nullptr;
    size_t n() const { return size_t(B) * T * C; }
};

struct QuantIn {   // the [hi; lo] planes, row shifts and geometry of a row-quantised input (src/engine.h:46)
    int8_t* hi = nullptr;
    int8_t* lo = nullptr;
    int32_t* e = nullptr;
    int B = 0, T = 0, K = 0, Kp = 0, Mp = 0;
    int rows() const { return B * T; }
};

struct HeadQ {   // head-quantised attention operand (src/engine.h:47-49)
    int8_t *hi = nullptr, *lo = nullptr;
    int32_t* e = nullptr;
    int64_t *hs = nullptr, *ls = nullptr, *tsum = nullptr;
    int B = 0, T = 0, Tp = 0, heads = 0;
};

struct AttnKV {   // quantised key/value operands (src/engine.h:50-54)
    int8_t *khi = nullptr, *klo = nullptr, *vthi = nullptr, *vtlo = nullptr;
    int32_t *ek = nullptr, *ev = nullptr;
    int64_t *ksum = nullptr, *vsum = nullptr;
    int Tk = 0, Tkp = 0;
    int B = 0, heads = 0;   // the context's samples and heads (cross-attention K/V only)
};

}  // namespace

struct VgemmEngine {
    const VgemmModel* model = nullptr;
    bool gn_fuse = false;
    // EngineConfig defaults (src/engine.h:56): fused attention, fused loaders, custom GEMM up to Kp 1536
    static constexpr bool fused_attention = true, fused_loader = true;
    static constexpr int custom_gemm_max_k = 1536;
    char* arena = nullptr;
    size_t cap = 0, off = 0, peak = 0;
    const int32_t* lut_phi = nullptr;
    const int32_t* lut_sig = nullptr;
    int64_t* lut_exp = nullptr;   // "lut.exp" widened to int64 (DevModel::lutExp, src/engine.cu:59)
    std::map<std::string, std::pair<AttnKV, std::vector<void*>>> cross;   // per transformer block
    hipStream_t st = nullptr;

    // ---- the arena (src/engine.h:38-44): 256-byte aligned bump allocation, released by marks
    void* alloc(size_t nbytes) {
        const size_t o = align_up(off, 256);
        if (o + nbytes > cap) throw Fail(VGEMM_ERR_ARG, "engine arena too small: need " + std::to_string(o + nbytes) + " bytes");
        off = o + nbytes;
        if (off > peak) peak = off;
        return arena + o;
    }
    size_t mark() const { return off; }
    void release(size_t m) { off = m; }

    VgemmLin lin(const std::string& name) const {
        VgemmLin L;
        call(vgemm_model_lin(model, name.c_str(), &L));
        if (!L.w) throw Fail(VGEMM_ERR_ARG, "engine: model not uploaded");
        return L;
    }
    bool has_lin(const std::string& name) const {
        VgemmLin L;
        return vgemm_model_lin(model, name.c_str(), &L) == VGEMM_OK;
    }
    VgemmNorm norm(const std::string& name) const {
        VgemmNorm N;
        call(vgemm_model_norm(model, name.c_str(), &N));
        return N;
    }

    // ---- ops (src/engine.cu:140-388), same names and roles
    Tensor talloc(int B, int T, int C) {
        Tensor t;
        t.B = B; t.T = T; t.C = C;
        t.d = static_cast<int32_t*>(alloc(t.n() * 4));
        return t;
    }
    bool gn_fusable(int T, int C) const { return gn_fuse && fused_loader && C % 32 == 0 && (size_t(T) * C) % 1024 == 0 && T % 64 == 0; }
    VgemmGnStat* gn_alloc(int B) {
        VgemmGnStat* g = static_cast<VgemmGnStat*>(alloc(sizeof(VgemmGnStat) * B * 32));
        call(vgemm_gn_init(st, g, B * 32));
        return g;
    }
    uint32_t* rowmax_alloc(int rows) {
        uint32_t* p = static_cast<uint32_t*>(alloc(size_t(rows) * 4));
        call(vgemm_fill_u32(st, p, size_t(rows), 0u));   // the reference's cudaMemsetAsync (src/engine.cu:161), capture-safe
        return p;
    }
    bool use_hl(const VgemmLin& L) const { return custom_gemm_max_k > 0 && L.Kp <= custom_gemm_max_k && vgemm_supported(64, L.Np, L.Kp); }

    QuantIn qalloc(int B, int T, int K) {
        QuantIn q;
        q.B = B; q.T = T; q.K = K;
        q.Kp = int(align_up(K, 16));
        q.Mp = int(align_up(size_t(B) * T, 64));
        q.hi = static_cast<int8_t*>(alloc(size_t(2) * q.Mp * q.Kp));   // stacked [hi; lo]
        q.lo = q.hi + size_t(q.Mp) * q.Kp;
        q.e = static_cast<int32_t*>(alloc(size_t(q.Mp) * 4));
        return q;
    }

    // linQ (src/engine.cu:147-157): the planes through the fused GEMM, PLAIN (+ residual)
    Tensor linQ(const QuantIn& q, const VgemmLin& L, int32_t* out = nullptr, const int32_t* residual = nullptr) {
        if (q.K != L.K || q.Kp != L.Kp) throw Fail(VGEMM_ERR_ARG, "linQ: K mismatch " + std::to_string(q.K) + " vs " + std::to_string(L.K));
        Tensor y;
        y.B = q.B; y.T = q.T; y.C = L.N;
        y.d = out ? out : static_cast<int32_t*>(alloc(y.n() * 4));
        call(vgemm_hl(st, q.hi, q.lo, L.Kp, q.Mp, q.rows(), L.w, L.Kp, L.Np, L.N, L.Kp, L.cst, q.e, y.d, L.N, residual, VGEMM_EPI_PLAIN, 0,
                      nullptr, nullptr, nullptr));
        return y;
    }

    // lin (src/engine.cu:177-186): k_quant_rows, then linQ
    Tensor lin(const Tensor& x, const VgemmLin& L, int32_t* out = nullptr, const int32_t* residual = nullptr) {
        if (x.C != L.K) throw Fail(VGEMM_ERR_ARG, "lin: K mismatch " + std::to_string(x.C) + " vs " + std::to_string(L.K));
        Tensor y;
        y.B = x.B; y.T = x.T; y.C = L.N;
        y.d = out ? out : static_cast<int32_t*>(alloc(y.n() * 4));
        const size_t mk = mark();
        QuantIn q = qalloc(x.B, x.T, x.C);
        call(vgemm_quant_rows(st, x.d, q.rows(), L.K, L.K, q.hi, q.lo, q.e, L.Kp));
        linQ(q, L, y.d, residual);
        release(mk);
        return y;
    }

    // linX (src/engine.cu:162-175): int32 rows quantised inside the GEMM from their row maxima
    Tensor linX(const Tensor& x, const VgemmLin& L, int32_t* out = nullptr, const int32_t* residual = nullptr, int epi = VGEMM_EPI_PLAIN,
                bool want_rowmax = false, VgemmGnStat* gn_out = nullptr) {
        if (!(fused_loader && x.rowmax && use_hl(L) && L.K % 16 == 0)) {
            if (epi == VGEMM_EPI_GELU) {
                Tensor y = lin(x, L, out, residual);
                call(vgemm_act(st, y.d, y.n(), lut_phi));
                return y;
            }
            return lin(x, L, out, residual);
        }
        const int rows = x.B * x.T, Mp = int(align_up(rows, 64));
        Tensor y;
        y.B = x.B; y.T = x.T; y.C = L.N;
        y.d = out ? out : static_cast<int32_t*>(alloc(y.n() * 4));
        if (want_rowmax) y.rowmax = rowmax_alloc(rows);
        if (gn_out && epi == VGEMM_EPI_PLAIN && gn_fusable(x.T, L.N)) y.gnst = gn_out;
        VgemmASrc A;
        vgemm_asrc_init(&A);
        A.src = VGEMM_SRC_X32; A.x = x.d; A.ldx = x.C; A.rowmax = x.rowmax; A.K = L.K;
        VgemmAEpi E;
        vgemm_aepi_init(&E);
        E.epi = epi; E.Y = y.d; E.ldy = L.N; E.residual = residual; E.Lphi = lut_phi; E.rowmax = y.rowmax; E.gnstat = y.gnst; E.gnT = x.T;
        call(vgemm_hl2(st, &A, Mp, rows, L.w, L.Kp, L.Np, L.N, L.Kp, L.cst, &E));
        return y;
    }

    // gegluX (src/engine.cu:230-238): the interleaved GEGLU GEMM with its row maxima
    Tensor geglu_x(const QuantIn& q, const VgemmLin& Li, int F) {
        const int rows = q.rows();
        Tensor v;
        v.B = q.B; v.T = q.T; v.C = F;
        v.d = static_cast<int32_t*>(alloc(size_t(q.Mp) * F * 4));
        v.rowmax = rowmax_alloc(rows);
        VgemmASrc A;
        vgemm_asrc_init(&A);
        A.src = VGEMM_SRC_I8; A.hi = q.hi; A.lo = q.lo; A.ld8 = Li.Kp; A.e = q.e;
        VgemmAEpi E;
        vgemm_aepi_init(&E);
        E.epi = VGEMM_EPI_GEGLU; E.Y = v.d; E.ldy = F; E.Lphi = lut_phi; E.rowmax = v.rowmax;
        call(vgemm_hl2(st, &A, q.Mp, rows, Li.w, Li.Kp, Li.Np, Li.N, Li.Kp, Li.cst, &E));
        return v;
    }

    QuantIn layernorm_q(const Tensor& x, const VgemmNorm& nm) {   // src/engine.cu:239-244
        if (nm.C != x.C) throw Fail(VGEMM_ERR_ARG, "layernormQ: C mismatch");
        QuantIn q = qalloc(x.B, x.T, x.C);
        call(vgemm_lnorm_q(st, x.d, q.rows(), x.C, nm.g, nm.beta, nm.den, q.hi, q.lo, q.e, q.Kp));
        return q;
    }

    // the GroupNorm statistics of x: the producer's records finalised, or gathered now
    VgemmGnStat* gn_stats(const Tensor& x, const VgemmNorm& nm) {
        VgemmGnStat* gs = x.gnst;
        if (gs) {
            call(vgemm_gn_fin1(st, gs, x.B * 32, i64(x.T) * (x.C / 32)));
        } else {
            gs = static_cast<VgemmGnStat*>(alloc(sizeof(VgemmGnStat) * x.B * 32));
            call(vgemm_gn_stats1(st, x.d, x.B, x.T, x.C, 32, gs));
        }
        call(vgemm_gn_stats2(st, x.d, x.B, x.T, x.C, 32, nm.den, gs));
        return gs;
    }

    QuantIn groupnorm_q(const Tensor& x, const VgemmNorm& nm) {   // src/engine.cu:245-255
        if (nm.C != x.C) throw Fail(VGEMM_ERR_ARG, "groupnormQ: C mismatch");
        QuantIn q = qalloc(x.B, x.T, x.C);
        const size_t mk = mark();
        VgemmGnStat* gs = gn_stats(x, nm);
        call(vgemm_gn_apply_row(st, x.d, x.B, x.T, x.C, 32, gs, nm.g, nm.beta, nullptr, nullptr, nullptr, q.hi, q.lo, q.e, q.Kp));
        release(mk);
        return q;
    }

    Tensor groupnorm_silu(const Tensor& x, const VgemmNorm& nm, uint32_t*& pm) {   // src/engine.cu:256-267
        if (nm.C != x.C) throw Fail(VGEMM_ERR_ARG, "groupnormSilu: C mismatch");
        Tensor y = talloc(x.B, x.T, x.C);
        pm = static_cast<uint32_t*>(alloc(size_t(x.B) * x.T * 4));
        const size_t mk = mark();
        VgemmGnStat* gs = gn_stats(x, nm);
        call(vgemm_gn_apply_row(st, x.d, x.B, x.T, x.C, 32, gs, nm.g, nm.beta, lut_sig, y.d, pm, nullptr, nullptr, nullptr, 0));
        release(mk);
        return y;
    }

    // conv3 (src/engine.cu:268-289): the pixel maxima (pmIn, or k_pixmax's), k_conv_e's row shifts and
    // the implicit im2col of the int32 image inside the GEMM; the planar route (k_im2col3 into planes)
    // when the channels are not a multiple of 16
    Tensor conv3(const Tensor& x, int H, int W, const VgemmLin& L, int stride, int32_t* out = nullptr, const int32_t* residual = nullptr,
                 const uint32_t* pm_in = nullptr, VgemmGnStat* gn_out = nullptr) {
        if (!L.conv3 || x.C * 9 != L.K) throw Fail(VGEMM_ERR_ARG, "conv3: shape mismatch");
        const int Ho = (H - 1) / stride + 1, Wo = (W - 1) / stride + 1, rows = x.B * Ho * Wo, Mp = int(align_up(rows, 64));
        Tensor y;
        y.B = x.B; y.T = Ho * Wo; y.C = L.N;
        y.d = out ? out : static_cast<int32_t*>(alloc(y.n() * 4));
        if (gn_out && gn_fusable(y.T, L.N)) y.gnst = gn_out;
        const size_t mk = mark();
        const uint32_t* pm = pm_in;
        if (!pm) {
            uint32_t* p = static_cast<uint32_t*>(alloc(size_t(x.B) * H * W * 4));
            call(vgemm_pixmax(st, x.d, x.B * H * W, x.C, p));
            pm = p;
        }
        int32_t* e = static_cast<int32_t*>(alloc(size_t(Mp) * 4));
        VgemmASrc A;
        vgemm_asrc_init(&A);
        VgemmAEpi E;
        vgemm_aepi_init(&E);
        E.epi = VGEMM_EPI_PLAIN; E.Y = y.d; E.ldy = L.N; E.residual = residual; E.gnstat = y.gnst; E.gnT = y.T;
        if (!use_hl(L)) throw Fail(VGEMM_ERR_UNSUPPORTED, "conv3: Kp above the fused GEMM's limit");
        if (fused_loader && x.C % 16 == 0) {
            call(vgemm_conv_e(st, pm, x.B, H, W, stride, e));
            A.src = VGEMM_SRC_CONV32; A.img = x.d; A.H = H; A.W = W; A.C = x.C; A.stride = stride; A.Ho = Ho; A.Wo = Wo; A.K = L.K; A.e = e;
        } else {
            int8_t* hi = static_cast<int8_t*>(alloc(size_t(2) * Mp * L.Kp));
            int8_t* lo = hi + size_t(Mp) * L.Kp;
            call(vgemm_im2col3(st, x.d, pm, x.B, H, W, x.C, stride, hi, lo, e, L.Kp));
            A.src = VGEMM_SRC_I8; A.hi = hi; A.lo = lo; A.ld8 = L.Kp; A.e = e;
        }
        call(vgemm_hl2(st, &A, Mp, rows, L.w, L.Kp, L.Np, L.N, L.Kp, L.cst, &E));
        release(mk);
        return y;
    }

    HeadQ head_alloc(int B, int heads, int T, int Tp) {   // src/engine.cu:319-324
        HeadQ h;
        h.B = B; h.T = T; h.Tp = Tp; h.heads = heads;
        const size_t G = size_t(B) * heads;
        h.hi = static_cast<int8_t*>(alloc(G * Tp * 64));
        h.lo = static_cast<int8_t*>(alloc(G * Tp * 64));
        h.e = static_cast<int32_t*>(alloc(G * Tp * 4));
        h.hs = static_cast<int64_t*>(alloc(G * Tp * 8));
        h.ls = static_cast<int64_t*>(alloc(G * Tp * 8));
        h.tsum = static_cast<int64_t*>(alloc(G * Tp * 8));
        return h;
    }

    // linQ3H (src/engine.cu:325-339): merged q|k|v GEMM, q and k head-quantised in its epilogue
    void linQ3H(const QuantIn& q, const VgemmLin& L, int C, int heads, int Treal, HeadQ& qh, HeadQ& kh, Tensor& v) {
        if (q.K != L.K || L.N != 3 * C || C != heads * 64) throw Fail(VGEMM_ERR_ARG, "linQ3H: shape mismatch");
        const int rows = q.rows();
        const int TpQ = int(align_up(Treal, 128)), TpK = int(align_up(Treal, 64));
        qh = head_alloc(q.B, heads, Treal, TpQ);
        kh = head_alloc(q.B, heads, Treal, TpK);
        v = talloc(q.B, q.T, C);
        VgemmASrc A;
        vgemm_asrc_init(&A);
        A.src = VGEMM_SRC_I8; A.hi = q.hi; A.lo = q.lo; A.ld8 = L.Kp; A.e = q.e;
        VgemmAEpi E;
        vgemm_aepi_init(&E);
        E.epi = VGEMM_EPI_QKV; E.Y2 = v.d; E.heads = heads; E.T = q.T; E.TpQ = TpQ; E.TpK = TpK; E.C = C;
        E.qhi = qh.hi; E.qlo = qh.lo; E.qe = qh.e; E.qhs = qh.hs; E.qls = qh.ls; E.qts = qh.tsum;
        E.khi = kh.hi; E.klo = kh.lo; E.ke = kh.e; E.khs = kh.hs; E.kls = kh.ls; E.kts = kh.tsum;
        call(vgemm_hl2(st, &A, q.Mp, rows, L.w, L.Kp, L.Np, L.N, L.Kp, L.cst, &E));
        const int G = q.B * heads;
        call(vgemm_quant_heads_pad(st, G, q.T, TpQ, qh.hi, qh.lo, qh.e, qh.hs, qh.ls, qh.tsum));   // rows the GEMM did not write
        call(vgemm_quant_heads_pad(st, G, q.T, TpK, kh.hi, kh.lo, kh.e, kh.hs, kh.ls, kh.tsum));
    }

    AttnKV quant_kvh(const HeadQ& k, const Tensor& v, int heads) {   // src/engine.cu:340-348
        AttnKV kv;
        kv.Tk = k.T; kv.Tkp = k.Tp;
        const size_t G = size_t(v.B) * heads;
        kv.khi = k.hi; kv.klo = k.lo; kv.ek = k.e; kv.ksum = k.tsum;
        kv.vthi = static_cast<int8_t*>(alloc(G * 64 * kv.Tkp));
        kv.vtlo = static_cast<int8_t*>(alloc(G * 64 * kv.Tkp));
        kv.ev = static_cast<int32_t*>(alloc(G * 64 * 4));
        kv.vsum = static_cast<int64_t*>(alloc(G * 64 * 8));
        call(vgemm_quant_v(st, v.d, v.B, k.T, v.C, heads, kv.Tkp, kv.vthi, kv.vtlo, kv.ev, kv.vsum, nullptr));
        return kv;
    }

    // attentionH / attention (src/engine.cu:341-388, fusedAttention): the exact fused attention, the
    // output's row maxima for the SRC_X32 projection that follows
    Tensor attention_h(const HeadQ& q, const AttnKV& kv, int heads, bool causal, int Tq, int C) {
        const int B = q.B;
        Tensor out = talloc(B, Tq, C);
        if (fused_loader) out.rowmax = rowmax_alloc(B * Tq);
        call(vgemm_fused_attention(st, q.hi, q.lo, q.e, q.hs, q.ls, kv.khi, kv.klo, kv.ek, kv.ksum, kv.vthi, kv.vtlo, kv.ev, kv.vsum, B, heads, Tq,
                                   q.Tp, kv.Tk, kv.Tkp, causal ? 1 : 0, lut_exp, C, nullptr, nullptr, out.d, out.rowmax));
        return out;
    }
    Tensor attention(const Tensor& q, const AttnKV& kv, int heads, bool causal, int Tq) {
        const int B = q.B, C = q.C;
        if (C != heads * 64) throw Fail(VGEMM_ERR_ARG, "attention: C != heads*64");
        const int Tqp = int(align_up(q.T, 128));   // fusedAttention (src/engine.cu:354)
        HeadQ h = head_alloc(B, heads, q.T, Tqp);
        call(vgemm_quant_heads(st, q.d, B, Tq, C, heads, Tqp, h.hi, h.lo, h.e, h.hs, h.ls, h.tsum));
        return attention_h(h, kv, heads, causal, Tq, C);
    }

    // ---- blocks
    Tensor resnet(const Tensor& x, int H, int W, const std::string& p, int32_t* out_d, VgemmGnStat* out_gn) {   // src/engine.cu:389-405
        const VgemmLin c1 = lin(p + ".conv1"), c2 = lin(p + ".conv2");
        Tensor out;
        out.B = x.B; out.T = x.T; out.C = c2.N; out.d = out_d;
        VgemmGnStat* g_out = gn_fusable(out.T, out.C) ? out_gn : nullptr;
        if (g_out) call(vgemm_gn_init(st, g_out, out.B * 32));   // gnAlloc's k_gn_init, on the caller's records
        const size_t mk = mark();
        uint32_t *pm1 = nullptr, *pm2 = nullptr;
        Tensor h = groupnorm_silu(x, norm(p + ".norm1"), pm1);
        VgemmGnStat* g1 = gn_fusable(h.T, c1.N) ? gn_alloc(h.B) : nullptr;
        h = conv3(h, H, W, c1, 1, nullptr, nullptr, pm1, g1);
        Tensor h2 = groupnorm_silu(h, norm(p + ".norm2"), pm2);
        Tensor o;
        if (has_lin(p + ".conv_shortcut")) {
            Tensor xs = lin(x, lin(p + ".conv_shortcut"));
            o = conv3(h2, H, W, c2, 1, out.d, xs.d, pm2, g_out);
        } else {
            o = conv3(h2, H, W, c2, 1, out.d, x.d, pm2, g_out);
        }
        out.gnst = o.gnst;
        release(mk);
        return out;
    }

    Tensor transformer(const Tensor& x, const std::string& p, int heads, int32_t* out_d, VgemmGnStat* out_gn) {   // src/engine.cu:406-454
        Tensor out;
        out.B = x.B; out.T = x.T; out.C = x.C; out.d = out_d;
        VgemmGnStat* g_out = gn_fusable(out.T, out.C) ? out_gn : nullptr;
        if (g_out) call(vgemm_gn_init(st, g_out, out.B * 32));
        const size_t mk = mark();
        const std::string b = p + ".transformer_blocks.0";
        Tensor h = talloc(x.B, x.T, lin(p + ".proj_in").N);
        {
            const size_t m2 = mark();
            QuantIn xq = groupnorm_q(x, norm(p + ".norm"));
            linQ(xq, lin(p + ".proj_in"), h.d);
            release(m2);
        }
        {
            const size_t m2 = mark();
            QuantIn n = layernorm_q(h, norm(b + ".norm1"));
            const VgemmLin qkv = lin(b + ".attn1.to_qkv");
            if (!(fused_attention && use_hl(qkv))) throw Fail(VGEMM_ERR_UNSUPPORTED, "transformer: the unfused attention route is not part of this library");
            HeadQ qh, kh;
            Tensor v;
            linQ3H(n, qkv, h.C, heads, h.T, qh, kh, v);
            AttnKV kv = quant_kvh(kh, v, heads);
            Tensor a = attention_h(qh, kv, heads, false, h.T, h.C);
            linX(a, lin(b + ".attn1.to_out.0"), h.d, h.d);
            release(m2);
        }
        {
            const size_t m2 = mark();
            QuantIn n = layernorm_q(h, norm(b + ".norm2"));
            Tensor q = linQ(n, lin(b + ".attn2.to_q"));
            auto it = cross.find(b);
            if (it == cross.end()) throw Fail(VGEMM_ERR_ARG, "no cross KV for " + b);
            if (it->second.first.B != x.B || it->second.first.heads != heads)
                throw Fail(VGEMM_ERR_ARG, "cross KV of " + b + " set for another batch or head count");
            Tensor a = attention(q, it->second.first, heads, false, q.T);
            linX(a, lin(b + ".attn2.to_out.0"), h.d, h.d);
            release(m2);
        }
        {
            const size_t m2 = mark();
            QuantIn n = layernorm_q(h, norm(b + ".norm3"));
            const int F = lin(b + ".ff.net.0.proj.a").N;
            const VgemmLin Li = lin(b + ".ff.net.0.proj.agi");
            if (fused_loader && use_hl(Li)) {
                Tensor v = geglu_x(n, Li, F);
                Tensor hh = linX(v, lin(b + ".ff.net.2"), h.d, h.d, VGEMM_EPI_PLAIN, true);
                h.rowmax = hh.rowmax;
            } else {
                // the reference's linQGegluQ route (src/engine.cu:449) is taken only above Kp 1536
                throw Fail(VGEMM_ERR_UNSUPPORTED, "transformer: the GEGLU up-projection needs Kp <= 1536");
            }
            release(m2);
        }
        {
            Tensor o = linX(h, lin(p + ".proj_out"), out.d, x.d, VGEMM_EPI_PLAIN, false, g_out);
            out.gnst = o.gnst;
        }
        release(mk);
        return out;
    }

    // the cross-attention K/V of one block (src/engine.cu:545-560 for a context per sample)
    void set_context(const Tensor& ctx, const std::string& b, int heads) {
        const size_t mk = mark();
        Tensor k = lin(ctx, lin(b + ".attn2.to_k")), v = lin(ctx, lin(b + ".attn2.to_v"));
        if (k.C != heads * 64 || v.C != k.C) throw Fail(VGEMM_ERR_ARG, "set_context: to_k / to_v width != heads*64");
        const int Tk = ctx.T, Tkp = int(align_up(Tk, 64));
        const size_t G = size_t(ctx.B) * heads;
        auto& slot = cross[b];
        for (void* q : slot.second) (void)hipFree(q);
        slot.second.clear();
        auto pa = [&](size_t n) {
            void* q = nullptr;
            if (hipMalloc(&q, n) != hipSuccess) throw Fail(VGEMM_ERR_HIP, "set_context: hipMalloc failed");
            slot.second.push_back(q);
            return q;
        };
        AttnKV& kv = slot.first;
        kv = AttnKV();
        kv.Tk = Tk; kv.Tkp = Tkp; kv.B = ctx.B; kv.heads = heads;
        kv.khi = static_cast<int8_t*>(pa(G * Tkp * 64));
        kv.klo = static_cast<int8_t*>(pa(G * Tkp * 64));
        kv.ek = static_cast<int32_t*>(pa(G * Tkp * 4));
        kv.ksum = static_cast<int64_t*>(pa(G * Tkp * 8));
        int64_t* hs = static_cast<int64_t*>(alloc(G * Tkp * 8));
        int64_t* ls = static_cast<int64_t*>(alloc(G * Tkp * 8));
        kv.vthi = static_cast<int8_t*>(pa(G * 64 * Tkp));
        kv.vtlo = static_cast<int8_t*>(pa(G * 64 * Tkp));
        kv.ev = static_cast<int32_t*>(pa(G * 64 * 4));
        kv.vsum = static_cast<int64_t*>(pa(G * 64 * 8));
        call(vgemm_quant_heads(st, k.d, k.B, k.T, k.C, heads, Tkp, kv.khi, kv.klo, kv.ek, hs, ls, kv.ksum));
        call(vgemm_quant_v(st, v.d, v.B, v.T, v.C, heads, Tkp, kv.vthi, kv.vtlo, kv.ev, kv.vsum, nullptr));
        if (hipStreamSynchronize(st) != hipSuccess) throw Fail(VGEMM_ERR_HIP, "set_context: stream failed");
        release(mk);
    }
};

namespace {

Tensor tensor_of(const VgemmActivation* a) {
    Tensor t;
    t.d = a->d; t.B = a->B; t.T = a->T; t.C = a->C; t.rowmax = a->rowmax;
    t.gnst = static_cast<VgemmGnStat*>(a->gnst);
    return t;
}

bool valid(const VgemmActivation* a) { return a && a->d && a->B > 0 && a->T > 0 && a->C > 0; }

template <class F>
int guarded(VgemmEngine* e, void* stream, F&& f) {
    if (!e) return vk::set_error(VGEMM_ERR_ARG, "engine: null engine");
    e->st = static_cast<hipStream_t>(stream);
    const size_t mk = e->mark();
    try {
        f();
    } catch (const Fail& x) {
        e->release(mk);
        return vk::set_error(x.code, x.what());
    } catch (const std::exception& x) {
        e->release(mk);
        return vk::set_error(VGEMM_ERR_ARG, x.what());
    }
    vk::clear_error();
    return VGEMM_OK;
}

}  // namespace

extern "C" {

int vgemm_engine_create(const VgemmModel* model, size_t arena_bytes, int gn_fuse, VgemmEngine** out) {
    if (!out) return vk::set_error(VGEMM_ERR_ARG, "engine: null out");
    *out = nullptr;
    if (!model || !arena_bytes) return vk::set_error(VGEMM_ERR_ARG, "engine: a model and an arena size are needed");
    VgemmEngine* e = new VgemmEngine;
    e->model = model;
    e->gn_fuse = gn_fuse != 0;
    try {
        int n = 0;
        call(vgemm_model_table(model, "lut.phi", &e->lut_phi, &n));
        call(vgemm_model_table(model, "lut.sigmoid", &e->lut_sig, &n));
        VgemmTensor t;
        call(vgemm_model_tensor(model, "lut.exp", &t));
        if (t.dtype != VGEMM_DT_I32 || t.count < 1025) throw Fail(VGEMM_ERR_FORMAT, "lut.exp: 1025 int32 entries needed");
        std::vector<int64_t> lx(t.count);
        for (size_t i = 0; i < t.count; ++i) {
            int32_t v;
            std::memcpy(&v, static_cast<const char*>(t.data) + 4 * i, 4);
            lx[i] = v;
        }
        if (hipMalloc(reinterpret_cast<void**>(&e->lut_exp), lx.size() * 8) != hipSuccess ||
            hipMemcpy(e->lut_exp, lx.data(), lx.size() * 8, hipMemcpyHostToDevice) != hipSuccess)
            throw Fail(VGEMM_ERR_HIP, "engine: exp table upload failed");
        if (hipMalloc(reinterpret_cast<void**>(&e->arena), arena_bytes) != hipSuccess) throw Fail(VGEMM_ERR_HIP, "engine: arena hipMalloc failed");
        e->cap = arena_bytes;
    } catch (const Fail& x) {
        vgemm_engine_destroy(e);
        return vk::set_error(x.code, x.what());
    }
    *out = e;
    vk::clear_error();
    return VGEMM_OK;
}

void vgemm_engine_destroy(VgemmEngine* e) {
    if (!e) return;
    for (auto& kv : e->cross)
        for (void* p : kv.second.second) (void)hipFree(p);
    if (e->lut_exp) (void)hipFree(e->lut_exp);
    if (e->arena) (void)hipFree(e->arena);
    delete e;
}

size_t vgemm_engine_arena_peak(const VgemmEngine* e) { return e ? e->peak : 0; }

int vgemm_engine_resnet(VgemmEngine* e, void* stream, const VgemmActivation* x, int H, int W, const char* prefix, VgemmActivation* out) {
    if (!valid(x) || !out || !out->d || !prefix || H <= 0 || W <= 0 || x->T != H * W) return vk::set_error(VGEMM_ERR_ARG, "resnet: bad arguments");
    return guarded(e, stream, [&] {
        const Tensor o = e->resnet(tensor_of(x), H, W, prefix, out->d, static_cast<VgemmGnStat*>(out->gnst));
        out->B = o.B; out->T = o.T; out->C = o.C; out->rowmax = nullptr; out->gnst = o.gnst;
    });
}

int vgemm_engine_set_context(VgemmEngine* e, void* stream, const VgemmActivation* ctx, const char* block, int heads) {
    if (!valid(ctx) || !block || heads <= 0) return vk::set_error(VGEMM_ERR_ARG, "set_context: bad arguments");
    return guarded(e, stream, [&] { e->set_context(tensor_of(ctx), block, heads); });
}

int vgemm_engine_transformer(VgemmEngine* e, void* stream, const VgemmActivation* x, const char* prefix, int heads, VgemmActivation* out) {
    if (!valid(x) || !out || !out->d || !prefix || heads <= 0) return vk::set_error(VGEMM_ERR_ARG, "transformer: bad arguments");
    return guarded(e, stream, [&] {
        const Tensor o = e->transformer(tensor_of(x), prefix, heads, out->d, static_cast<VgemmGnStat*>(out->gnst));
        out->B = o.B; out->T = o.T; out->C = o.C; out->rowmax = nullptr; out->gnst = o.gnst;
    });
}

}  // extern "C"

"""The reference engine's resnet and transformer blocks (src/engine.cu:140-454) composed from the
oracle's functions, step for step as Engine::resnet / Engine::transformer run them with the engine
configuration's defaults (fusedAttention, fusedLoader, customGemmMaxK 1536) and gnFuse on or off:
the GroupNorm / LayerNorm producers, the fused GEMM on each source (planes, int32 rows with row
maxima, implicit 3x3 im2col), the QKV epilogue and its pad rows, the exact attention, and the
GroupNorm records a fused GEMM gathers by the reference's per-tile rule. Test infrastructure: the
GPU tests compare vela_amd.engine's blocks with these compositions byte for byte.

Every function used here is pinned on its own (tests/test_oracle_*.py); this module adds only the
wiring, which follows src/engine.cu line by line (cited per step)."""
from __future__ import annotations

import numpy as np

import oracle
from oracle import model as om

GROUPS = 32


def _r(v, a):
    return (v + a - 1) // a * a


class Act:
    """meow::Tensor (src/engine.h:36) on the host: d [B * T, C], optional rowmax and GroupNorm records."""

    def __init__(self, d, B, T, rowmax=None, gs=None):
        self.d = np.ascontiguousarray(d, np.int32)
        self.B, self.T = B, T
        self.rowmax = rowmax
        self.gs = gs

    @property
    def C(self):
        return self.d.shape[1]

    @property
    def rows(self):
        return self.B * self.T


class OracleEngine:
    def __init__(self, model_bytes: bytes, gn_fuse: bool):
        ents = om.parse_poisd(model_bytes)
        self.lins, self.norms = om.dev_model(ents)
        self.gn_fuse = gn_fuse
        self.Lphi = ents["lut.phi"][2].reshape(-1).astype(np.int32)
        self.Lsig = ents["lut.sigmoid"][2].reshape(-1).astype(np.int32)
        self.Lexp = ents["lut.exp"][2].reshape(-1).astype(np.int64)   # DevModel::lutExp = up64 (src/engine.cu:59)
        self.cross = {}

    # ---- helpers
    def lin(self, name):
        W, cst, N, K, conv3 = self.lins[name]
        return W, cst, N, K, conv3

    def gn_fusable(self, T, C):   # src/engine.h:110 (fusedLoader is on)
        return self.gn_fuse and C % 32 == 0 and (T * C) % 1024 == 0 and T % 64 == 0

    @staticmethod
    def records_of(stats, cnt):
        gs = oracle.gn_records(cnt)
        gs["sum"], gs["mn"], gs["mx"] = stats["sum"], stats["mn"], stats["mx"]
        return gs

    # ---- ops (src/engine.cu:140-388)
    def linQ(self, hi, lo, e, B, T, name, residual=None):   # :147-157, the fused route (useHl)
        W, cst, N, K, _ = self.lin(name)
        Y = oracle.gemm(oracle.SRC_I8, hi=hi, lo=lo, e=e, Mreal=B * T, Nreal=N, Kp=W.shape[1], w=W, cst=cst,
                        residual=None if residual is None else residual.copy())
        return Act(Y, B, T)

    def lin_(self, x: Act, name, residual=None):   # :177-186: k_quant_rows, then linQ
        W, cst, N, K, _ = self.lin(name)
        assert x.C == K
        hi, lo, e = oracle.quant_rows(x.d, x.rows, K, K, W.shape[1])
        return self.linQ(hi, lo, e, x.B, x.T, name, residual)

    def linX(self, x: Act, name, residual=None, epi=oracle.EPI_PLAIN, want_rowmax=False, gn_out=False):   # :162-175
        W, cst, N, K, _ = self.lin(name)
        Kp = W.shape[1]
        if x.rowmax is None or Kp > 1536 or K % 16:
            y = self.lin_(x, name, residual)
            if epi == oracle.EPI_GELU:
                y.d = oracle.act(y.d, self.Lphi)
            return y
        rm = np.zeros(x.rows, np.uint32) if want_rowmax else None
        Y = oracle.gemm(oracle.SRC_X32, x=x.d, xrowmax=x.rowmax, K=K, Mreal=x.rows, Nreal=N, Kp=Kp, w=W, cst=cst, epi=epi,
                        Lphi=self.Lphi, residual=None if residual is None else residual.copy(), rowmax=rm)
        y = Act(Y, x.B, x.T, rowmax=rm)
        if gn_out and epi == oracle.EPI_PLAIN and self.gn_fusable(x.T, N):
            st = oracle.gn_stats_fused(Y, x.rows, N, x.T, _r(x.rows, 64), W.shape[0], Kp, oracle.SRC_X32)
            y.gs = self.records_of(st, x.B * GROUPS)
        return y

    def gn_stats(self, x: Act, den):   # the statistics part of :245-267
        if x.gs is not None:
            gs = x.gs.copy()
            oracle.gn_fin1(gs, x.T * (x.C // GROUPS))
        else:
            gs = oracle.gn_stats1(x.d, x.B, x.T, x.C, GROUPS)
        oracle.gn_stats2(x.d, x.B, x.T, x.C, GROUPS, den, gs)
        return gs

    def groupnorm_q(self, x: Act, name):   # :245-255
        g, beta, den = self.norms[name]
        gs = self.gn_stats(x, den)
        return oracle.gn_apply_row(x.d, x.B, x.T, x.C, GROUPS, gs, g, beta, None, Kp=_r(x.C, 16))

    def groupnorm_silu(self, x: Act, name):   # :256-267
        g, beta, den = self.norms[name]
        gs = self.gn_stats(x, den)
        y, pm = oracle.gn_apply_row(x.d, x.B, x.T, x.C, GROUPS, gs, g, beta, self.Lsig)
        return Act(y, x.B, x.T), pm

    def layernorm_q(self, x: Act, name):   # :239-244
        g, beta, den = self.norms[name]
        return oracle.lnorm_q(x.d, x.rows, x.C, g, beta, den, _r(x.C, 16))

    def conv3(self, x: Act, H, W_, name, residual=None, pm=None, gn_out=False):   # :268-289, stride 1
        Wt, cst, N, K, conv3 = self.lin(name)
        assert conv3 and K == 9 * x.C
        Kp = Wt.shape[1]
        rows = x.rows
        if pm is None:
            pm = oracle.pixmax(x.d, x.B * H * W_, x.C)
        kw = dict(Mreal=rows, Nreal=N, Kp=Kp, w=Wt, cst=cst, residual=None if residual is None else residual.copy())
        if x.C % 16 == 0:
            e = oracle.conv_e(pm, x.B, H, W_, 1)
            Y = oracle.gemm(oracle.SRC_CONV32, img=x.d, H=H, W=W_, C=x.C, stride=1, e=e, **kw)
            src = oracle.SRC_CONV32
        else:
            hi, lo, e = oracle.im2col3(x.d, pm, x.B, H, W_, x.C, 1, Kp)
            Y = oracle.gemm(oracle.SRC_I8, hi=hi, lo=lo, e=e, **kw)
            src = oracle.SRC_I8
        y = Act(Y, x.B, H * W_)
        if gn_out and self.gn_fusable(y.T, N):
            st = oracle.gn_stats_fused(Y, rows, N, y.T, _r(rows, 64), Wt.shape[0], Kp, src)
            y.gs = self.records_of(st, x.B * GROUPS)
        return y

    def attention_h(self, q, kv, B, heads, Tq, Tqp, C):   # :341-350 / :351-361: the exact fused attention
        qh, ql, eq = q[0], q[1], q[2]
        kh, kl, ek, vth, vtl, ev, Tk, Tkp = kv
        rm = np.zeros(B * Tq, np.uint32)
        out = oracle.attention(qh, ql, eq, kh, kl, ek, vth, vtl, ev, B, heads, Tq, Tqp, Tk, Tkp, False, self.Lexp, C, rowmax=rm)
        return Act(out, B, Tq, rowmax=rm)

    # ---- blocks
    def resnet(self, x: Act, H, W_, p):   # :389-405
        h, pm1 = self.groupnorm_silu(x, p + ".norm1")
        h = self.conv3(h, H, W_, p + ".conv1", pm=pm1, gn_out=True)
        h2, pm2 = self.groupnorm_silu(h, p + ".norm2")
        if p + ".conv_shortcut" in self.lins:
            xs = self.lin_(x, p + ".conv_shortcut")
            return self.conv3(h2, H, W_, p + ".conv2", residual=xs.d, pm=pm2, gn_out=True)
        return self.conv3(h2, H, W_, p + ".conv2", residual=x.d, pm=pm2, gn_out=True)

    def set_context(self, ctx: Act, block, heads):   # :545-560 (k_quant_heads and k_quant_v of one context per sample)
        k = self.lin_(ctx, block + ".attn2.to_k")
        v = self.lin_(ctx, block + ".attn2.to_v")
        Tkp = _r(ctx.T, 64)
        kh, kl, ek, _, _, _ = oracle.quant_heads(k.d, ctx.B, ctx.T, k.C, heads, Tkp)
        vth, vtl, ev, _ = oracle.quant_v(v.d, ctx.B, ctx.T, v.C, heads, Tkp)
        self.cross[block] = (kh, kl, ek, vth, vtl, ev, ctx.T, Tkp)

    def transformer(self, x: Act, p, heads):   # :406-454
        b = p + ".transformer_blocks.0"
        B, T, C = x.B, x.T, x.C
        M = B * T
        hi, lo, e = self.groupnorm_q(x, p + ".norm")
        h = self.linQ(hi, lo, e, B, T, p + ".proj_in")
        # self-attention: linQ3H (:325-339), quantKVH (:340-348), attentionH, to_out.0 on the int32 rows
        hi, lo, e = self.layernorm_q(h, b + ".norm1")
        Wq, cq, N3, _, _ = self.lin(b + ".attn1.to_qkv")
        assert N3 == 3 * C and C == heads * 64
        Y = oracle.gemm(oracle.SRC_I8, hi=hi, lo=lo, e=e, Mreal=M, Nreal=N3, Kp=Wq.shape[1], w=Wq, cst=cq)
        TpQ, TpK = _r(T, 128), _r(T, 64)
        o = oracle.qkv_heads(Y, M, C, heads, T, TpQ, TpK)
        for part, Tp in (("q", TpQ), ("k", TpK)):
            oracle.quant_heads_pad(B * heads, T, Tp, *o[part])
        qh, kh = o["q"], o["k"]
        vth, vtl, ev, _ = oracle.quant_v(o["v"], B, T, C, heads, TpK)
        a = self.attention_h(qh, (kh[0], kh[1], kh[2], vth, vtl, ev, T, TpK), B, heads, T, TpQ, C)
        h = self.linX(a, b + ".attn1.to_out.0", residual=h.d)
        # cross-attention (:428-435): to_q on the LayerNorm planes, k_quant_heads of q, the block's context K/V
        hi, lo, e = self.layernorm_q(h, b + ".norm2")
        q = self.linQ(hi, lo, e, B, T, b + ".attn2.to_q")
        Tqp = _r(T, 128)
        qq = oracle.quant_heads(q.d, B, T, C, heads, Tqp)
        a = self.attention_h(qq, self.cross[b], B, heads, T, Tqp, C)
        h = self.linX(a, b + ".attn2.to_out.0", residual=h.d)
        # feed-forward (:436-443): the interleaved GEGLU GEMM with row maxima, then ff.net.2 on the int32 rows
        hi, lo, e = self.layernorm_q(h, b + ".norm3")
        Wi, ci, Ni, _, _ = self.lin(b + ".ff.net.0.proj.agi")
        F = self.lins[b + ".ff.net.0.proj.a"][2]
        rm = np.zeros(M, np.uint32)
        v = oracle.gemm(oracle.SRC_I8, hi=hi, lo=lo, e=e, Mreal=M, Nreal=Ni, Kp=Wi.shape[1], w=Wi, cst=ci, epi=oracle.EPI_GEGLU,
                        Lphi=self.Lphi, rowmax=rm)
        assert v.shape[1] == F
        h = self.linX(Act(v, B, T, rowmax=rm), b + ".ff.net.2", residual=h.d, want_rowmax=True)
        # proj_out with the block's input as the residual (:444)
        return self.linX(h, p + ".proj_out", residual=x.d, gn_out=True)

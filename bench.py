#!/usr/bin/env python3
"""Benchmark of the MI355X W8A16 hi/lo integer GEMM (BASELINE.json metric).

One "step" is one launch of the headline GEMM: config C2, the GEGLU FF up-projection of a 64x64
latent at batch 8 (A int16 [32768 x 320], W int8 [2560 x 320] with interleaved a/g rows, per-column
requantisation, GEGLU epilogue to int32 [32768 x 1280] + per-row max). Inputs are seeded synthetic
data resident in HBM before the timed region. `value` is effective int8 TOPS = 4*M*N*K / time (two
int8 passes, 2 ops per MAC, real M, N, K), timed with HIP events on the launch stream.

Also reported on the same JSON line: the roofline of that kernel (the larger of its MFMA time at
5.0 POPS dense int8 and its HBM time at 8 TB/s bounds it), the HBM traffic per launch from the
committed rocprofv3 counter summary, the 194-GEMM UNet set (config C5) as one hipGraph in ms per
replay, every other config's time, and the CPU baseline: the oracle restatement of the reference's
integer semantics (the reference has no CPU GEMM of its own), timed on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-unet] [--no-cpu] [--no-configs]
       python bench.py --only {c1,c2,c2plain,c2view,c3,c4a,c4b,c4c,copy,norms,attention,unet<i>}   (one kernel, for profiler runs)
       python bench.py --unet-layers   (each C5 layer timed alone)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA, 5.0 POPS
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
METRIC = "effective W8A16 TOPS & % int8 MFMA peak; UNet GEMM-set ms at batch 8"


ONLY_NAMES = ("c1", "c2", "c2plain", "c2view", "c3", "c4a", "c4b", "c4c", "copy", "norms", "attention")
COPY_BYTES = 256 << 20       # the calibration copy of --only copy: 256 MiB read + 256 MiB written


def only_layer(name):
    from vela_amd import configs as cf

    if name.startswith("unet"):
        return cf.unet_layers()[int(name[4:])]
    return {"c1": cf.c1, "c2": lambda: cf.c2(cf.EPI_GEGLU), "c2plain": lambda: cf.c2(cf.EPI_PLAIN), "c3": cf.c3,
            "c4a": lambda: cf.c4()[0], "c4b": lambda: cf.c4()[1], "c4c": lambda: cf.c4()[2]}[name]()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_launches(fn, stream, steps, warmup):
    """Average duration of `fn` (which launches on `stream`) over `steps` back-to-back launches,
    from HIP events recorded on that stream."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        fn()
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def time_graphed(fn, stream, reps, replays):
    """Average duration of one `fn` call with no host launch cost in it: `reps` calls captured into one
    HIP graph on `stream`, replayed `replays` times between HIP events (after two untimed replays)."""
    import torch
    from vela_amd import gemm as vg

    g = vg.Graph(stream)
    g.begin()
    for _ in range(reps):
        fn()
    g.end()
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(replays):
        g.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    g.destroy()
    return t0.elapsed_time(t1) / (reps * replays)


def pmc_traffic():
    """HBM bytes per launch of the C2 kernel from the committed rocprofv3 counter summary, if present."""
    p = ROOT / "profiles" / "stripe16_kernel_c2_geglu_pmc.json"
    if p.exists():
        try:
            d = json.loads(p.read_text())
            return d.get("hbm_bytes_per_launch"), d.get("source")
        except (OSError, ValueError):
            return None, None
    return None, None


def roofline(ops, nbytes, seconds):
    """The roof that bounds a kernel is the larger of its MFMA time and its HBM time."""
    t_mfma = ops / (PEAK_INT8_TOPS * 1e12)
    t_hbm = nbytes / (PEAK_HBM_GBS * 1e9)
    if t_hbm > t_mfma:
        achieved = nbytes / seconds / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4)}
    achieved = ops / seconds / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
            "frac": round(achieved / PEAK_INT8_TOPS, 4)}


def vendor_planar_us(L, stream, steps=10, warmup=3):
    """hipBLASLt (torch._int_mm) on the int8 GEMM of the reference's planar route for this layer:
    the stacked [hi; lo] planes [2M x K] times W^T [K x N] -> int32 (src/engine.cu:155, 195, 212,
    276), without the separate epilogue or im2col passes that route also needs. A comparison point
    for the fused kernel, not part of the product."""
    import torch

    try:
        A = torch.randint(-128, 128, (2 * L.M, L.Kp), dtype=torch.int8, device="cuda")
        W = torch.randint(-128, 128, (L.Np, L.Kp), dtype=torch.int8, device="cuda")
        Wt = W.t()
        with torch.cuda.stream(stream):
            return round(time_launches(lambda: torch._int_mm(A, Wt), stream, steps, warmup) * 1e3, 2)
    except RuntimeError:
        return None


class ViewRun:
    """C2 with the int16 view as its output (vgemm_hl2_view): the row-maxima clear, the
    row-stationary kernel writing each chunk at its running exponent, and the fix-up pass; and, for
    comparison, the two-pass route (int32 Y + rowmax, then k_quant_rows)."""

    def __init__(self, prob):
        import torch
        from vela_amd import gemm as vg

        L = prob.L
        self.prob, self.L = prob, L
        F = L.Nout
        self.hi = torch.empty((L.M, F), dtype=torch.int8, device="cuda")
        self.lo = torch.empty_like(self.hi)
        self.e = torch.empty(L.M, dtype=torch.int32, device="cuda")
        nb = vg.view_workspace_bytes(L.M, L.N, L.Kp, L.epi)
        self.ws = torch.empty(nb // 4 + 64, dtype=torch.int32, device="cuda")
        self.E = vg.AEpi(epi=L.epi, Lphi=vg.ptr(prob.lphi), ws=vg.ptr(self.ws), ws_bytes=nb)
        # A + W + the int16 view + e + cst
        self.bytes = 2 * L.M * L.K + L.N * L.K + 2 * L.M * F + 4 * L.M + 16 * L.N

    def fused(self, stream):
        from vela_amd import gemm as vg

        p, L = self.prob, self.L
        vg.k_gemm_hl2_view(p.A, L.Mp, L.M, p.w, p.w.shape[1], L.Np, L.N, L.Kp, p.cst, self.E, self.hi, self.lo, self.e, L.Nout,
                           stream=stream)

    def two_pass(self, stream):
        from vela_amd import gemm as vg

        p, L = self.prob, self.L
        vg.fill_u32(p.rowmax, 0, stream=stream)
        p.run(stream=stream)
        vg.k_quant_rows(p.y, L.M, L.Nout, L.Nout, self.hi, self.lo, self.e, L.Nout, stream=stream)


def norms_lines(stream, steps, warmup):
    """GroupNorm of a UNet activation X [8, 4096, 320] (32 groups) as a resnet runs it after a GEMM
    that gathered the sum/min/max in its epilogue: fin1, the squared deviations (stats2: reads X),
    the row apply with SiLU and the pixel maxima (reads X, writes Y); and LayerNorm to the int16 view
    of the transformer input [8 * 4096, 320]. Bytes are the algorithmic reads and writes."""
    import torch
    from vela_amd import gemm as vg
    from vela_amd import norms as vn

    B, T, C, G = 8, 4096, 320, 32
    M = B * T
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    x = torch.randint(-(1 << 20), 1 << 20, (M, C), generator=g, device="cuda", dtype=torch.int32)
    gam = torch.randint(30000, 90000, (C,), generator=g, device="cuda", dtype=torch.int32)
    bet = torch.randint(-20000, 20000, (C,), generator=g, device="cuda", dtype=torch.int32)
    lut = torch.arange(2049, device="cuda", dtype=torch.int32) * 32
    gs = vg.gn_stats_alloc(B * G)
    y = torch.empty_like(x)
    pm = torch.empty(M, device="cuda", dtype=torch.int32)
    hi = torch.empty((M, C), device="cuda", dtype=torch.int8)
    lo = torch.empty_like(hi)
    e = torch.empty(M, device="cuda", dtype=torch.int32)
    vn.k_gn_stats1(x, B, T, C, G, gs)   # the records a producing GEMM's epilogue would leave
    torch.cuda.synchronize()

    def t_us(fn):
        return round(time_graphed(fn, stream, 20, max(2, steps // 20)) * 1e3, 2)

    xb = M * C * 4
    res = {}
    us = t_us(lambda: vn.k_gn_stats2(x, B, T, C, G, 100000, gs, stream=stream))
    res["gn_stats2 [8,4096,320]"] = {"us": us, "gbs": round(xb / (us * 1e-6) / 1e9, 1)}
    us = t_us(lambda: vn.k_gn_apply_row(x, B, T, C, G, gs, gam, bet, lut, y, pm, None, None, None, 0, stream=stream))
    res["gn_apply_row + SiLU + pm [8,4096,320]"] = {"us": us, "gbs": round((2 * xb + 4 * M) / (us * 1e-6) / 1e9, 1)}
    us = t_us(lambda: vn.k_gn_stats1(x, B, T, C, G, gs, stream=stream))
    res["gn_stats1 [8,4096,320]"] = {"us": us, "gbs": round(xb / (us * 1e-6) / 1e9, 1)}
    us = t_us(lambda: vn.k_lnorm_q(x, M, C, gam, bet, 100000, hi, lo, e, C, stream=stream))
    res["lnorm_q [32768,320] -> int16 view"] = {"us": us, "gbs": round((xb + 2 * M * C + 4 * M) / (us * 1e-6) / 1e9, 1)}
    return res


def attention_lines(stream, steps, warmup):
    """The exact attention of the UNet's transformer blocks (k_fused_attention), operands from
    seeded activations through k_quant_heads / k_quant_v: self-attention at 64x64 (B 8, 5 heads,
    4096 queries and keys) and 32x32 (10 heads, 1024), cross-attention to the 77-token context.
    ops: three passes of Q.K^T (four int8 plane products each) and one P.V (four), 2048 int8 ops
    per (query, key) pair -- the reference's own kernel structure (src/attn.cu:1-6)."""
    import numpy as np
    import torch

    from vela_amd import attention as va

    def t_us(fn):
        return round(time_graphed(fn, stream, 10, max(2, steps // 10)) * 1e3, 2)

    g = torch.Generator(device="cuda").manual_seed(0x41545431)
    # an exp table of the model's shape: Q30 at z = 0, falling by a factor e every 2^16 of z
    L = torch.from_numpy(np.round(np.exp(-np.arange(1025) * 1024.0 / 65536.0) * 2.0**30).astype(np.int64)).cuda()
    res = {}
    for name, B, heads, Tq, Tk in (("self 64x64", 8, 5, 4096, 4096), ("self 32x32", 8, 10, 1024, 1024), ("cross 64x64 -> 77", 8, 5, 4096, 77)):
        C, G = 64 * heads, B * heads
        Tqp, Tkp = (Tq + 63) // 64 * 64, (Tk + 63) // 64 * 64
        ops = {}
        for part, T, Tp in (("q", Tq, Tqp), ("k", Tk, Tkp)):
            X = (torch.randn((B * T, C), generator=g, device="cuda") * 3000).to(torch.int32)
            t = [torch.empty((G * Tp, 64), dtype=torch.int8, device="cuda") for _ in range(2)]
            t += [torch.empty(G * Tp, dtype=torch.int32, device="cuda")] + [torch.empty(G * Tp, dtype=torch.int64, device="cuda") for _ in range(3)]
            va.k_quant_heads(X, B, T, C, heads, Tp, *t)
            ops[part] = t
        Xv = (torch.randn((B * Tk, C), generator=g, device="cuda") * 30000).to(torch.int32)
        v = [torch.empty((G * 64, Tkp), dtype=torch.int8, device="cuda") for _ in range(2)]
        v += [torch.empty(G * 64, dtype=torch.int32, device="cuda"), torch.empty(G * 64, dtype=torch.int64, device="cuda")]
        va.k_quant_v(Xv, B, Tk, C, heads, Tkp, *v)
        out = torch.empty((B * Tq, C), dtype=torch.int32, device="cuda")
        q, k = ops["q"], ops["k"]
        run = lambda: va.k_fused_attention(q[0], q[1], q[2], q[3], q[4], k[0], k[1], k[2], k[5], v[0], v[1], v[2], v[3], B, heads, Tq, Tqp,   # noqa: E731
                                           Tk, Tkp, False, L, C, None, None, out, stream=stream)
        us = t_us(run)
        nops = 2048.0 * G * Tqp * Tkp
        res[f"{name}: B {B}, {heads} heads, Tq {Tq}, Tk {Tk}"] = {"us": us, "tops": round(nops / (us * 1e-6) / 1e12, 1),
                                                                 "mfma_frac": round(nops / (us * 1e-6) / 5e15, 4)}
    return res


def dropin_sources(stream, steps, warmup):
    """Time the A sources and routes the reference engine actually passes (src/engine.cu), on the
    BASELINE shapes, with seeded synthetic inputs resident in HBM:
      * SRC_X32: int32 rows quantised on load from their row maxima (linX, :162-175), C1 shape;
      * SRC_CONV32: an int32 NHWC image, implicit im2col (conv3's fused loader, :254-270), C3 shape,
        the GEMM alone, with the k_pixmax + k_conv_e passes before it, and given the pixel maxima
        (ASrc.rowmax) so that the GEMM derives the shifts itself;
      * SRC_I8: int8 hi/lo planes + per-row e (linQ, :148-159), C1 shape;
      * Gemm::run on the stacked [hi; lo] planes [2M x K] (the cuBLASLt route, :271-277), C3 shape,
        alone and as im2col3 + Gemm::run + k_epilogue;
      * the C4 512-row convolution through AEpi without a split-K workspace (what a caller of the
        reference's AEpi, which has none, runs), and through the route the reference engine itself
        takes for that Kp (im2col3 + Gemm::run + k_epilogue)."""
    import torch

    from vela_amd import configs as cf
    from vela_amd import gemm as vg

    g = torch.Generator(device="cuda").manual_seed(0x56454C41)
    dev = torch.device("cuda")

    def rbits(shape):
        bits = torch.randint(1, 32, shape, generator=g, device=dev, dtype=torch.int64)
        v = torch.randint(0, 2**31, shape, generator=g, device=dev, dtype=torch.int64) & ((1 << bits) - 1)
        return (v - (1 << (bits - 1))).to(torch.int32)

    def wcst(L):
        h = cf.make_host(L)
        return torch.from_numpy(h["w"]).to(dev), torch.from_numpy(h["cst"]).to(dev)

    def t_us(fn):
        with torch.cuda.stream(stream):
            return round(time_launches(fn, stream, steps, warmup) * 1e3, 2)

    out = {}
    # SRC_X32, C1 shape, residual (to_out / ff.net.2 add into the residual stream)
    L = cf.c1()
    w, cst = wcst(L)
    x = rbits((L.M, L.K))
    rm = x.to(torch.int64).abs().amax(1).to(torch.int32)
    y = torch.zeros((L.M, L.N), dtype=torch.int32, device=dev)
    A = vg.ASrc(src=vg.SRC_X32, x=vg.ptr(x), ldx=L.K, rowmax=vg.ptr(rm), K=L.K)
    E = vg.AEpi(epi=vg.EPI_PLAIN, Y=vg.ptr(y), ldy=L.N, residual=vg.ptr(y))
    us = t_us(lambda: vg.k_gemm_hl2(A, L.Mp, L.M, w, L.Kp, L.Np, L.N, L.Kp, cst, E, stream=stream))
    out["SRC_X32 linear 4096x320x320 + residual"] = {"us": us, "tops": round(L.ops / (us * 1e-6) / 1e12, 1),
                                                     "gbs_algorithmic": round((4 * L.M * L.K + L.N * L.K + 8 * L.M * L.N) / (us * 1e-6) / 1e9, 1)}
    # SRC_I8 planes, C1 shape
    hi = torch.randint(-128, 128, (L.Mp, L.Kp), generator=g, device=dev, dtype=torch.int8)
    lo = torch.randint(-128, 128, (L.Mp, L.Kp), generator=g, device=dev, dtype=torch.int8)
    e = torch.randint(0, 4, (L.Mp,), generator=g, device=dev, dtype=torch.int32)
    us = t_us(lambda: vg.k_gemm_hl(hi, lo, L.Kp, L.Mp, L.M, w, L.Kp, L.Np, L.N, L.Kp, cst, e, y, L.N, stream=stream))
    out["SRC_I8 planes linear 4096x320x320"] = {"us": us, "tops": round(L.ops / (us * 1e-6) / 1e12, 1),
                                                "gbs_algorithmic": round((2 * L.M * L.K + L.N * L.K + 4 * L.M * L.N) / (us * 1e-6) / 1e9, 1)}
    del x, rm, y, hi, lo, e
    # SRC_CONV32, C3 shape: GEMM alone, and pixmax + conv_e + GEMM
    L = cf.c3()
    w, cst = wcst(L)
    img = rbits((L.B, L.H, L.W, L.C)) >> 12   # 1..19-bit values: row shifts e from 0 to 4
    pm = torch.zeros(L.B * L.H * L.W, dtype=torch.int32, device=dev)
    e = torch.zeros(L.Mp, dtype=torch.int32, device=dev)
    y = torch.zeros((L.M, L.N), dtype=torch.int32, device=dev)
    vg.k_pixmax(img, L.B * L.H * L.W, L.C, pm)
    vg.k_conv_e(pm, L.B, L.H, L.W, 1, e)
    A = vg.ASrc(src=vg.SRC_CONV32, img=vg.ptr(img), H=L.H, W=L.W, C=L.C, stride=1, Ho=L.Ho, Wo=L.Wo, K=L.K, e=vg.ptr(e))
    E = vg.AEpi(epi=vg.EPI_PLAIN, Y=vg.ptr(y), ldy=L.N)
    gemm = lambda: vg.k_gemm_hl2(A, L.Mp, L.M, w, L.Kp, L.Np, L.N, L.Kp, cst, E, stream=stream)   # noqa: E731

    def conv_route():
        vg.k_pixmax(img, L.B * L.H * L.W, L.C, pm, stream=stream)
        vg.k_conv_e(pm, L.B, L.H, L.W, 1, e, stream=stream)
        gemm()

    # the pixel maxima from the producer (its AEpi.rowmax), the shifts derived inside the GEMM
    Apm = vg.ASrc(src=vg.SRC_CONV32, img=vg.ptr(img), H=L.H, W=L.W, C=L.C, stride=1, Ho=L.Ho, Wo=L.Wo, K=L.K, rowmax=vg.ptr(pm))
    gemm_pm = lambda: vg.k_gemm_hl2(Apm, L.Mp, L.M, w, L.Kp, L.Np, L.N, L.Kp, cst, E, stream=stream)   # noqa: E731

    us, us_all, us_pm = t_us(gemm), t_us(conv_route), t_us(gemm_pm)
    out["SRC_CONV32 conv3x3 [8,32,32,640]->640"] = {"us": us, "tops": round(L.ops / (us * 1e-6) / 1e12, 1),
                                                    "us_with_pixmax_conv_e": us_all, "us_shift_from_pixel_maxima": us_pm}
    # the cuBLASLt route: im2col3 planes + Gemm::run on [2M x K] + k_epilogue
    planes = torch.empty((2, L.Mp, L.Kp), dtype=torch.int8, device=dev)
    C = torch.empty((2 * L.Mp, L.Np), dtype=torch.int32, device=dev)
    ge = vg.Gemm()
    ge.init(32 << 20)   # the reference engine's Gemm::init(cfg.gemmWorkspace), 32 MiB (src/engine.h:56)
    run = lambda: ge.run(planes, L.Kp, 0, w, L.Kp, 0, C, L.Np, 0, 2 * L.Mp, L.Np, L.Kp, stream=stream)   # noqa: E731

    def planar_route():
        vg.k_pixmax(img, L.B * L.H * L.W, L.C, pm, stream=stream)
        vg.k_im2col3(img, pm, L.B, L.H, L.W, L.C, 1, planes[0], planes[1], e, L.Kp, stream=stream)
        run()
        vg.k_epilogue(C[:L.Mp], C[L.Mp:], L.M, L.N, L.Np, cst, e, y, L.N, stream=stream)

    us, us_all = t_us(run), t_us(planar_route)
    out["Gemm::run planar [2x8192 x 5760] x [640 x 5760]^T (C3 via im2col3)"] = {
        "us": us, "tops": round(L.ops / (us * 1e-6) / 1e12, 1), "us_im2col3_run_epilogue": us_all}
    del img, pm, e, y, planes, C
    # C4 512-row conv through AEpi without a workspace
    L = cf.c4()[1]
    p = cf.DeviceProblem(L, with_ws=False)
    p.reset()
    us = t_us(lambda: p.run(stream=stream))
    # ... and through the route the reference engine takes for it (Kp 11520 > customGemmMaxK 1536,
    # src/engine.cu:176,279-288): k_pixmax, k_im2col3 of the int32 image, Gemm::run on the stacked
    # planes with the engine's 32 MiB workspace, k_epilogue
    img = rbits((L.B, L.H, L.W, L.C))
    w, cst = wcst(L)
    pm = torch.empty(L.B * L.H * L.W, dtype=torch.int32, device=dev)
    e = torch.empty(L.Mp, dtype=torch.int32, device=dev)
    y = torch.empty((L.M, L.N), dtype=torch.int32, device=dev)
    planes = torch.empty((2, L.Mp, L.Kp), dtype=torch.int8, device=dev)
    C = torch.empty((2 * L.Mp, L.Np), dtype=torch.int32, device=dev)

    def engine_route():
        vg.k_pixmax(img, L.B * L.H * L.W, L.C, pm, stream=stream)
        vg.k_im2col3(img, pm, L.B, L.H, L.W, L.C, 1, planes[0], planes[1], e, L.Kp, stream=stream)
        ge.run(planes, L.Kp, 0, w, L.Kp, 0, C, L.Np, 0, 2 * L.Mp, L.Np, L.Kp, stream=stream)
        vg.k_epilogue(C[:L.Mp], C[L.Mp:], L.M, L.N, L.Np, cst, e, y, L.N, stream=stream)

    us_route = t_us(engine_route)
    out["C4 conv3x3 [8,8,8,1280]->1280, AEpi without workspace"] = {
        "us": us, "tops": round(L.ops / (us * 1e-6) / 1e12, 1),
        "us_engine_route_pixmax_im2col3_run_epilogue": us_route}
    del img, pm, e, y, planes, C, ge
    return out


def cpu_time(L, h, reps, rows=None):
    import numpy as np

    import oracle

    times = []
    for _ in range(reps):
        t = time.perf_counter()
        oracle.layer_reference(L, h, rows=rows)
        times.append(time.perf_counter() - t)
    return float(np.median(times))


def cpu_baseline(L, h, unet_fraction=4):
    """The oracle on this host: the full C2 GEMM (median of 5) at all cores and a 2048-row sample on
    one core, and the C5 set with every layer run on its first 1/unet_fraction rows (time scaled by
    M / rows: each output row costs the same)."""
    import oracle
    from vela_amd import configs as cf

    threads = oracle.lib().orc_get_threads()
    tmed = cpu_time(L, h, 5)
    oracle.set_threads(1)
    rows = 2048
    t1 = cpu_time(L, h, 1, rows=(0, rows))
    oracle.set_threads(0)
    out = {
        "value": round(L.ops / tmed / 1e12, 4), "unit": "TOPS", "cores": threads, "kind": "port",
        "sample": f"the full C2 GEMM ({L.M}x{L.K}x{L.N}, GEGLU + rowmax) by the C oracle (oracle/oracle.c, OpenMP "
                  f"over rows, {threads} threads), median of 5",
        "ms": round(tmed * 1e3, 2),
        "one_thread": {"value": round(L.ops * rows / L.M / t1 / 1e12, 5), "unit": "TOPS", "cores": 1,
                        "sample": f"first {rows} rows of C2"},
        "cpu": _cpu_model(),
    }
    if unet_fraction:
        total = 0.0
        t_all = time.perf_counter()
        for Lu in cf.unet_layers():
            hu = cf.make_host(Lu)
            r1 = max(1, -(-Lu.M // unet_fraction))
            total += cpu_time(Lu, hu, 1, rows=(0, r1)) * Lu.M / r1
        out["unet_gemm_set_ms"] = round(total * 1e3, 1)
        out["unet_sample"] = (f"all 194 C5 layers, each on its first ceil(M/{unet_fraction}) rows, time scaled by "
                              f"M/rows ({time.perf_counter() - t_all:.1f} s wall including input generation)")
    return out


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    # a long window: the GPU's clocks settle only after some milliseconds of sustained load, and a
    # window of a few launches catches a transient (C2: 88 us at 20 launches, 81.5 us sustained)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-unet", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true")
    ap.add_argument("--only", help="time one configuration only (for profiler runs): one of " + ", ".join(ONLY_NAMES) +
                    ", or unet<i> for layer i of the C5 set")
    ap.add_argument("--unet-layers", action="store_true", help="time each C5 layer alone (one JSON line per layer)")
    args = ap.parse_args()
    if args.only and args.only not in ONLY_NAMES and not (args.only.startswith("unet") and args.only[4:].isdigit()):
        ap.error(f"--only: unknown configuration {args.only}")
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the GEMM would shard by output rows "
              "with replicated weights and no communication). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    from vela_amd import configs as cf
    from vela_amd import gemm as vg

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)

    if args.only == "copy":
        # calibration kernel for the HBM byte counters: a plain device copy of known size
        src = torch.empty(COPY_BYTES // 4, dtype=torch.int32, device=dev).fill_(7)
        dst = torch.empty_like(src)
        with torch.cuda.stream(stream):
            t = time_launches(lambda: dst.copy_(src), stream, args.steps, args.warmup)
        log(f"[bench] copy {COPY_BYTES >> 20} MiB: {t * 1e3:.2f} us/launch, {2 * COPY_BYTES / (t * 1e-3) / 1e9:.0f} GB/s")
        print(json.dumps({"workload": "copy", "bytes_read": COPY_BYTES, "bytes_written": COPY_BYTES, "us": round(t * 1e3, 3)}), flush=True)
        return
    if args.unet_layers:
        total = 0.0
        for i, L in enumerate(cf.unet_layers()):
            p = cf.DeviceProblem(L)
            p.reset()
            torch.cuda.synchronize()
            t = time_launches(lambda: p.run(stream=stream), stream, args.steps, args.warmup)
            total += t
            print(json.dumps({"i": i, "layer": L.name, "kind": L.kind, "M": L.M, "K": L.K, "N": L.N, "epi": L.epi,
                              "residual": L.residual, "us": round(t * 1e3, 2),
                              "tops": round(L.ops / (t * 1e-3) / 1e12, 1)}), flush=True)
            del p
        log(f"[bench] C5 layers launched one at a time: {total:.3f} ms in total")
        return
    if args.only == "attention":
        res = attention_lines(stream, args.steps, args.warmup)
        log(f"[bench] attention: {res}")
        print(json.dumps({"workload": "exact attention, UNet transformer shapes", "lines": res}), flush=True)
        return
    if args.only == "norms":
        res = norms_lines(stream, args.steps, args.warmup)
        log(f"[bench] norms: {res}")
        print(json.dumps({"workload": "integer norms, UNet 64x64 activation", "lines": res}), flush=True)
        return
    if args.only == "c2view":
        L = cf.c2(cf.EPI_GEGLU)
        p = cf.DeviceProblem(L)
        p.reset()
        v = ViewRun(p)
        torch.cuda.synchronize()
        t = time_launches(lambda: v.fused(stream), stream, args.steps, args.warmup)
        log(f"[bench] C2 + int16 view: {t * 1e3:.2f} us/call")
        print(json.dumps({"workload": "C2 GEGLU -> int16 view", "us": round(t * 1e3, 3), "tops": round(L.ops / (t * 1e-3) / 1e12, 2)}), flush=True)
        return
    if args.only:
        L = only_layer(args.only)
        p = cf.DeviceProblem(L)
        p.reset()
        torch.cuda.synchronize()
        t = time_launches(lambda: p.run(stream=stream), stream, args.steps, args.warmup)
        log(f"[bench] {L.name}: {t * 1e3:.2f} us/launch, {L.ops / (t * 1e-3) / 1e12:.1f} TOPS")
        print(json.dumps({"workload": L.name, "us": round(t * 1e3, 3), "tops": round(L.ops / (t * 1e-3) / 1e12, 2)}), flush=True)
        return

    # ---- headline: C2 GEGLU
    L = cf.c2(cf.EPI_GEGLU)
    log(f"[bench] {L.name}: generating inputs")
    prob = cf.DeviceProblem(L)
    prob.reset()
    torch.cuda.synchronize()
    ms = time_launches(lambda: prob.run(stream=stream), stream, args.steps, args.warmup)
    tops = L.ops / (ms * 1e-3) / 1e12
    log(f"[bench] {L.name}: {ms * 1e3:.1f} us/launch, {tops:.1f} TOPS ({100 * tops / PEAK_INT8_TOPS:.1f}% of int8 peak)")
    traffic, traffic_src = pmc_traffic()

    vendor_c2 = vendor_planar_us(L, stream, args.steps, args.warmup)
    roof = roofline(L.ops, L.hbm_bytes, ms * 1e-3)
    roof["traffic"] = traffic
    roof.update({"traffic_source": traffic_src, "kernel": "vk::stripe16_kernel<SRC_I16, EPI_GEGLU>",
                 "algorithmic_ops_per_launch": L.ops, "algorithmic_bytes_per_launch": L.hbm_bytes,
                 "mfma_frac": round(tops / PEAK_INT8_TOPS, 4),
                 "hbm_frac": round(L.hbm_bytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})
    out = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded: Laplace(1500) int16 activations, Gaussian(40) int8 weights)",
        "config": {"workload": "C2: W8A16 GEGLU up-proj, A int16 [32768x320] x W int8 [320x2560] -> int32 [32768x1280] + rowmax",
                   "M": L.M, "K": L.K, "N": L.N, "epilogue": "GEGLU + rowmax", "source": "SRC_I16"},
        "pct_int8_peak": round(100 * tops / PEAK_INT8_TOPS, 2),
        "roofline": roof,
        "hipblaslt_planar_gemm_us": vendor_c2,
    }

    # ---- C2 with the int16 view (hi/lo planes + e) as its output, against its own roofline
    v = ViewRun(prob)
    torch.cuda.synchronize()
    tv = time_launches(lambda: v.fused(stream), stream, args.steps, args.warmup)
    t2 = time_launches(lambda: v.two_pass(stream), stream, max(5, args.steps // 4), max(2, args.warmup // 4))
    rv = roofline(L.ops, v.bytes, tv * 1e-3)
    rv.update({"algorithmic_bytes_per_launch": v.bytes, "hbm_floor_us": round(v.bytes / (PEAK_HBM_GBS * 1e9) * 1e6, 2),
               "mfma_floor_us": round(L.ops / (PEAK_INT8_TOPS * 1e12) * 1e6, 2),
               "hbm_frac": round(v.bytes / (tv * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})
    out["c2_int16_view"] = {"workload": "C2 GEGLU -> int16 view (hi/lo [32768x1280] + e), quant_row_out semantics",
                            "us": round(tv * 1e3, 2), "tops": round(L.ops / (tv * 1e-3) / 1e12, 2), "roofline": rv,
                            "us_two_pass_int32_then_quant_rows": round(t2 * 1e3, 2)}
    log(f"[bench] C2 + int16 view: {out['c2_int16_view']}")
    del v

    # ---- the other configurations (one line each in "configs")
    if not args.no_configs:
        table = {}
        for Lc in [cf.c1(), cf.c2(cf.EPI_PLAIN), cf.c3(), *cf.c4()]:
            p = cf.DeviceProblem(Lc)
            p.reset()
            torch.cuda.synchronize()
            t = time_launches(lambda: p.run(stream=stream), stream, max(5, args.steps), args.warmup)
            table[Lc.name] = {"us": round(t * 1e3, 2), "tops": round(Lc.ops / (t * 1e-3) / 1e12, 2),
                              "pct_int8_peak": round(100 * Lc.ops / (t * 1e-3) / 1e12 / PEAK_INT8_TOPS, 2),
                              "gbs_algorithmic": round(Lc.hbm_bytes / (t * 1e-3) / 1e9, 1),
                              "roofline": roofline(Lc.ops, Lc.hbm_bytes, t * 1e-3)}
            table[Lc.name]["hipblaslt_planar_gemm_us"] = vendor_planar_us(Lc, stream, max(5, args.steps), args.warmup)
            if not args.no_cpu:
                table[Lc.name]["cpu_ms"] = round(cpu_time(Lc, p.h, 3) * 1e3, 2)
            log(f"[bench] {Lc.name}: {table[Lc.name]}")
            del p
        out["configs"] = table

    # ---- the A sources and routes a drop-in caller passes
    if not args.no_configs:
        out["dropin_sources"] = dropin_sources(stream, max(5, args.steps // 4), max(2, args.warmup // 4))
        log(f"[bench] drop-in sources: {out['dropin_sources']}")

    # ---- the integer normalisations around the GEMMs, at the UNet's 64x64 resolution
    if not args.no_configs:
        out["norms"] = norms_lines(stream, max(5, args.steps // 4), max(2, args.warmup // 4))
        log(f"[bench] norms: {out['norms']}")

    # ---- the exact attention of the transformer blocks
    if not args.no_configs:
        out["attention"] = attention_lines(stream, max(5, args.steps // 4), max(2, args.warmup // 4))
        log(f"[bench] attention: {out['attention']}")

    # ---- C5: the UNet GEMM set as one graph
    if not args.no_unet:
        from vela_amd.unet import GemmSet

        log("[bench] C5: building the 194-GEMM UNet set")
        gs = GemmSet()
        gs.capture(reseed=False)   # GEMMs + rowmax fills only: no residual re-seeding copies
        t = time_launches(gs.replay, gs.stream, max(5, min(100, args.steps // 2)), max(2, min(10, args.warmup // 20)))
        out["unet_gemm_set_ms"] = round(t, 4)
        out["unet_gemm_set"] = {"gemms": len(gs.layers), "ms": round(t, 4), "tops": round(gs.ops / (t * 1e-3) / 1e12, 2),
                                "pct_int8_peak": round(100 * gs.ops / (t * 1e-3) / 1e12 / PEAK_INT8_TOPS, 2),
                                "ideal_mfma_ms": round(gs.ops / (PEAK_INT8_TOPS * 1e12) * 1e3, 4)}
        log(f"[bench] C5: {out['unet_gemm_set']}")
        del gs

    # ---- CPU baseline (rank 0, N = 1)
    if not args.no_cpu:
        log("[bench] CPU baseline (oracle)")
        out["cpu_baseline"] = cpu_baseline(L, prob.h, unet_fraction=0 if args.no_unet else 4)
        out["gpu_over_cpu"] = round(tops / out["cpu_baseline"]["value"], 1)
        if "unet_gemm_set_ms" in out and "unet_gemm_set_ms" in out["cpu_baseline"]:
            out["unet_gpu_over_cpu"] = round(out["cpu_baseline"]["unet_gemm_set_ms"] / out["unet_gemm_set_ms"], 1)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

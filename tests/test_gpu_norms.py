"""GPU parity of the integer normalisations (vela_amd.norms over the C ABI) against the oracle
(oracle/oracle.c: orc_gn_*, orc_lnorm*): GroupNorm statistics, finalisation, the row apply with and
without the SiLU table and the int16 view, the elementwise apply, LayerNorm, on the input kinds of the
reference's own test (src/test_normalization.cpp: zeros, +-1e6, full int32 range with INT_MIN /
INT_MAX, random g and beta, e = 12); and the chain a UNet resnet runs: a GEMM gathering GroupNorm
statistics in its epilogue, fin1, the squared deviations, the apply with the pixel maxima, and the
following 3x3 convolution taking those maxima instead of e."""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_equal, to_np
from tests.test_gpu_gemm import Case, dev
from vela_amd import gemm as vg
from vela_amd import norms as vn

pytestmark = pytest.mark.gpu

FIELDS = ("sum", "mn", "mx", "mean", "e", "ss", "sd")


def records_dev(gs_np):
    return torch.from_numpy(gs_np.view(np.uint8).copy()).cuda()


def records_np(gs_dev):
    return to_np(gs_dev).view(oracle.GN_DTYPE).copy()


def check_records(got, want, what, fields=FIELDS):
    for f in fields:
        assert_equal(got[f], want[f], f"{what} {f}")


def make_x(r, M, C, mode):
    if mode == 0:
        return np.zeros((M, C), np.int32)
    if mode == 1:
        return r.integers(-1000000, 1000001, (M, C)).astype(np.int32)
    x = r.integers(-(2**31), 2**31, (M, C), dtype=np.int64).astype(np.int32)
    x[0, 0], x[0, 1] = -(2**31), 2**31 - 1
    return x


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("B,T,C,groups", [(2, 5, 64, 32), (2, 300, 320, 32), (1, 64, 1280, 32), (2, 77, 2560, 32), (3, 129, 96, 8),
                                          (2, 77, 1280, 64), (1, 64, 2560, 64), (2, 9, 128, 64)])
def test_gn_stats(gpu, mode, B, T, C, groups):
    r = np.random.default_rng(mode + 3 * C + T)
    x = make_x(r, B * T, C, mode)
    want = oracle.gn_stats1(x, B, T, C, groups)
    gs = vg.gn_stats_alloc(B * groups)
    X = dev(x)
    vn.k_gn_stats1(X, B, T, C, groups, gs)
    torch.cuda.synchronize()
    check_records(records_np(gs), want, f"stats1 mode {mode} {B}x{T}x{C}", ("sum", "mn", "mx", "mean", "e"))
    den = 100000
    oracle.gn_stats2(x, B, T, C, groups, den, want)
    vn.k_gn_stats2(X, B, T, C, groups, den, gs)
    torch.cuda.synchronize()
    check_records(records_np(gs), want, f"stats2 mode {mode} {B}x{T}x{C}")
    # ss accumulates, as the reference's atomicAdd does (src/kernels.cu:201): a repeat adds it again
    oracle.gn_stats2(x, B, T, C, groups, den, want)
    vn.k_gn_stats2(X, B, T, C, groups, den, gs)
    torch.cuda.synchronize()
    check_records(records_np(gs), want, f"stats2 twice mode {mode} {B}x{T}x{C}")


@pytest.mark.parametrize("C", [32, 64, 128, 320, 512, 640, 960, 1024, 1280, 1920, 2560])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_gn_apply_row_reference_cases(gpu, C, mode):
    """src/test_normalization.cpp:17-36: B 2, T 5, 32 groups, supplied statistics; every combination
    of the SiLU table and the int16 view."""
    r = np.random.default_rng(20261022 + C * 3 + mode)
    B, T, groups = 2, 5, 32
    M, Kp = B * T, (C + 15) // 16 * 16
    x = make_x(r, M, C, mode)
    g = (r.integers(-(2**31), 2**31, C, dtype=np.int64) if mode == 2 else np.full(C, 65536)).astype(np.int32)
    beta = (r.integers(-(2**31), 2**31, C, dtype=np.int64) if mode == 2 else np.zeros(C)).astype(np.int32)
    L = (np.arange(2049) * 32).astype(np.int32)
    st = oracle.gn_records(B * groups)
    st["mean"] = 0 if mode == 0 else (r.integers(-500000, 500001, B * groups) if mode == 1 else r.integers(-(2**31), 2**31, B * groups, dtype=np.int64))
    st["e"] = 12 if mode == 2 else 0
    st["sd"] = 65536 + r.integers(0, 100000000, B * groups)
    X, G, Bt, Ld, S = dev(x), dev(g), dev(beta), dev(L), records_dev(st)
    for act in (False, True):
        for quant in (False, True):
            what = f"C={C} mode={mode} act={act} quant={quant}"
            if quant:
                want = oracle.gn_apply_row(x, B, T, C, groups, st, g, beta, Lsig=L if act else None, Kp=Kp)
                hi = torch.full((M, Kp), 0x5a, dtype=torch.int8, device="cuda")
                lo = torch.full((M, Kp), 0x5a, dtype=torch.int8, device="cuda")
                e = torch.full((M,), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
                vn.k_gn_apply_row(X, B, T, C, groups, S, G, Bt, Ld if act else None, None, None, hi, lo, e, Kp)
                torch.cuda.synchronize()
                for got, w, n in zip((hi, lo, e), want, ("hi", "lo", "e")):
                    assert_equal(to_np(got), w, f"{what} {n}")
            else:
                Yw, pmw = oracle.gn_apply_row(x, B, T, C, groups, st, g, beta, Lsig=L if act else None)
                Y = torch.full((M, C), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
                pm = torch.full((M,), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
                vn.k_gn_apply_row(X, B, T, C, groups, S, G, Bt, Ld if act else None, Y, pm, None, None, None, 0)
                torch.cuda.synchronize()
                assert_equal(to_np(Y), Yw, f"{what} Y")
                assert_equal(to_np(pm).view(np.uint32), pmw, f"{what} pm")
    if C <= 640:
        Y = torch.zeros((M, C), dtype=torch.int32, device="cuda")
        vn.k_gn_apply(X, B, T, C, groups, S, dev(g.astype(np.int64)), dev(beta.astype(np.int64)), Y)
        torch.cuda.synchronize()
        assert_equal(to_np(Y), oracle.gn_apply(x, B, T, C, groups, st, g.astype(np.int64), beta.astype(np.int64)), f"gn_apply C={C} mode={mode}")


@pytest.mark.parametrize("B,T,C,groups", [(2, 77, 1280, 64), (1, 64, 2560, 64), (2, 5, 64, 64), (3, 10, 96, 48)])
def test_gn_apply_many_groups(gpu, B, T, C, groups):
    """The elementwise k_gn_apply with more than 32 groups (up to 64): statistics from k_gn_stats1/2,
    every element against the oracle. (The row kernel, like the reference's, takes at most 32.)"""
    r = np.random.default_rng(B * T + C + groups)
    x = make_x(r, B * T, C, 1)
    den = 100000
    st = oracle.gn_stats1(x, B, T, C, groups)
    oracle.gn_stats2(x, B, T, C, groups, den, st)
    g = r.integers(30000, 90000, C).astype(np.int64)
    beta = r.integers(-20000, 20000, C).astype(np.int64)
    X = dev(x)
    gs = vg.gn_stats_alloc(B * groups)
    vn.k_gn_stats1(X, B, T, C, groups, gs)
    vn.k_gn_stats2(X, B, T, C, groups, den, gs)
    Y = torch.zeros((B * T, C), dtype=torch.int32, device="cuda")
    vn.k_gn_apply(X, B, T, C, groups, gs, dev(g), dev(beta), Y)
    torch.cuda.synchronize()
    check_records(records_np(gs), st, f"records {groups} groups C={C}")
    assert_equal(to_np(Y), oracle.gn_apply(x, B, T, C, groups, st, g, beta), f"gn_apply {groups} groups C={C}")


@pytest.mark.parametrize("C", [4, 12, 124, 128, 132, 320, 512, 640, 768, 1024, 1280, 2560])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_lnorm(gpu, C, mode):
    """src/test_normalization.cpp:70-100: M 9 rows, den 100000, both outputs."""
    r = np.random.default_rng(20261021 + C + 7 * mode)
    M, den, Kp = 9, 100000, (C + 15) // 16 * 16
    x = make_x(r, M, C, mode)
    g = (r.integers(-(2**31), 2**31, C, dtype=np.int64) if mode == 2 else np.full(C, 65536)).astype(np.int32)
    beta = (r.integers(-(2**31), 2**31, C, dtype=np.int64) if mode == 2 else np.zeros(C)).astype(np.int32)
    X = dev(x)
    hi = torch.full((M, Kp), 0x5a, dtype=torch.int8, device="cuda")
    lo = torch.full((M, Kp), 0x5a, dtype=torch.int8, device="cuda")
    e = torch.full((M,), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
    vn.k_lnorm_q(X, M, C, dev(g), dev(beta), den, hi, lo, e, Kp)
    Y = torch.zeros((M, C), dtype=torch.int32, device="cuda")
    vn.k_lnorm(X, M, C, dev(g.astype(np.int64)), dev(beta.astype(np.int64)), den, Y)
    torch.cuda.synchronize()
    for got, w, n in zip((hi, lo, e), oracle.lnorm_q(x, M, C, g, beta, den, Kp), ("hi", "lo", "e")):
        assert_equal(to_np(got), w, f"lnorm_q C={C} mode={mode} {n}")
    assert_equal(to_np(Y), oracle.lnorm(x, M, C, g.astype(np.int64), beta.astype(np.int64), den), f"lnorm C={C} mode={mode}")


def test_resnet_chain(gpu):
    """GEMM with GroupNorm statistics in its epilogue (T = 256 rows per sample) -> fin1 -> stats2 ->
    apply_row with SiLU and the pixel maxima -> 3x3 convolution (SRC_CONV32) taking the maxima as
    ASrc.rowmax: every stage against the oracle."""
    B, H, W, C = 2, 16, 16, 64
    T, groups, den = H * W, 32, 100000
    c = Case(vg.SRC_I16, B * T, C, 320, seed=77, s_range=(14, 20))
    Yg = torch.zeros((c.M, C), dtype=torch.int32, device="cuda")
    gs = vg.gn_stats_alloc(B * groups)
    vg.k_gn_init(gs, B * groups)
    keep = {}
    A = c.asrc(keep)
    E = vg.AEpi(epi=vg.EPI_PLAIN, Y=vg.ptr(Yg), ldy=C, gnstat=vg.ptr(gs), gnT=T)
    vg.k_gemm_hl2(A, c.Mp, c.M, dev(c.w), c.Kp, c.Np, c.N, c.Kp, dev(c.cst), E)
    vn.k_gn_fin1(gs, B * groups, T * (C // groups))
    vn.k_gn_stats2(Yg, B, T, C, groups, den, gs)
    r = np.random.default_rng(3)
    g = r.integers(30000, 90000, C).astype(np.int32)
    beta = r.integers(-20000, 20000, C).astype(np.int32)
    L = (np.arange(2049) * 32).astype(np.int32)
    Xn = torch.zeros((c.M, C), dtype=torch.int32, device="cuda")
    pm = torch.zeros(c.M, dtype=torch.int32, device="cuda")
    vn.k_gn_apply_row(Yg, B, T, C, groups, gs, dev(g), dev(beta), dev(L), Xn, pm, None, None, None, 0)
    torch.cuda.synchronize()
    # the oracle's chain
    y, _ = c.reference()
    assert_equal(to_np(Yg), y, "GEMM Y")
    fused = oracle.gn_stats_fused(y, c.M, C, T, c.Mp, c.Np, c.Kp, oracle.SRC_I16)
    st = oracle.gn_records(B * groups)
    for f in ("sum", "mn", "mx"):
        st[f] = fused[f]
    oracle.gn_fin1(st, T * (C // groups))
    oracle.gn_stats2(y, B, T, C, groups, den, st)
    check_records(records_np(gs)[: B * groups], st, "chain records")
    xw, pmw = oracle.gn_apply_row(y, B, T, C, groups, st, g, beta, Lsig=L)
    assert_equal(to_np(Xn), xw, "chain apply")
    assert_equal(to_np(pm).view(np.uint32), pmw, "chain pixel maxima")
    # the 3x3 convolution of the normalised image, its shifts from the pixel maxima
    conv = Case(vg.SRC_CONV32, B * T, 128, 9 * C, seed=78, conv=(B, H, W, C, 1))
    conv.img = xw.reshape(B, H, W, C)
    conv.kw["img"] = conv.img
    conv.pm = pmw
    conv.e = oracle.conv_e(pmw, B, H, W, 1)
    conv.pm_in_kernel = True
    conv.check(what="chain conv")


@pytest.mark.parametrize("table", ["small_random", "large_random"])
def test_gn_apply_row_silu_tables(gpu, table):
    """The SiLU tail with non-monotone tables: entries within 2^20 (the double form, decreasing segments
    included) and entries up to 2^31 (the exact 32-bit wrapping interpolation)."""
    r = np.random.default_rng(7 if table == "small_random" else 8)
    B, T, C, groups = 2, 37, 320, 32
    M, Kp = B * T, 336
    x = make_x(r, M, C, 1)
    g = r.integers(-200000, 200000, C).astype(np.int32)
    beta = r.integers(-(2**20), 2**20, C).astype(np.int32)
    lim = 2**20 - 1 if table == "small_random" else 2**31 - 1
    L = r.integers(-lim, lim + 1, 2049, dtype=np.int64).astype(np.int32)
    st = oracle.gn_records(B * groups)
    st["mean"] = r.integers(-500000, 500001, B * groups)
    st["e"] = 0
    st["sd"] = 65536 + r.integers(0, 10000000, B * groups)
    X, G, Bt, Ld, S = dev(x), dev(g), dev(beta), dev(L), records_dev(st)
    Yw, pmw = oracle.gn_apply_row(x, B, T, C, groups, st, g, beta, Lsig=L)
    Y = torch.full((M, C), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
    pm = torch.full((M,), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
    vn.k_gn_apply_row(X, B, T, C, groups, S, G, Bt, Ld, Y, pm, None, None, None, 0)
    hi = torch.full((M, Kp), 0x5a, dtype=torch.int8, device="cuda")
    lo = torch.full((M, Kp), 0x5a, dtype=torch.int8, device="cuda")
    e = torch.full((M,), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
    vn.k_gn_apply_row(X, B, T, C, groups, S, G, Bt, Ld, None, None, hi, lo, e, Kp)
    torch.cuda.synchronize()
    assert_equal(to_np(Y), Yw, f"{table} Y")
    assert_equal(to_np(pm).view(np.uint32), pmw, f"{table} pm")
    for got, w, n in zip((hi, lo, e), oracle.gn_apply_row(x, B, T, C, groups, st, g, beta, Lsig=L, Kp=Kp), ("hi", "lo", "e")):
        assert_equal(to_np(got), w, f"{table} {n}")

"""The int16 view of a GEMM's output (vgemm_hl2_view): the row-stationary kernel's speculative
per-chunk quantisation plus the fix-up pass must give exactly the reference's quant_row_out
(src/kernels.cu:317-331) of the GEMM's int32 output -- e = row_exp(max |y|), q = quant16_32(y, e),
hi = q >> 8, lo = (q & 255) - 128, pad columns (0, -128) -- checked against the oracle's
k_quant_rows of its own GEMM output and, for GEGLU, against its k_epilogue_geglu_q on the planar
(cuBLASLt-route) partials of the same product."""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_equal, to_np
from tests.test_gpu_gemm import Case, dev, make_w_cst, rng
from vela_amd import configs as cf
from vela_amd import gemm as vg
from vela_amd._lib import VgemmError

pytestmark = pytest.mark.gpu


def run_view(c: Case, vld: int):
    """The view of Case c on the GPU: (hi, lo, e) as numpy arrays."""
    keep = {}
    A = c.asrc(keep)
    w, cst, lut = dev(c.w), dev(c.cst), dev(c.lut)
    hi = torch.full((c.M, vld), 0x55, dtype=torch.int8, device="cuda")
    lo = torch.full((c.M, vld), 0x55, dtype=torch.int8, device="cuda")
    e = torch.full((c.M,), -7, dtype=torch.int32, device="cuda")
    nb = vg.view_workspace_bytes(c.M, c.N, c.Kp, c.epi)
    ws = torch.empty(nb // 4 + 64, dtype=torch.int32, device="cuda")
    E = vg.AEpi(epi=c.epi, Lphi=vg.ptr(lut), ws=vg.ptr(ws), ws_bytes=nb)
    vg.k_gemm_hl2_view(A, c.Mp, c.M, w, c.Kp, c.Np, c.N, c.Kp, cst, E, hi, lo, e, vld)
    torch.cuda.synchronize()
    return to_np(hi), to_np(lo), to_np(e)


def expect_view(c: Case, vld: int):
    Y, _ = c.reference()
    hi, lo, e = oracle.quant_rows(Y, c.M, c.nout, c.nout, vld)
    return hi[:c.M], lo[:c.M], e[:c.M]


def check(c: Case, vld: int, what: str):
    got = run_view(c, vld)
    want = expect_view(c, vld)
    for g, w_, name in zip(got, want, ("hi", "lo", "e")):
        assert_equal(g, w_, f"{what} {name}")
    return got


@pytest.mark.parametrize("src", [vg.SRC_I16, vg.SRC_I8])
@pytest.mark.parametrize("epi,M,N,K,vld", [
    (vg.EPI_GEGLU, 3000, 2560, 320, 1280),     # C2's columns and depth, fewer rows
    (vg.EPI_GEGLU, 777, 640, 320, 352),        # ragged rows, padded view
    (vg.EPI_PLAIN, 1000, 320, 320, 320),
    (vg.EPI_PLAIN, 257, 200, 64, 208),         # a partial 32-column group, padded
    (vg.EPI_GELU, 640, 1280, 96, 1280),
])
def test_view_matches_quant_rows(src, epi, M, N, K, vld):
    c = Case(src, M, N, K, epi=epi, seed=M + N + K + src)
    check(c, vld, f"view src {src} epi {epi} {M}x{N}x{K}")


@pytest.mark.parametrize("src", [vg.SRC_I16, vg.SRC_I8])
@pytest.mark.parametrize("epi,M,N,K,vld", [
    (vg.EPI_GEGLU, 600, 5120, 640, 2560),      # the UNet's GEGLU up-projection at 640 channels (Kp 640)
    (vg.EPI_GEGLU, 256, 10240, 1280, 5120),    # at 1280 channels (Kp 1280)
    (vg.EPI_PLAIN, 300, 640, 1280, 656),       # padded view
    (vg.EPI_GELU, 130, 256, 4096, 256),        # deep K over few tiles: split-K in the workspace's tail
])
def test_view_deep_k(src, epi, M, N, K, vld):
    """Kp > 320: the GEMM's int32 rows in the workspace, then their quantisation."""
    c = Case(src, M, N, K, epi=epi, seed=M + K + src, s_range=(18, 26))
    check(c, vld, f"deep-K view src {src} epi {epi} {M}x{N}x{K}")


def test_view_exponent_grows_across_chunks():
    """Rows whose outputs grow from column to column, so that almost every group was written at a
    smaller running exponent (from e = 0 up) and is rewritten by the fix-up pass; and rows of zeros."""
    M, N, K = 512, 1280, 320
    c = Case(vg.SRC_I16, M, N, K, epi=vg.EPI_PLAIN, seed=3, s_range=(24, 24))
    # m grows with the column: 2^4 .. 2^30
    c.cst[:N, 0] = (np.int64(1) << np.linspace(4, 30, N).astype(np.int64)).astype(np.int64).clip(max=2**31 - 1).astype(np.int32)
    c.cst[:N, 2] = 0
    c.q[:64] = 0            # zero rows: y = 0 everywhere, e = 0
    c.q[64:128] = 1         # tiny rows
    check(c, N, "growing exponents")


def test_view_exact_form():
    """Per-row shifts e (and shifts outside [0, 31]) send blocks to the kernel's int64 form."""
    c = Case(vg.SRC_I16, 640, 640, 320, epi=vg.EPI_GEGLU, seed=9, e_max=17, s_range=(10, 40))
    check(c, 320, "exact form")
    c = Case(vg.SRC_I8, 384, 256, 192, epi=vg.EPI_PLAIN, seed=10, s_range=(-3, 45), m_range=(-(2**31), 2**31 - 1))
    check(c, 256, "exact form, saturating")


def test_view_matches_planar_geglu_q():
    """GEGLU view over interleaved a/g rows == k_epilogue_geglu_q (src/kernels.cu:499-534) on the
    planar partials of [W_a; W_g] (the cuBLASLt route's layout)."""
    r = rng(21)
    M, F, K = 300, 320, 320
    Kp = cf.align(K, 16)
    wa, ca = make_w_cst(r, F, K, F, Kp)
    wg, cg = make_w_cst(r, F, K, F, Kp)
    wi, ci = oracle.interleave2(wa, ca, wg, cg, F, Kp)
    c = Case(vg.SRC_I16, M, 2 * F, K, epi=vg.EPI_GEGLU, seed=22)
    c.w, c.cst = wi, ci
    got = run_view(c, F)
    Chi, Clo = oracle.planes(oracle.SRC_I16, Mreal=M, Nreal=2 * F, Kp=Kp, w=np.concatenate([wa, wg]), q16=c.q, K=K)
    want = oracle.epilogue_geglu_q(Chi, Clo, M, F, 2 * F, np.concatenate([ca, cg]), np.zeros(M, np.int32), c.lut, F)
    for g, w_, name in zip(got, want, ("hi", "lo", "e")):
        assert_equal(g, w_, f"planar geglu_q {name}")


def test_view_c2_full_rows_sampled():
    """The C2 configuration (32768 x 320 x 2560, GEGLU) at full size: every row's e and three
    row blocks of the planes against the oracle, and the view against the int32 run's own rows."""
    L = cf.c2(cf.EPI_GEGLU)
    p = cf.DeviceProblem(L)
    p.reset()
    p.run()
    torch.cuda.synchronize()
    y = to_np(p.y)
    F = L.Nout
    hi = torch.empty((L.M, F), dtype=torch.int8, device="cuda")
    lo = torch.empty_like(hi)
    e = torch.empty(L.M, dtype=torch.int32, device="cuda")
    nb = vg.view_workspace_bytes(L.M, L.N, L.Kp, L.epi)
    ws = torch.empty(nb // 4 + 64, dtype=torch.int32, device="cuda")
    E2 = vg.AEpi(epi=L.epi, Lphi=vg.ptr(p.lphi), ws=vg.ptr(ws), ws_bytes=nb)
    vg.k_gemm_hl2_view(p.A, L.Mp, L.M, p.w, p.w.shape[1], L.Np, L.N, L.Kp, p.cst, E2, hi, lo, e, F)
    torch.cuda.synchronize()
    # the view of the (separately oracle-checked) int32 output, all rows
    qh, ql, qe = oracle.quant_rows(y, L.M, F, F, F)
    assert_equal(to_np(e), qe[:L.M], "C2 view e")
    assert_equal(to_np(hi), qh[:L.M], "C2 view hi")
    assert_equal(to_np(lo), ql[:L.M], "C2 view lo")
    # and the int32 output itself on three row blocks against the oracle
    for r0 in (0, 16384, L.M - 64):
        want, _ = oracle.layer_reference(L, p.h, rows=(r0, r0 + 64))
        assert_equal(y[r0:r0 + 64], want[r0:r0 + 64], f"C2 rows {r0}")


def test_view_and_plain_call_agree():
    """The view call and a plain call of the same GEMM on the same inputs: Y of the plain call is
    left untouched by the view call, and the view is the quantisation of that Y."""
    c = Case(vg.SRC_I16, 2048, 2560, 320, epi=vg.EPI_GEGLU, seed=31)
    y, _ = c.run_gpu()
    hi, lo, e = run_view(c, 1280)
    qh, ql, qe = oracle.quant_rows(y, c.M, c.nout, c.nout, 1280)
    for g, w_, name in zip((hi, lo, e), (qh[:c.M], ql[:c.M], qe[:c.M]), ("hi", "lo", "e")):
        assert_equal(g, w_, f"view of the plain call's Y {name}")


def test_view_errors():
    c = Case(vg.SRC_I16, 256, 128, 64, epi=vg.EPI_PLAIN, seed=1)
    keep = {}
    A = c.asrc(keep)
    w, cst = dev(c.w), dev(c.cst)
    hi = torch.empty((256, 128), dtype=torch.int8, device="cuda")
    lo, e = torch.empty_like(hi), torch.empty(256, dtype=torch.int32, device="cuda")
    run = lambda E, ld=128, a=A, d=c: vg.k_gemm_hl2_view(a, d.Mp, d.M, w if d is c else dev(d.w), d.Kp, d.Np, d.N, d.Kp,
                                                          cst if d is c else dev(d.cst), E, hi, lo, e, ld)
    with pytest.raises(VgemmError, match="needs a workspace"):
        run(vg.AEpi(epi=vg.EPI_PLAIN))
    ws = torch.empty(1 << 20, dtype=torch.int32, device="cuda")
    with pytest.raises(VgemmError, match="no residual"):
        run(vg.AEpi(epi=vg.EPI_PLAIN, residual=vg.ptr(e), ws=vg.ptr(ws), ws_bytes=4 << 20))
    with pytest.raises(VgemmError, match="ld >= output columns"):
        run(vg.AEpi(epi=vg.EPI_PLAIN, ws=vg.ptr(ws), ws_bytes=4 << 20), ld=120)
    d = Case(vg.SRC_I16, 256, 128, 640, epi=vg.EPI_PLAIN, seed=2)
    keep2 = {}
    need = vg.view_workspace_bytes(256, 128, d.Kp, vg.EPI_PLAIN)
    with pytest.raises(VgemmError, match="needs a workspace"):
        run(vg.AEpi(epi=vg.EPI_PLAIN, ws=vg.ptr(ws), ws_bytes=need - 16), a=d.asrc(keep2), d=d)

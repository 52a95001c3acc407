"""GPU parity of the EPI_QKV epilogue and of the GroupNorm statistics (EPI_PLAIN with gnstat, and the
planar k_epilogue with gs) against the CPU oracle, byte for byte.

QKV follows its use in src/engine.cu:318-330: rows B*T, N = 3C with C = 64*heads, q into planes of
TpQ = align(T, 128) rows per (sample, head), k into TpK = align(T, 64); every output buffer starts
filled with 0x5A bytes, so rows t >= T must come back untouched. The statistics follow
src/engine.cu:431-440 (a residual GEMM that also feeds the next GroupNorm): records initialised by
k_gn_init, sample lengths that put two samples in one 128-row tile (T = 64, 192), and every kernel
family that serves EPI_PLAIN (DMA tiles, register tiles for int32 sources, the halo 3x3 kernel).
"""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_equal, to_np
from tests.test_gpu_gemm import Case, dev
from vela_amd import configs as cf
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu

FILL = 0x5A


@pytest.fixture(autouse=True)
def _knobs(gpu):
    vg.set_variant(-1)
    vg.set_splitk(0)
    yield
    vg.set_variant(-1)
    vg.set_splitk(0)


def filled(shape, dtype):
    t = torch.full((int(np.prod(shape)) * np.dtype(dtype).itemsize,), FILL, dtype=torch.uint8, device="cuda")
    return t.view(getattr(torch, np.dtype(dtype).name)).view(*shape)


def run_qkv(c: Case, heads, T, TpQ, TpK, ws_bytes=0, extra=None):
    C = 64 * heads
    B = c.M // T
    keep = {}
    A = c.asrc(keep)
    w, cst = dev(c.w), dev(c.cst)
    out = {}
    for part, Tp in (("q", TpQ), ("k", TpK)):
        G = B * heads * Tp
        out[part] = (filled((G, 64), np.int8), filled((G, 64), np.int8), filled((G,), np.int32),
                     filled((G,), np.int64), filled((G,), np.int64), filled((G,), np.int64))
    V = filled((c.M, C), np.int32)
    q, k = out["q"], out["k"]
    E = vg.AEpi(epi=vg.EPI_QKV, heads=heads, T=T, TpQ=TpQ, TpK=TpK, C=C, Y2=vg.ptr(V),
                qhi=vg.ptr(q[0]), qlo=vg.ptr(q[1]), qe=vg.ptr(q[2]), qhs=vg.ptr(q[3]), qls=vg.ptr(q[4]), qts=vg.ptr(q[5]),
                khi=vg.ptr(k[0]), klo=vg.ptr(k[1]), ke=vg.ptr(k[2]), khs=vg.ptr(k[3]), kls=vg.ptr(k[4]), kts=vg.ptr(k[5]))
    for f, v in (extra or {}).items():
        setattr(E, f, v)
    ws = None
    if ws_bytes:
        ws = torch.empty(ws_bytes // 4 + 16, dtype=torch.int32, device="cuda")
        E.ws, E.ws_bytes = vg.ptr(ws), ws_bytes
    vg.k_gemm_hl2(A, c.Mp, c.M, w, c.Kp, c.Np, c.N, c.Kp, cst, E)
    torch.cuda.synchronize()
    return {p: tuple(to_np(x) for x in v) for p, v in out.items()} | {"v": to_np(V)}


def check_qkv(src, heads, T, B=2, K=320, seed=0, variant=-1, ws_bytes=0, extra=None, **kw):
    C = 64 * heads
    M = B * T
    TpQ, TpK = cf.align(T, 128), cf.align(T, 64)
    vg.set_variant(variant)
    c = Case(src, M, 3 * C, K, seed=seed, **kw)
    got = run_qkv(c, heads, T, TpQ, TpK, ws_bytes, extra)
    Y, _ = c.reference()
    want = oracle.qkv_heads(Y, M, C, heads, T, TpQ, TpK, fill=FILL)
    what = f"qkv src {src} heads {heads} T {T} K {K}"
    assert_equal(got["v"], want["v"], f"{what} v")
    for part in ("q", "k"):
        for name, g, w in zip(("hi", "lo", "e", "hs", "ls", "ts"), got[part], want[part]):
            assert_equal(g, w, f"{what} {part}.{name}")


@pytest.mark.parametrize("heads,T", [(1, 64), (5, 77), (2, 130)])
@pytest.mark.parametrize("src", [vg.SRC_I16, vg.SRC_I8, vg.SRC_X32])
def test_qkv(src, heads, T):
    check_qkv(src, heads, T, seed=heads * 7 + T, s_range=(12, 24))


def test_qkv_row_shifts_and_wide_range():
    """Per-row shifts, and m/s giving y from 0 to saturation (e from 0 to 17 within one call)."""
    check_qkv(vg.SRC_I8, 3, 100, K=256, seed=5, e_max=9, s_range=(4, 30))
    check_qkv(vg.SRC_I16, 2, 64, K=512, seed=6, s_range=(-2, 40), m_range=(1, 1 << 20))


@pytest.mark.parametrize("variant", [1, 2, 3, 4])
def test_qkv_ignores_tile_override(variant):
    """QKV runs on the 128 x 128 tiles whatever variant is forced (src/gemm_hl.cu:358 forces 64 x 64)."""
    check_qkv(vg.SRC_I16, 2, 77, K=320, seed=20 + variant, variant=variant)


def test_qkv_ignores_unread_fields():
    """A residual, row maxima and GroupNorm records given to EPI_QKV are neither read nor written, as
    the reference's QKV epilogue returns before it reaches them (src/gemm_hl.cu:179-241)."""
    sentinel = torch.full((4096,), 0x3C3C3C3C, dtype=torch.int32, device="cuda")
    extra = dict(residual=vg.ptr(sentinel), rowmax=vg.ptr(sentinel[1024:]), gnstat=vg.ptr(sentinel[2048:]), gnT=64)
    check_qkv(vg.SRC_I8, 2, 64, seed=31, s_range=(12, 24), extra=extra)
    assert (to_np(sentinel) == 0x3C3C3C3C).all()


def test_qkv_with_workspace():
    """A split-K workspace is ignored: the partial pass does not carry the head layout."""
    check_qkv(vg.SRC_I8, 5, 96, K=1280, seed=30, ws_bytes=64 << 20)


def test_qkv_c5_geometry():
    """The UNet's first transformer block at 64 x 64: C = 320 (5 heads), T = 4096, two samples."""
    check_qkv(vg.SRC_I16, 5, 4096, K=320, seed=40, s_range=(14, 22))


# ---------------------------------------------------------------- GroupNorm statistics


def run_gn(c: Case, T, ws_bytes=0, twice=False):
    """The case with gnstat on (Y aliases the residual), records prepared by k_gn_init."""
    B = -(-c.M // T)
    gs = vg.gn_stats_alloc(B * 32)
    vg.k_gn_init(gs, B * 32)
    keep = {}
    A = c.asrc(keep)
    w, cst = dev(c.w), dev(c.cst)
    Y = dev(c.res) if c.res is not None else torch.zeros((c.M, c.N), dtype=torch.int32, device="cuda")
    rm = torch.zeros(c.M, dtype=torch.int32, device="cuda") if c.rowmax else None
    E = vg.AEpi(epi=vg.EPI_PLAIN, Y=vg.ptr(Y), ldy=c.N, residual=vg.ptr(Y) if c.res is not None else None, rowmax=vg.ptr(rm),
                gnstat=vg.ptr(gs), gnT=T)
    ws = None
    if ws_bytes:
        ws = torch.empty(ws_bytes // 4 + 16, dtype=torch.int32, device="cuda")
        E.ws, E.ws_bytes = vg.ptr(ws), ws_bytes
    vg.k_gemm_hl2(A, c.Mp, c.M, w, c.Kp, c.Np, c.N, c.Kp, cst, E)
    if twice:
        vg.k_gemm_hl2(A, c.Mp, c.M, w, c.Kp, c.Np, c.N, c.Kp, cst, E)
    torch.cuda.synchronize()
    return to_np(Y), (to_np(rm).view(np.uint32) if rm is not None else None), vg.gn_stats_read(gs, B * 32)


def check_gn(c: Case, T, what, ws_bytes=0):
    Yg, rmg, st = run_gn(c, T, ws_bytes)
    Y, rm = c.reference()
    assert_equal(Yg, Y, f"{what} Y")
    if rm is not None:
        assert_equal(rmg, rm, f"{what} rowmax")
    want = oracle.gn_stats_fused(Y, c.M, c.N, T, c.Mp, c.Np, c.Kp, c.src)
    for k in ("sum", "mn", "mx"):
        assert_equal(st[k], want[k], f"{what} gn.{k}")
    return Y, want


@pytest.mark.parametrize("T", [64, 192, 256])
@pytest.mark.parametrize("variant", [-1, 0, 1, 2, 3, 4])
def test_gn_i16(variant, T):
    """Every tile shape; variant 4 (the row-stationary kernel) falls back to the tiles with statistics."""
    vg.set_variant(variant)
    c = Case(vg.SRC_I16, 3 * T, 320, 320, seed=T + variant, residual=True, rowmax=True, s_range=(16, 24))
    check_gn(c, T, f"gn I16 v{variant} T{T}")


@pytest.mark.parametrize("src", [vg.SRC_I8, vg.SRC_X32])
def test_gn_i8_x32(src):
    c = Case(src, 2 * 192, 640, 256, seed=50 + src, residual=True, e_max=5 if src == vg.SRC_I8 else 0)
    check_gn(c, 192, f"gn src {src}")


@pytest.mark.parametrize("conv,variant", [
    ((2, 16, 16, 64, 1), -1),    # the halo 3x3 kernel (T = 256)
    ((2, 16, 16, 64, 1), 0),     # the DMA tile kernel on the same geometry
    ((2, 32, 32, 64, 1), -1),    # T = 1024
    ((3, 16, 16, 32, 2), -1),    # stride 2: T = 64
])
def test_gn_conv16(conv, variant):
    vg.set_variant(variant)
    B, H, W, C, stride = conv
    Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
    c = Case(vg.SRC_CONV16, B * Ho * Wo, 320, 9 * C, seed=60 + H + variant, conv=conv, residual=True, s_range=(16, 24))
    check_gn(c, Ho * Wo, f"gn conv16 {conv} v{variant}")


def test_gn_conv32():
    B, H, W, C = 2, 8, 8, 32
    c = Case(vg.SRC_CONV32, B * H * W, 128, 9 * C, seed=70, conv=(B, H, W, C, 1), residual=True)
    check_gn(c, H * W, "gn conv32")


def test_gn_ignores_workspace():
    """Statistics run without split-K (the partial pass does not carry them)."""
    c = Case(vg.SRC_I16, 128, 1280, 11520 // 4, seed=80, residual=True, s_range=(18, 26))
    check_gn(c, 64, "gn ws", ws_bytes=256 << 20)


@pytest.mark.parametrize("variant", [-1, 0, 1, 2, 3])
def test_gn_saturated_groups(variant):
    """Outputs that saturate to INT_MAX through whole groups of one of the reference's 64 x 64 tiles
    (y > 0 plus a residual of INT_MAX): that tile adds nothing for those groups, as the reference's
    flush test (min != INT_MAX, src/gemm_hl.cu:306-309) skips it; a tile with one value below INT_MAX
    in the group counts in full. Every forced tile shape gives the same records."""
    vg.set_variant(variant)
    c = Case(vg.SRC_I16, 256, 320, 320, seed=95, residual=True, s_range=(30, 30), m_range=(1, 2), b_range=(1000, 2000))
    c.res[:64, :40] = 2**31 - 1        # tile (0, 0), groups 0..3 saturated through
    c.res[64:128, 100:] = 2**31 - 1    # tiles (1, 1..4): groups 10..31 saturated through
    c.res[127, 200] = -5               # ... except one value of group 20 in tile (1, 3)
    Y, want = check_gn(c, 128, f"gn saturated v{variant}")
    exact = oracle.gn_stats(Y, c.M, c.N, 128)
    assert (want["sum"] != exact["sum"]).any() and (want["mx"] != exact["mx"]).any(), "the case must exercise the flush rule"


@pytest.mark.parametrize("variant", [-1, 0, 1, 2])
def test_gn_saturated_deep_tiles(variant):
    """Deep K (Kp >= 2048) with Np % 128 == 0: the reference's tile is 64 x 128, so the statistics
    regions are 64 x 128 whatever tile shape runs here."""
    vg.set_variant(variant)
    c = Case(vg.SRC_I16, 256, 256, 2048, seed=96, residual=True, s_range=(34, 34), m_range=(1, 2), b_range=(1000, 2000))
    assert oracle.gn_ref_tile(c.Mp, c.Np, c.Kp, c.src) == (64, 128)
    c.res[:64, :128] = 2**31 - 1       # one whole 64 x 128 tile
    c.res[64:128, :64] = 2**31 - 1     # half of the next: not a whole tile, counts
    Y, want = check_gn(c, 128, f"gn saturated deep v{variant}")
    exact = oracle.gn_stats(Y, c.M, c.N, 128)
    assert (want["sum"] != exact["sum"]).any()


def test_gn_accumulates_over_calls():
    """Two GEMMs into the same records (the atomics add up): sum doubles, min/max unchanged."""
    c = Case(vg.SRC_I16, 256, 320, 320, seed=90, s_range=(16, 24))
    _, _, once = run_gn(c, 128)
    _, _, two = run_gn(c, 128, twice=True)
    assert_equal(two["sum"], 2 * once["sum"], "sum")
    assert_equal(two["mn"], once["mn"], "mn")
    assert_equal(two["mx"], once["mx"], "mx")


@pytest.mark.parametrize("M,N,T", [(192, 128, 64), (512, 320, 256), (300, 1280, 100)])
def test_planar_epilogue_gn(M, N, T):
    """k_epilogue with gs (src/kernels.cu:70-95) from random planes, with a residual."""
    r = np.random.default_rng(M + N)
    ldc = N + 4
    Chi = r.integers(-(1 << 20), 1 << 20, (M, ldc)).astype(np.int32)
    Clo = r.integers(-(1 << 20), 1 << 20, (M, ldc)).astype(np.int32)
    cst = np.stack([r.integers(1 << 10, 1 << 15, N), r.integers(16, 30, N), r.integers(-50000, 50000, N),
                    r.integers(-20000, 20000, N)], 1).astype(np.int32)
    e = r.integers(0, 6, M).astype(np.int32)
    R = r.integers(-(2**31), 2**31, (M, N), dtype=np.int64).astype(np.int32)
    want = oracle.epilogue(Chi, Clo, M, N, ldc, cst, e, N, R)
    Mb = -(-M // T)
    gs = vg.gn_stats_alloc(Mb * 32)
    vg.k_gn_init(gs, Mb * 32)
    Y = dev(R)
    vg.k_epilogue(dev(Chi), dev(Clo), M, N, ldc, dev(cst), dev(e), Y, N, residual=Y, gs=gs, T=T)
    torch.cuda.synchronize()
    assert_equal(to_np(Y), want, "planar Y")
    st = vg.gn_stats_read(gs, Mb * 32)
    ref = oracle.gn_stats_planar(want, M, N, T)
    for k in ("sum", "mn", "mx"):
        assert_equal(st[k], ref[k], f"planar gn.{k}")


@pytest.mark.parametrize("M,N,T", [(256, 320, 64), (64, 1024, 16)])
def test_planar_epilogue_gn_saturated(M, N, T):
    """k_epilogue statistics by the reference's rule (src/kernels.cu:67-68): a 1024-element block whose
    outputs of a group all saturate to INT_MAX (residual INT_MAX, y >= 0) adds nothing for it."""
    r = np.random.default_rng(M * 3 + N)
    ldc = N
    Chi = r.integers(0, 1 << 12, (M, ldc)).astype(np.int32)
    Clo = r.integers(0, 1 << 12, (M, ldc)).astype(np.int32)
    cst = np.stack([r.integers(1, 4, N), np.full(N, 20), r.integers(0, 1000, N), r.integers(0, 100, N)], 1).astype(np.int32)
    e = np.zeros(M, np.int32)
    R = r.integers(-(1 << 20), 1 << 20, (M, N)).astype(np.int32)
    flat = R.reshape(-1)
    flat[1024:2048] = 2**31 - 1            # the whole second block
    flat[3 * 1024:3 * 1024 + 300] = 2**31 - 1
    want = oracle.epilogue(Chi, Clo, M, N, ldc, cst, e, N, R)
    Mb = -(-M // T)
    gs = vg.gn_stats_alloc(Mb * 32)
    vg.k_gn_init(gs, Mb * 32)
    Y = dev(R)
    vg.k_epilogue(dev(Chi), dev(Clo), M, N, ldc, dev(cst), dev(e), Y, N, residual=Y, gs=gs, T=T)
    torch.cuda.synchronize()
    assert_equal(to_np(Y), want, "planar Y")
    st = vg.gn_stats_read(gs, Mb * 32)
    ref = oracle.gn_stats_planar(want, M, N, T)
    assert (ref["sum"] != oracle.gn_stats(want, M, N, T)["sum"]).any(), "the case must exercise the flush rule"
    for k in ("sum", "mn", "mx"):
        assert_equal(st[k], ref[k], f"planar saturated gn.{k}")

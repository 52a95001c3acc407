"""GPU parity of the hi/lo GEMM (vgemm_hl2 / vgemm_hl through the C ABI) against the CPU oracle.

Mirrors the reference's own GEMM tests: src/test_gemm_hl.cu:53-86 (random int8 planes, e in [0,12),
m in [2^14, 2^15), s in [20, 30), b in [-50000, 50000), a random residual, every tile variant) and
:10-52 (int32 sources of random bit width 1..31, so saturation and e up to 17 occur, against the
planar path). Here every result is compared byte for byte with oracle/ instead of with cuBLASLt.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_equal, to_np
from vela_amd import configs as cf
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu


def rng(seed):
    return np.random.default_rng(seed)


def make_w_cst(r, N, K, Np, Kp, s_range=(20, 29), m_range=(1 << 14, 1 << 15), wlo=-128, b_range=(-50000, 50000)):
    w = np.zeros((Np, Kp), np.int8)
    w[:N, :K] = r.integers(wlo, 128, (N, K))
    cst = np.zeros((Np, 4), np.int32)
    cst[:, 0] = 1
    cst[:N, 0] = r.integers(m_range[0], m_range[1], N, dtype=np.int64)
    cst[:N, 1] = r.integers(s_range[0], s_range[1] + 1, N)
    cst[:N, 2] = r.integers(b_range[0], b_range[1], N, dtype=np.int64)
    cst[:N, 3] = w[:N].astype(np.int64).sum(1)
    return w, cst


def rand_bits(r, shape):
    bits = r.integers(1, 32, shape)
    v = r.integers(0, 1 << 31, shape, dtype=np.int64) & ((np.int64(1) << bits) - 1)
    return (v - (np.int64(1) << (bits - 1))).astype(np.int32)


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


class Case:
    """Host inputs + oracle + device run of one vgemm_hl2 call."""

    def __init__(self, src, M, N, K, epi=vg.EPI_PLAIN, seed=0, residual=False, rowmax=False, e_max=0, s_range=(20, 29),
                 m_range=(1 << 14, 1 << 15), conv=None, lut=None, Cs=0, b_range=(-50000, 50000)):
        r = rng(seed)
        self.src, self.M, self.N, self.K, self.epi = src, M, N, K, epi
        self.Kp = cf.align(K, 16)
        self.Np = cf.align(N, 64)
        self.Mp = cf.align(M, 64)
        self.conv = conv
        self.w, self.cst = make_w_cst(r, N, K, self.Np, self.Kp, s_range, m_range, b_range=b_range)
        self.e = r.integers(0, e_max + 1, M).astype(np.int32) if e_max else None
        self.kw = {}
        if src == vg.SRC_I8:
            self.hi = r.integers(-128, 128, (self.Mp, self.Kp)).astype(np.int8)
            self.lo = r.integers(-128, 128, (self.Mp, self.Kp)).astype(np.int8)
            self.kw = dict(hi=self.hi, lo=self.lo)
        elif src == vg.SRC_I16:
            self.q = r.integers(-32768, 32768, (M, K)).astype(np.int16)
            self.kw = dict(q16=self.q, K=K)
        elif src == vg.SRC_X32:
            self.x = rand_bits(r, (M, K))
            self.xrm = np.abs(self.x.astype(np.int64)).max(1).astype(np.uint32)
            self.kw = dict(x=self.x, xrowmax=self.xrm, K=K)
        else:
            B, H, W, C, stride = conv
            if src == vg.SRC_CONV32:
                self.img = rand_bits(r, (B, H, W, C))
            else:
                self.img = r.integers(-32768, 32768, (B, H, W, C)).astype(np.int16)
            pm = oracle.pixmax(self.img.astype(np.int32).reshape(-1, C), B * H * W, C)
            self.pm = pm
            self.e = oracle.conv_e(pm, B, H, W, stride)
            self.kw = dict(img=self.img, H=H, W=W, C=C, stride=stride)
        self.lut = lut if lut is not None else cf.phi_lut()
        self.Cs = Cs
        nout = N // 2 if epi == vg.EPI_GEGLU else N
        self.nout = nout
        self.res = r.integers(-(2**31), 2**31, (M, nout), dtype=np.int64).astype(np.int32) if residual else None
        self.rowmax = rowmax
        self.pm_in_kernel = False   # convolution sources: pass the per-pixel maxima instead of e

    def reference(self):
        kw = dict(self.kw)
        if self.epi == vg.EPI_SPLIT3:
            Y0, Y1, Y2 = (np.zeros((self.M, self.Cs), np.int32) for _ in range(3))
            oracle.gemm(self.src, Mreal=self.M, Nreal=self.N, Kp=self.Kp, w=self.w, cst=self.cst, epi=self.epi, e=self.e,
                        Lphi=self.lut, Y=Y0, ldy=self.Cs, Cs=self.Cs, Y1=Y1, Y2=Y2, **kw)
            return (Y0, Y1, Y2), None
        Y = np.zeros((self.M, self.nout), np.int32) if self.res is None else self.res.copy()
        rm = np.zeros(self.M, np.uint32) if self.rowmax else None
        oracle.gemm(self.src, Mreal=self.M, Nreal=self.N, Kp=self.Kp, w=self.w, cst=self.cst, epi=self.epi, e=self.e,
                    Lphi=self.lut, Y=Y, residual=Y if self.res is not None else None, rowmax=rm, **kw)
        return Y, rm

    def asrc(self, keep):
        """The device A operand of this case; device buffers are kept alive in `keep`."""
        A = vg.ASrc(src=self.src)
        if self.pm_in_kernel:
            keep["pm"] = dev(self.pm.view(np.int32))
            A.rowmax = vg.ptr(keep["pm"])
        else:
            keep["e"] = dev(self.e)
            A.e = vg.ptr(keep["e"])
        if self.src == vg.SRC_I8:
            keep["hi"], keep["lo"] = dev(self.hi), dev(self.lo)
            A.hi, A.lo, A.ld8 = vg.ptr(keep["hi"]), vg.ptr(keep["lo"]), self.Kp
        elif self.src == vg.SRC_I16:
            keep["q"] = dev(self.q)
            A.q16, A.ld16, A.K = vg.ptr(keep["q"]), self.K, self.K
        elif self.src == vg.SRC_X32:
            keep["x"], keep["rm"] = dev(self.x), dev(self.xrm.view(np.int32))
            A.x, A.ldx, A.rowmax, A.K = vg.ptr(keep["x"]), self.K, vg.ptr(keep["rm"]), self.K
        else:
            B, H, W, C, stride = self.conv
            keep["img"] = dev(self.img)
            if self.src == vg.SRC_CONV32:
                A.img = vg.ptr(keep["img"])
            else:
                A.img16 = vg.ptr(keep["img"])
            A.H, A.W, A.C, A.stride = H, W, C, stride
            A.Ho, A.Wo, A.K = (H - 1) // stride + 1, (W - 1) // stride + 1, 9 * C
        return A

    def run_gpu(self, ws_bytes=0, extra=None):
        keep = {}
        A = self.asrc(keep)
        w, cst = dev(self.w), dev(self.cst)
        lut = dev(self.lut)
        E = vg.AEpi(epi=self.epi, Lphi=vg.ptr(lut))
        if self.epi == vg.EPI_SPLIT3:
            Ys = [torch.zeros((self.M, self.Cs), dtype=torch.int32, device="cuda") for _ in range(3)]
            E.Y, E.Y1, E.Y2, E.Cs, E.ldy = vg.ptr(Ys[0]), vg.ptr(Ys[1]), vg.ptr(Ys[2]), self.Cs, self.Cs
        else:
            Y = dev(self.res) if self.res is not None else torch.zeros((self.M, self.nout), dtype=torch.int32, device="cuda")
            E.Y, E.ldy = vg.ptr(Y), self.nout
            if self.res is not None:
                E.residual = vg.ptr(Y)    # aliases Y, as src/engine.cu:431 does
        rm = torch.zeros(self.M, dtype=torch.int32, device="cuda") if self.rowmax else None
        E.rowmax = vg.ptr(rm)
        ws = None
        if ws_bytes:
            ws = torch.empty(ws_bytes // 4 + 16, dtype=torch.int32, device="cuda")
            E.ws, E.ws_bytes = vg.ptr(ws), ws_bytes
        for f, v in (extra or {}).items():
            setattr(E, f, v)
        vg.k_gemm_hl2(A, self.Mp, self.M, w, self.Kp, self.Np, self.N, self.Kp, cst, E)
        torch.cuda.synchronize()
        if self.epi == vg.EPI_SPLIT3:
            return tuple(to_np(y) for y in Ys), None
        return to_np(Y), (to_np(rm).view(np.uint32) if rm is not None else None)

    def check(self, ws_bytes=0, what="", extra=None):
        got, grm = self.run_gpu(ws_bytes, extra)
        want, wrm = self.reference()
        if self.epi == vg.EPI_SPLIT3:
            for i in range(3):
                assert_equal(got[i], want[i], f"{what} Y{i}")
        else:
            assert_equal(got, want, f"{what} Y")
        if wrm is not None:
            assert_equal(grm, wrm, f"{what} rowmax")


@pytest.fixture(autouse=True)
def _reset_knobs(gpu):
    vg.set_variant(-1)
    vg.set_splitk(0)
    yield
    vg.set_variant(-1)
    vg.set_splitk(0)


SHAPES = [(64, 64, 64), (100, 80, 48), (300, 200, 320), (257, 130, 96), (640, 320, 1280)]


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
@pytest.mark.parametrize("shape", SHAPES)
def test_i8_planes_plain_residual(variant, shape):
    """src/test_gemm_hl.cu:55-80 scaled down: random planes, e in [0,12), s in [20,30), residual."""
    vg.set_variant(variant)
    M, N, K = shape
    Case(vg.SRC_I8, M, N, K, seed=hash(shape) % 1000 + variant, residual=True, e_max=11).check(what=f"I8 {shape} v{variant}")


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
@pytest.mark.parametrize("shape", SHAPES)
def test_i16_plain(variant, shape):
    vg.set_variant(variant)
    M, N, K = shape
    K = cf.align(K, 8)
    Case(vg.SRC_I16, M, N, K, seed=7 + variant, s_range=(16, 24)).check(what=f"I16 {shape} v{variant}")


# Shallow calls that the automatic dispatch sends to the row-stationary kernels by their tile count
# (at least 960 tiles of 64x128, from 1024 rows): few rows over many columns, partial row stripes and
# W chunks, K below 320, each epilogue, a residual; and deeper calls of few rows that it sends to the
# K-split-over-waves kernel by its grid (at most 1024 rows and 1280 columns, Kp >= 768, at most one
# 64x64 block per CU).
AUTO_MID = [(vg.SRC_I16, 8192, 960, 160, vg.EPI_PLAIN, False), (vg.SRC_I8, 1030, 9600, 320, vg.EPI_PLAIN, False),
            (vg.SRC_I16, 4100, 2560, 320, vg.EPI_GEGLU, False), (vg.SRC_I16, 6150, 1288, 200, vg.EPI_GELU, False),
            (vg.SRC_I16, 8200, 1280, 320, vg.EPI_PLAIN, True), (vg.SRC_I16, 700, 1270, 1280, vg.EPI_PLAIN, True),
            (vg.SRC_I8, 616, 1280, 768, vg.EPI_PLAIN, False), (vg.SRC_I16, 1000, 640, 1000, vg.EPI_GELU, False)]


@pytest.mark.parametrize("case", AUTO_MID, ids=lambda c: f"{c[1]}x{c[2]}x{c[3]}-epi{c[4]}{'-res' if c[5] else ''}")
def test_auto_shallow_tile_count(case):
    src, M, N, K, epi, res = case
    Case(src, M, N, K, epi=epi, seed=M % 101 + epi, residual=res, rowmax=M % 2 == 0, s_range=(16, 24)).check(
        what=f"auto {M}x{N}x{K} epi {epi} res {res}")


@pytest.mark.parametrize("epi", [vg.EPI_PLAIN, vg.EPI_GEGLU, vg.EPI_GELU])
@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_i16_epilogues_rowmax(epi, variant):
    vg.set_variant(variant)
    Case(vg.SRC_I16, 384, 256, 320, epi=epi, seed=11, rowmax=True, e_max=3, s_range=(16, 24)).check(what=f"epi {epi} v{variant}")


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_split3(variant):
    vg.set_variant(variant)
    Case(vg.SRC_I16, 200, 3 * 96, 128, epi=vg.EPI_SPLIT3, seed=12, Cs=96).check(what=f"split3 v{variant}")


@pytest.mark.parametrize("variant", [0, 1, 3])
@pytest.mark.parametrize("shape", [(96, 64, 1024), (130, 320, 960), (64, 128, 64)])
def test_x32_source(variant, shape):
    """SRC_X32: int32 rows of random bit width 1..31 quantised on load (src/test_gemm_hl.cu:16,31-36)."""
    vg.set_variant(variant)
    M, N, K = shape
    Case(vg.SRC_X32, M, N, K, seed=13).check(what=f"X32 {shape}")


@pytest.mark.parametrize("variant", [-1, 3])
@pytest.mark.parametrize("src", [vg.SRC_CONV32, vg.SRC_CONV16])
@pytest.mark.parametrize("geom", [(2, 8, 8, 32, 1), (1, 7, 5, 64, 2), (2, 6, 6, 320, 1), (1, 9, 11, 16, 2)])
def test_conv_sources(src, geom, variant):
    """Implicit 3x3 im2col (src/test_gemm_hl.cu:12,25-29 cases scaled down), e from conv_e(pixmax)."""
    vg.set_variant(variant)
    B, H, W, C, stride = geom
    Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
    Case(src, B * Ho * Wo, 96, 9 * C, seed=14, conv=geom, residual=True).check(what=f"conv {src} {geom}")


@pytest.mark.parametrize("src", [vg.SRC_CONV32, vg.SRC_CONV16])
@pytest.mark.parametrize("geom,variant,split", [((2, 8, 8, 32, 1), -1, 0), ((1, 7, 5, 64, 2), 3, 0), ((2, 6, 6, 320, 1), 0, 0),
                                                ((1, 9, 11, 16, 2), 1, 0), ((8, 8, 8, 256, 1), -1, 0), ((2, 8, 8, 512, 1), 1, 3),
                                                ((2, 16, 16, 64, 1), -1, 0)])
def test_conv_shift_from_pixel_maxima(src, geom, variant, split):
    """A convolution given the image's per-pixel maxima (ASrc.rowmax, e = NULL) derives each row's
    shift in the kernel by k_conv_e's rule: the same bytes as with e from k_conv_e, on the tile,
    halo and split-K paths (the split-K reduction derives it too)."""
    vg.set_variant(variant)
    vg.set_splitk(split)
    B, H, W, C, stride = geom
    Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
    c = Case(src, B * Ho * Wo, 128, 9 * C, seed=15 + C, conv=geom, residual=True)
    if src == vg.SRC_CONV16:
        c.img.reshape(-1)[::97] = -32768   # |x| = 32768 gives e = 1 where it enters a window
        c.pm = oracle.pixmax(c.img.astype(np.int32).reshape(-1, C), B * H * W, C)
        c.e = oracle.conv_e(c.pm, B, H, W, stride)
    assert c.e.max() > 0
    c.pm_in_kernel = True
    c.check(ws_bytes=(64 << 20) if split else 0, what=f"conv {src} {geom} pm")


@pytest.mark.parametrize("variant", [-1, 0, 3])
def test_conv16_with_shifts(variant):
    """SRC_CONV16 with caller-provided shifts e in [0, 17] (the image is quantised on load with
    quant16_32 per output row, src/gemm_hl.cu:104-114), and an image holding -32768."""
    vg.set_variant(variant)
    B, H, W, C, stride = 2, 6, 5, 64, 1
    c = Case(vg.SRC_CONV16, B * H * W, 128, 9 * C, seed=31, conv=(B, H, W, C, stride), residual=True)
    c.img[0, :2] = -32768
    c.e = rng(32).integers(0, 18, c.M).astype(np.int32)
    c.e[::7] = 0
    c.check(what=f"conv16 e v{variant}")


@pytest.mark.parametrize("variant", [-1, 1, 0])
@pytest.mark.parametrize("geom", [(2, 6, 5, 64, 1), (1, 9, 7, 128, 2), (2, 8, 8, 192, 1)])
def test_conv32_dma_tiles(geom, variant):
    """SRC_CONV32 with C % 64 == 0 on the DMA tile kernel (raw int32 rows staged in LDS, quantised
    per fragment; variants -1 and 1) and on the register-staged kernel (variant 0): images whose
    values fit 16 bits (every row e = 0, so whole waves take the clamp-only form; +-32768 and
    +-32767 present), then caller shifts e in [0, 17] on full-width int32 values."""
    vg.set_variant(variant)
    B, H, W, C, stride = geom
    Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
    c = Case(vg.SRC_CONV32, B * Ho * Wo, 192, 9 * C, seed=41 + C, conv=geom, residual=True)
    small = rng(42).integers(-32768, 32768, c.img.shape).astype(np.int32)
    small.reshape(-1)[::53] = -32768
    small.reshape(-1)[::59] = 32767
    c.img = small
    c.kw["img"] = small
    c.e = np.zeros(c.M, np.int32)
    c.check(what=f"conv32 e=0 {geom} v{variant}")
    c2 = Case(vg.SRC_CONV32, B * Ho * Wo, 192, 9 * C, seed=43 + C, conv=geom, residual=True)
    c2.e = rng(44).integers(0, 18, c2.M).astype(np.int32)
    c2.e[::5] = 0
    c2.check(what=f"conv32 e {geom} v{variant}")
    # shifts in [0, 16] only (whole waves take the three-instruction form), with values at and just
    # below INT_MAX, where v + 2^(e-1) saturates, and INT_MIN + 1
    c3 = Case(vg.SRC_CONV32, B * Ho * Wo, 192, 9 * C, seed=45 + C, conv=geom, residual=True)
    big = rng(46).integers(-(2**31) + 1, 2**31, c3.img.shape, dtype=np.int64).astype(np.int32)
    flat = big.reshape(-1)
    flat[::7] = 2**31 - 1
    flat[3::11] = 2**31 - 2**15
    flat[5::13] = 2**31 - 3
    flat[6::17] = -(2**31) + 1
    c3.img = big
    c3.kw["img"] = big
    c3.e = rng(47).integers(0, 17, c3.M).astype(np.int32)
    c3.e[::6] = 16
    c3.check(what=f"conv32 e <= 16, extremes {geom} v{variant}")


# (B, H, W, C) of stride-1 SRC_CONV16 problems that run the halo kernel (128-row tiles of whole
# output rows)
HALO_GEOMS = [
    (3, 16, 16, 64),    # eight output rows per tile, two tiles per image
    (2, 16, 8, 128),    # sixteen rows of 8 pixels: one tile per image
    (1, 32, 16, 192),   # three channel chunks
    (1, 32, 4, 64),     # 32 rows of 4 pixels
]


@pytest.mark.parametrize("epi", [vg.EPI_PLAIN, vg.EPI_SPLIT3])
@pytest.mark.parametrize("geom", HALO_GEOMS)
def test_conv16_halo(geom, epi):
    """The halo-reuse 3x3 kernel (one input patch per 64-channel chunk shared by the nine taps) gives
    the oracle's bytes: whole-row and whole-image tiles, partial last tiles, partial column tiles,
    residual and row max (src/gemm_hl.cu:104-114 addressing, :40-52 epilogue)."""
    B, H, W, C = geom
    assert vg.conv16_halo_rows(H, W, C, 1, epi) == 128
    if epi == vg.EPI_SPLIT3:
        c = Case(vg.SRC_CONV16, B * H * W, 192, 9 * C, epi=epi, seed=50, conv=(B, H, W, C, 1), Cs=64)
    else:
        c = Case(vg.SRC_CONV16, B * H * W, 200, 9 * C, seed=51, conv=(B, H, W, C, 1), residual=True, rowmax=True)
    c.img[0, 0, :3] = -32768
    c.check(what=f"halo {geom} epi {epi}")


@pytest.mark.parametrize("geom", HALO_GEOMS[:3])
def test_conv16_halo_shifts(geom):
    """Caller shifts e in [0, 17] per output row: the patch is shared by rows with different e, so the
    quantisation happens per fragment row as the nine taps read it."""
    B, H, W, C = geom
    assert vg.conv16_halo_rows(H, W, C, 1, vg.EPI_PLAIN) == 128
    c = Case(vg.SRC_CONV16, B * H * W, 128, 9 * C, seed=52, conv=(B, H, W, C, 1), residual=True)
    c.img[0, 1, :5] = -32768
    c.e = rng(53).integers(0, 18, c.M).astype(np.int32)
    c.e[::5] = 0
    c.check(what=f"halo e {geom}")


@pytest.mark.parametrize("splits", [2, 3])
def test_conv16_halo_splitk(splits):
    """Split-K over channel chunks (2 + 1 and 1 + 1 + 1 of three chunks) through the workspace."""
    vg.set_splitk(splits)
    B, H, W, C = HALO_GEOMS[2]
    assert vg.conv16_halo_rows(H, W, C, 1, vg.EPI_PLAIN) == 128
    c = Case(vg.SRC_CONV16, B * H * W, 128, 9 * C, seed=54, conv=(B, H, W, C, 1), residual=True, rowmax=True)
    nb = vg.workspace_bytes(c.Mp, c.M, c.Np, c.N, c.Kp, 0)
    assert nb > 0
    c.check(ws_bytes=nb, what=f"halo splitk {splits}")


@pytest.mark.parametrize("src", [vg.SRC_I8, vg.SRC_I16])
def test_exact_slow_path(src):
    """Shifts s - e outside [1, 52] (left shifts, s = 0, deep right shifts) and |acc * m| beyond 2^52
    force the int64 epilogue; m up to 2^31 - 1 makes acc * m wrap exactly as the reference's int64."""
    K = 512
    for seed, s_range, m_range in [(1, (-6, 3), (1, 1 << 10)), (2, (50, 70), (1 << 14, 1 << 15)), (3, (20, 40), ((1 << 30), (1 << 31) - 1))]:
        Case(src, 200, 128, K, seed=seed, s_range=s_range, m_range=m_range, e_max=5, residual=True).check(what=f"slow {seed}")


@pytest.mark.parametrize("epi", [vg.EPI_PLAIN, vg.EPI_GEGLU, vg.EPI_GELU])
def test_fast_epilogue_branches(epi):
    """The three FP64 epilogue branches with e == 0: b folded into the FMA constant (no element can
    reach 2^31), b near +-2^31 (saturating add, not foldable), and a GEGLU product a*ge far beyond
    2^31 with y itself in range (folded, saturating only at the last step)."""
    cases = [
        ("fold", dict(s_range=(16, 20), m_range=(1 << 10, 1 << 12))),
        ("b near 2^31", dict(s_range=(16, 20), m_range=(1 << 10, 1 << 12), b_range=(-(2**31), 2**31))),
        ("large y", dict(s_range=(16, 16), m_range=(1 << 16, 1 << 18))),
    ]
    for i, (name, kw) in enumerate(cases):
        Case(vg.SRC_I16, 192, 128, 64, epi=epi, seed=40 + i, rowmax=True, residual=epi == vg.EPI_PLAIN, **kw).check(what=f"{name} epi {epi}")


def test_lut_outside_range_takes_exact_path():
    """A GELU table with entries outside [0, 65536] (the FP64 path's precondition) uses the exact path."""
    lut = rng(5).integers(-70000, 140000, 2049).astype(np.int32)
    for epi in (vg.EPI_GEGLU, vg.EPI_GELU):
        Case(vg.SRC_I16, 256, 128, 64, epi=epi, seed=15, lut=lut, rowmax=True).check(what=f"lut epi {epi}")


@pytest.mark.parametrize("variant", [-1, 3])
@pytest.mark.parametrize("splits", [2, 3, 7])
@pytest.mark.parametrize("epi", [vg.EPI_PLAIN, vg.EPI_GEGLU])
def test_splitk(splits, epi, variant):
    """Split-K partials through a workspace reduce to the same bytes."""
    vg.set_variant(variant)
    vg.set_splitk(splits)
    c = Case(vg.SRC_I16, 200, 192, 1536, epi=epi, seed=16, rowmax=True, residual=epi == vg.EPI_PLAIN)
    nb = vg.workspace_bytes(c.Mp, c.M, c.Np, c.N, c.Kp, epi)
    assert nb > 0
    c.check(ws_bytes=nb, what=f"splitk {splits}")


def test_conv_splitk():
    vg.set_splitk(4)
    c = Case(vg.SRC_CONV16, 2 * 8 * 8, 128, 9 * 256, seed=17, conv=(2, 8, 8, 256, 1), residual=True)
    c.check(ws_bytes=vg.workspace_bytes(c.Mp, c.M, c.Np, c.N, c.Kp, 0), what="conv splitk")


@pytest.mark.parametrize("epi,fields", [
    (vg.EPI_GEGLU, ("residual", "gnstat")),
    (vg.EPI_GELU, ("gnstat",)),
    (vg.EPI_SPLIT3, ("residual", "rowmax", "gnstat")),
])
@pytest.mark.parametrize("variant", [-1, 0, 4])
def test_unread_fields_are_ignored(epi, fields, variant):
    """AEpi fields an epilogue does not read are accepted and ignored, as the reference's epilogue
    ignores them (src/gemm_hl.cu:176-177, 279-296): the GroupNorm records outside EPI_PLAIN, the
    residual on GEGLU / SPLIT3, the row maxima on SPLIT3. Results equal the call without them and
    the buffers those fields point at are left untouched."""
    vg.set_variant(variant)
    sentinel = torch.full((3 * 4096,), 0x3C3C3C3C, dtype=torch.int32, device="cuda")
    extra = {f: vg.ptr(sentinel[i * 4096:]) for i, f in enumerate(fields)}
    if "gnstat" in fields:
        extra["gnT"] = 64
    c = Case(vg.SRC_I16, 128, 192, 320, epi=epi, seed=41 + epi, s_range=(16, 24), rowmax=epi != vg.EPI_SPLIT3,
             Cs=64 if epi == vg.EPI_SPLIT3 else 0)
    c.check(what=f"epi {epi} with {fields} v{variant}", extra=extra)
    assert (to_np(sentinel) == 0x3C3C3C3C).all(), f"epi {epi}: a buffer of an unread field was written"


@pytest.mark.parametrize("variant", [-1, 0, 1])
def test_x32_rowmax_understated(variant):
    """SRC_X32 with row maxima below the rows' true maxima (a caller's stale maxima): the shift comes
    from the given maximum and values beyond it saturate in quant16_32 exactly as the reference's
    formula has them, INT_MAX and INT_MIN with e = 1 included."""
    vg.set_variant(variant)
    c = Case(vg.SRC_X32, 192, 128, 256, seed=71)
    r = rng(72)
    c.x[:, :8] = np.array([2**31 - 1, -(2**31), 2**31 - 2, -(2**31) + 1, 65535, -65536, 32767, -32768], np.int32)
    c.xrm = r.integers(0, 1 << 18, c.M).astype(np.uint32)      # e from 0 to 4, far below the true maxima
    c.xrm[:16] = 40000                                          # e = 1
    c.xrm[16:32] = 0                                            # e = 0
    c.kw = dict(x=c.x, xrowmax=c.xrm, K=c.K)
    c.check(what=f"X32 understated rowmax v{variant}")


def test_stream_workspace_split():
    """A call without AEpi.ws whose shape wants a K split (deep K, few tiles) splits K in its stream's
    workspace: the same bytes as with a caller's workspace, with the stream workspaces off, captured
    into a graph on a fresh stream before any eager call (no workspace yet: unsplit inside the graph)
    and after one (the workspace exists: split inside the graph), every replay checked; replays
    after a larger call on the same stream replaced the workspace still use the one they captured."""
    c = Case(vg.SRC_I16, 256, 256, 8192, seed=61, residual=True, s_range=(22, 30))
    want, _ = c.reference()
    assert vg.workspace_bytes(c.Mp, c.M, c.Np, c.N, c.Kp, c.epi) > 0, "the shape must want a split"
    big = Case(vg.SRC_I16, 512, 1024, 8192, seed=62, s_range=(22, 30))
    big_need = vg.workspace_bytes(big.Mp, big.M, big.Np, big.N, big.Kp, big.epi)
    grain = 4 << 20
    assert big_need > -(-vg.workspace_bytes(c.Mp, c.M, c.Np, c.N, c.Kp, c.epi) // grain) * grain, \
        "the larger call must need a larger workspace"
    got, _ = c.run_gpu()                       # no ws: the current stream's workspace
    assert_equal(got, want, "stream workspace")
    vg.set_stream_workspaces(False)
    try:
        got, _ = c.run_gpu()
        assert_equal(got, want, "stream workspaces off")
    finally:
        vg.set_stream_workspaces(True)
    keep = {}
    A = c.asrc(keep)
    w, cst, lut = dev(c.w), dev(c.cst), dev(c.lut)
    for eager_first in (False, True):
        s = torch.cuda.Stream()
        Y = dev(c.res)
        E = vg.AEpi(epi=c.epi, Lphi=vg.ptr(lut), Y=vg.ptr(Y), ldy=c.nout, residual=vg.ptr(Y))
        if eager_first:
            Y.copy_(dev(c.res))
            vg.k_gemm_hl2(A, c.Mp, c.M, w, c.Kp, c.Np, c.N, c.Kp, cst, E, stream=s)
            s.synchronize()
            assert_equal(to_np(Y), want, "eager on the fresh stream")
        g = vg.Graph(s)
        torch.cuda.synchronize()
        g.begin()
        vg.k_gemm_hl2(A, c.Mp, c.M, w, c.Kp, c.Np, c.N, c.Kp, cst, E, stream=s)
        g.end()
        for rep in range(3):
            Y.copy_(dev(c.res))   # the residual aliases Y: re-seed before each replay
            torch.cuda.synchronize()
            g.replay()
            s.synchronize()
            assert_equal(to_np(Y), want, f"graph replay {rep} (eager first: {eager_first})")
        if eager_first:
            # a larger call on the same stream: a new workspace for it, the graph keeps the old one
            bkeep = {}
            bA = big.asrc(bkeep)
            bw, bcst, blut = dev(big.w), dev(big.cst), dev(big.lut)
            bY = torch.zeros((big.M, big.nout), dtype=torch.int32, device="cuda")
            bE = vg.AEpi(epi=big.epi, Lphi=vg.ptr(blut), Y=vg.ptr(bY), ldy=big.nout)
            vg.k_gemm_hl2(bA, big.Mp, big.M, bw, big.Kp, big.Np, big.N, big.Kp, bcst, bE, stream=s)
            Y.copy_(dev(c.res))
            torch.cuda.synchronize()
            g.replay()
            s.synchronize()
            bwant, _ = big.reference()
            assert_equal(to_np(bY), bwant, "the larger call")
            assert_equal(to_np(Y), want, "graph replay after the workspace was replaced")
        g.destroy()


def test_k_gemm_hl_wrapper():
    """meow::k_gemm_hl: the SRC_I8 convenience entry point with default arguments."""
    c = Case(vg.SRC_I8, 130, 64, 96, seed=18, e_max=4)
    want, _ = c.reference()
    hi, lo, w, cst, e = dev(c.hi), dev(c.lo), dev(c.w), dev(c.cst), dev(c.e)
    Y = torch.zeros((c.M, c.N), dtype=torch.int32, device="cuda")
    vg.k_gemm_hl(hi, lo, c.Kp, c.Mp, c.M, w, c.Kp, c.Np, c.N, c.Kp, cst, e, Y, c.N)
    torch.cuda.synchronize()
    assert_equal(to_np(Y), want, "k_gemm_hl")


def test_shape_errors():
    """Unsupported shapes raise like src/gemm_hl.cu:351,357 (gemm_hl: unsupported shape / conv source)."""
    c = Case(vg.SRC_I8, 64, 64, 64, seed=19)
    w, cst = dev(c.w), dev(c.cst)
    Y = torch.zeros((64, 64), dtype=torch.int32, device="cuda")
    A = vg.ASrc(src=vg.SRC_I8, hi=vg.ptr(dev(c.hi)), lo=vg.ptr(dev(c.lo)), ld8=c.Kp)
    E = vg.AEpi(Y=vg.ptr(Y), ldy=64)
    with pytest.raises(vg.VgemmError, match="unsupported shape"):
        vg.k_gemm_hl2(A, 63, 63, w, c.Kp, 64, 64, c.Kp, cst, E)
    A2 = vg.ASrc(src=vg.SRC_CONV32, img=vg.ptr(Y), H=4, W=4, C=8, K=72, Ho=4, Wo=4)
    with pytest.raises(vg.VgemmError, match="conv source"):
        vg.k_gemm_hl2(A2, 64, 16, w, c.Kp, 64, 64, c.Kp, cst, E)
    E.epi = vg.EPI_QKV
    with pytest.raises(vg.VgemmError, match="EPI_QKV"):
        vg.k_gemm_hl2(A, 64, 64, w, c.Kp, 64, 64, c.Kp, cst, E)

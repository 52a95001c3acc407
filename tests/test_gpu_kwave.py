"""GPU parity of the K-split-over-waves kernel (variant 5, vela_amd/csrc/kwave_kernel.h) against the
oracle: int8 planes with shifts and a residual, int16 rows with K tails (K % 64 and K % 16 == 8),
the PLAIN / GEGLU / GELU / SPLIT3 epilogues with the row maximum, SRC_CONV16 images (C % 64 == 0,
strides 1 and 2, shifts from e or from the pixel maxima), fewer K steps than waves, and the
skinny shapes it exists for (the cross-attention K/V projection and the batch-1 linear)."""
import numpy as np
import pytest

import oracle
from tests.test_gpu_gemm import Case, rng
from vela_amd import configs as cf
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu

KW = 5


@pytest.fixture(autouse=True)
def _variant(gpu):
    vg.set_variant(KW)
    yield
    vg.set_variant(-1)


@pytest.mark.parametrize("shape", [(64, 64, 64), (100, 80, 48), (300, 200, 320), (257, 130, 96), (640, 320, 1280), (70, 64, 16)])
def test_kw_i8_planes_residual(shape):
    M, N, K = shape
    Case(vg.SRC_I8, M, N, K, seed=hash(shape) % 1000 + 5, residual=True, e_max=11).check(what=f"kw I8 {shape}")


@pytest.mark.parametrize("shape", [(64, 64, 64), (100, 80, 40), (300, 200, 328), (257, 130, 96), (640, 320, 1288), (33, 64, 8)])
def test_kw_i16_plain(shape):
    M, N, K = shape
    Case(vg.SRC_I16, M, N, cf.align(K, 8), seed=77, s_range=(16, 24)).check(what=f"kw I16 {shape}")


@pytest.mark.parametrize("epi", [vg.EPI_PLAIN, vg.EPI_GEGLU, vg.EPI_GELU])
def test_kw_epilogues_rowmax(epi):
    Case(vg.SRC_I16, 384, 256, 320, epi=epi, seed=11, rowmax=True, e_max=3, s_range=(16, 24)).check(what=f"kw epi {epi}")
    Case(vg.SRC_I16, 130, 192, 1024, epi=epi, seed=12, rowmax=True, s_range=(20, 28)).check(what=f"kw epi {epi} deep")


def test_kw_split3():
    Case(vg.SRC_I16, 200, 3 * 96, 128, epi=vg.EPI_SPLIT3, seed=12, Cs=96).check(what="kw split3")


@pytest.mark.parametrize("geom", [(2, 8, 8, 64, 1), (1, 7, 5, 64, 2), (2, 6, 6, 320, 1), (2, 4, 4, 1280, 1)])
def test_kw_conv16(geom):
    B, H, W, C, stride = geom
    Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
    Case(vg.SRC_CONV16, B * Ho * Wo, 96, 9 * C, seed=14, conv=geom, residual=True).check(what=f"kw conv16 {geom}")


def test_kw_conv16_shifts_and_pixel_maxima():
    B, H, W, C, stride = 2, 6, 5, 64, 1
    c = Case(vg.SRC_CONV16, B * H * W, 128, 9 * C, seed=31, conv=(B, H, W, C, stride), residual=True)
    c.img[0, :2] = -32768
    c.e = rng(32).integers(0, 18, c.M).astype(np.int32)
    c.e[::7] = 0
    c.check(what="kw conv16 e")
    c = Case(vg.SRC_CONV16, B * H * W, 128, 9 * C, seed=33, conv=(B, H, W, C, stride), residual=True)
    c.img.reshape(-1)[::97] = -32768
    c.pm = oracle.pixmax(c.img.astype(np.int32).reshape(-1, C), B * H * W, C)
    c.e = oracle.conv_e(c.pm, B, H, W, stride)
    assert c.e.max() > 0
    c.pm_in_kernel = True
    c.check(what="kw conv16 pm")


def test_kw_skinny_shapes():
    """The cross-attention K/V projection [8 * 77 x 1024] x [1024 -> 1280] and the batch-1 linear
    4096 x 320 x 320 of the benchmark configurations."""
    Case(vg.SRC_I16, 616, 1280, 1024, seed=40, s_range=(16, 24)).check(what="kw K/V")
    Case(vg.SRC_I16, 4096, 320, 320, seed=41, s_range=(16, 24), residual=True).check(what="kw C1")

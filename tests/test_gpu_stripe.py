"""GPU parity of the row-stationary kernel (shallow K, many rows: the C2 GEGLU up-projection path)
against the CPU oracle, byte for byte.

The kernel is forced with variant 4 (stripe_kernel.h, 32 rows per wave) and variant 6
(stripe16_kernel.h, 16 rows per wave; calls with a residual stay on the former) on shapes where it
applies (int16 rows or int8 planes, Kp <= 320, output columns a multiple of four); shapes with a
deeper K run the tile kernels under the same setting, which these cases then cover as well. Cases
follow src/test_gemm_hl.cu:53-86 (random operands, e shifts, residual) and cover what is particular
to these kernels: K not a multiple of 64, partial row stripes and W chunks, blocks that stream many
chunks (large M) or one chunk (small M), and the two epilogue forms (the integer form, and the
int64 formula for blocks with row shifts, shifts outside [0, 31], possible saturation or a table
outside [0, 65536]).
"""
import numpy as np
import pytest

from tests.test_gpu_gemm import Case, rng
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=[4, 6], ids=["stripe", "stripe16"])
def _stripe(gpu, request):
    vg.set_variant(request.param)
    vg.set_splitk(0)
    yield
    vg.set_variant(-1)
    vg.set_splitk(0)


# (M, N, K): Kp <= 320 (the kernel) and deeper K (tile kernels), partial stripes/chunks, one-chunk
# and many-chunk blocks
SHAPES = [(300, 200, 320), (257, 136, 64), (130, 96, 200), (200, 128, 328), (129, 64, 640), (4100, 640, 320), (2100, 320, 600)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("src", [vg.SRC_I16, vg.SRC_I8])
def test_stripe_plain_residual(src, shape):
    M, N, K = shape
    Case(src, M, N, K, seed=60 + K % 97, residual=True, rowmax=True, s_range=(16, 24)).check(what=f"stripe {src} {shape}")


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("src", [vg.SRC_I16, vg.SRC_I8])
@pytest.mark.parametrize("epi", [vg.EPI_PLAIN, vg.EPI_GEGLU, vg.EPI_GELU])
def test_stripe_no_residual(src, shape, epi):
    """Calls without a residual (the ones both kernels serve), with and without the row maximum, in
    the integer form and (e != 0 on odd M) the int64 form."""
    M, N, K = shape
    kw = dict(e_max=7) if M % 2 else dict(s_range=(16, 24))
    Case(src, M, N, K, epi=epi, seed=100 + K % 83 + epi, rowmax=M % 3 != 0, **kw).check(what=f"stripe epi {epi} {src} {shape}")


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("src", [vg.SRC_I16, vg.SRC_I8])
def test_stripe_shifts(src, shape):
    """Per-row shifts e in [0, 11] (the general FP64 form, src/test_gemm_hl.cu:60-62)."""
    M, N, K = shape
    Case(src, M, N, K, seed=70 + K % 89, residual=True, e_max=11).check(what=f"stripe e {src} {shape}")


@pytest.mark.parametrize("epi", [vg.EPI_PLAIN, vg.EPI_GEGLU, vg.EPI_GELU])
@pytest.mark.parametrize("K", [320, 512])
def test_stripe_epilogues(epi, K):
    """Each epilogue in each form: folded (e = 0, small b), general (e != 0), b near +-2^31, a GEGLU
    product far beyond 2^31, and the int64 formula (shifts outside [1, 52], wrapping m)."""
    forms = [
        ("fold", dict(s_range=(16, 24))),
        ("e", dict(s_range=(16, 24), e_max=3)),
        ("b near 2^31", dict(s_range=(16, 20), m_range=(1 << 10, 1 << 12), b_range=(-(2**31), 2**31))),
        ("large y", dict(s_range=(16, 16), m_range=(1 << 16, 1 << 18))),
        ("left shifts", dict(s_range=(-6, 3), m_range=(1, 1 << 10), e_max=5)),
        ("deep shifts", dict(s_range=(50, 70))),
        ("wrapping m", dict(s_range=(20, 40), m_range=((1 << 30), (1 << 31) - 1))),
        # 2 |m| >= 2^s with no possible saturation at Kp = 320: the int64 form
        ("m at 2^(s-1)", dict(s_range=(16, 16), m_range=(1 << 15, 50000))),
    ]
    for i, (name, kw) in enumerate(forms):
        Case(vg.SRC_I16, 384, 256, K, epi=epi, seed=80 + i, rowmax=True, residual=epi == vg.EPI_PLAIN, **kw).check(what=f"{name} epi {epi} K {K}")
        if epi == vg.EPI_PLAIN:
            Case(vg.SRC_I16, 384, 256, K, epi=epi, seed=80 + i, rowmax=True, **kw).check(what=f"{name} epi {epi} K {K}, no residual")


def test_stripe_lut_outside_range():
    lut = rng(5).integers(-70000, 140000, 2049).astype(np.int32)
    for epi in (vg.EPI_GEGLU, vg.EPI_GELU):
        Case(vg.SRC_I16, 256, 128, 320, epi=epi, seed=90, lut=lut, rowmax=True).check(what=f"stripe lut epi {epi}")


def test_stripe_c2_rows():
    """The C2 geometry (K = 320, N = 2560 interleaved a/g columns, GEGLU + row max) on 4096 rows,
    with activations holding -32768 and 32767 and a Laplace-like spread."""
    c = Case(vg.SRC_I16, 4096, 2560, 320, epi=vg.EPI_GEGLU, seed=91, rowmax=True, s_range=(16, 24))
    c.q[0, :] = -32768
    c.q[1, :] = 32767
    c.q[2, ::2] = -32768
    c.check(what="stripe C2 rows")


def test_stripe_gelu_residual():
    """GELU with a residual (the reference adds it after the GELU, src/gemm_hl.cu:280-284) under the
    forced variant: the row-stationary kernel adds residuals to PLAIN outputs only, so the call runs
    on the tile kernels."""
    Case(vg.SRC_I16, 384, 256, 320, epi=vg.EPI_GELU, seed=92, residual=True, rowmax=True, s_range=(16, 24)).check(what="stripe gelu residual")


@pytest.mark.parametrize("src", [vg.SRC_I16, vg.SRC_I8])
def test_stripe_geglu_saturating_integer_form(src):
    """The integer form's saturating GEGLU products (|a ge| >= 2^47 while a and g themselves fit in
    int32, so the block keeps the integer form), both signs, in full and partial row stripes (M = 300:
    two full stripes of 128 rows and one of 44), with the row maximum."""
    c = Case(src, 300, 256, 64, epi=vg.EPI_GEGLU, seed=93, rowmax=True, s_range=(16, 16),
             m_range=(1 << 17, 1 << 18), b_range=(-1000, 1000))
    if src == vg.SRC_I16:
        c.q[::7, :] = 32767
        c.q[3::7, :] = -32768
    else:
        c.hi[:300:7, :] = 127
        c.lo[:300:7, :] = 127
        c.hi[3:300:7, :] = -128
        c.lo[3:300:7, :] = -128
    want, _ = c.reference()
    imax, imin = np.iinfo(np.int32).max, np.iinfo(np.int32).min
    for rows in (slice(0, 256), slice(256, 300)):
        assert (want[rows] == imax).any() and (want[rows] == imin).any(), "the case must saturate both ways"
    c.check(what=f"stripe saturating GEGLU {src}")

"""GPU parity where the reference's fixed-width arithmetic wraps.

* acc * m: the epilogue forms acc = 256*Chi + Clo + 128*wsum exactly and multiplies it by m in int64
  (src/gemm_hl.cu:40-43). With K = 11520 (the UNet's deepest convolution), activations at +-32767,
  weights at +-127 and m near 2^31, |acc * m| reaches 2^66: the product wraps mod 2^64 and the
  rounding add can wrap as well. The expected bytes come from an int64 matmul of the full 16-bit
  activations and the wrap-aware restatement tests/refmath.py:epi1_dev, and from the oracle.
* lut16i: the table interpolation a + (((b - a) * f) >> 10) runs in int32 (src/intops.cuh:42-50). A
  table with entries across the whole int32 range makes b - a and (b - a) * f wrap; expected bytes
  from refmath's gelu_dev / geglu_dev applied to the plain outputs, and from the oracle.
Each case first asserts that the wrap really happens on its inputs.
"""
import numpy as np
import pytest
import torch

from tests import refmath as rm
from tests.conftest import assert_equal
from tests.test_gpu_gemm import Case, rng
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _knobs(gpu):
    vg.set_variant(-1)
    vg.set_splitk(0)
    yield
    vg.set_variant(-1)
    vg.set_splitk(0)


def extreme_case(src, seed):
    """M = 128 rows of +-32767 (a few entries flipped), W rows at +-127, m in [2^31 - 2^16, 2^31)."""
    M, N, K = 128, 64, 11520
    c = Case(vg.SRC_I16, M, N, K, seed=seed, s_range=(0, 62), m_range=((1 << 31) - (1 << 16), (1 << 31) - 1),
             b_range=(-(2**31), 2**31 - 1))
    r = rng(seed + 1000)
    q = np.full((M, K), 32767, np.int64) * r.choice([-1, 1], (M, 1))
    flip = r.random((M, K)) < 0.02
    q[flip] = -q[flip]
    q[0, :7] = -32768                      # the one value the 16-bit range adds
    c.q = q.astype(np.int16)
    c.kw = dict(q16=c.q, K=K)
    wv = 127 * r.choice([-1, 1], (N, 1)) * np.ones((1, K), np.int64)
    wv[r.random((N, K)) < 0.02] *= -1
    c.w[:N, :K] = wv
    c.cst[:N, 3] = wv.sum(1)
    if src == vg.SRC_I8:
        hi, lo = rm.split(np.pad(q, ((0, c.Mp - M), (0, c.Kp - K))))
        hi[M:], lo[M:] = 0, -128
        c.src, c.hi, c.lo = vg.SRC_I8, hi, lo
        c.kw = dict(hi=hi, lo=lo)
    return c, q


def expected_wrapped(c, q):
    acc = q @ c.w[:c.N, :c.K].astype(np.int64).T          # |acc| < 2^36: exact in int64
    m, s, b = (c.cst[:c.N, i].astype(np.int64) for i in range(3))
    prod = [[int(acc[i, j]) * int(m[j]) for j in range(c.N)] for i in range(c.M)]
    nwrap = sum(abs(p) >= 2**63 for row in prod for p in row)
    y = np.array([[rm.epi1_dev(acc[i, j], m[j], s[j], 0, b[j]) for j in range(c.N)] for i in range(c.M)], np.int64)
    return y.astype(np.int32), nwrap


@pytest.mark.parametrize("src", [vg.SRC_I16, vg.SRC_I8])
@pytest.mark.parametrize("variant,splits", [(-1, 0), (0, 0), (3, 0), (1, 3)])
def test_acc_times_m_wraps(src, variant, splits):
    vg.set_variant(variant)
    vg.set_splitk(splits)
    c, q = extreme_case(src, seed=300 + 7 * variant + splits)
    want, nwrap = expected_wrapped(c, q)
    assert nwrap > c.M * c.N // 2, "the case must overflow the int64 product"
    oracle_y, _ = c.reference()
    assert_equal(oracle_y, want, "oracle vs refmath.epi1_dev")
    ws = vg.workspace_bytes(c.Mp, c.M, c.Np, c.N, c.Kp, 0) if splits else 0
    c.check(ws_bytes=ws, what=f"acc*m wrap src {src} v{variant} s{splits}")


def _wide_table(seed):
    return rng(seed).integers(-(2**31), 2**31, 2049, dtype=np.int64).astype(np.int32)


@pytest.mark.parametrize("epi", [vg.EPI_GELU, vg.EPI_GEGLU])
@pytest.mark.parametrize("variant", [-1, 4])
def test_lut_interpolation_wraps(epi, variant):
    vg.set_variant(variant)
    lut = _wide_table(31 + epi)
    kw = dict(seed=320 + epi, lut=lut, rowmax=True)
    plain = Case(vg.SRC_I16, 256, 128, 64, **kw)
    y, _ = plain.reference()
    c = Case(vg.SRC_I16, 256, 128, 64, epi=epi, **kw)
    assert np.array_equal(c.q, plain.q) and np.array_equal(c.w, plain.w)
    if epi == vg.EPI_GELU:
        pts = y.reshape(-1)
        want = np.array([[rm.gelu_dev(int(v), lut) for v in row] for row in y], np.int64).astype(np.int32)
    else:
        pts = y[:, 1::2].reshape(-1)
        want = np.array([[rm.geglu_dev(int(row[2 * j]), int(row[2 * j + 1]), lut) for j in range(y.shape[1] // 2)] for row in y],
                        np.int64).astype(np.int32)
    nwrap = sum(rm.lut_dev(int(x), lut) != rm.lut(int(x), lut) for x in pts)
    assert nwrap > len(pts) // 4, "the case must wrap the int32 interpolation"
    oracle_y, _ = c.reference()
    assert_equal(oracle_y, want, "oracle vs refmath")
    c.check(what=f"lut wrap epi {epi} v{variant}")

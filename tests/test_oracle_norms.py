"""Pins of the oracle's integer normalisations (oracle/oracle.c: orc_gn_*, orc_lnorm*, src/kernels.cu:172-305,
349-420) by what the mathematics fixes: exact integer square roots and floor divisions against Python's,
the GroupNorm statistics against numpy sums/minima/maxima and exact rounding, the normalised value
against an exact rational, special cases with closed forms (identity normalisation, constant rows,
symmetric rows), and the activation / int16-view tails against the already pinned GELU-table and
quant_rows definitions. The reference's own GPU test (src/test_normalization.cpp) is mirrored by the
edge inputs: INT_MIN / INT_MAX, random g and beta, e = 12."""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle
from tests import refmath as rm


def sat32(v):
    return max(-(2**31), min(2**31 - 1, v))


def rhu(fr: Fraction) -> int:
    """round half up of a rational."""
    return math.floor(fr + Fraction(1, 2))


def test_isqrt_and_floor_div():
    r = np.random.default_rng(1)
    vals = [0, 1, 2, 3, 4, 15, 16, 17, 2**31, 2**52 - 1, 2**52 + 1, 2**62, 2**62 + 12345] + [int(v) for v in r.integers(0, 2**62, 200)]
    vals += [k * k - 1 for k in (3, 2**20, 2**31 - 1)] + [k * k for k in (3, 2**20, 2**31 - 1)]
    for v in vals:
        assert oracle.isqrt(v) == math.isqrt(v), v
    for a_, b_ in [(-7, 2), (7, -2), (-8, 2), (0, 5), (-1, 2**40), (2**61, 3)] + [(int(x), int(y)) for x, y in
                                                                               zip(r.integers(-2**62, 2**62, 200), r.integers(1, 2**40, 200))]:
        assert oracle.floor_div(a_, b_) == a_ // b_, (a_, b_)


def make_x(r, B, T, C, mode):
    if mode == 0:
        return np.zeros((B * T, C), np.int32)
    if mode == 1:
        return r.integers(-1000000, 1000001, (B * T, C)).astype(np.int32)
    x = r.integers(-(2**31), 2**31, (B * T, C), dtype=np.int64).astype(np.int32)
    x[0, 0], x[0, 1] = -(2**31), 2**31 - 1
    return x


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("B,T,C,groups", [(2, 5, 64, 32), (1, 33, 320, 32), (2, 16, 96, 8)])
def test_gn_statistics(mode, B, T, C, groups):
    r = np.random.default_rng(mode * 100 + C)
    x = make_x(r, B, T, C, mode)
    gs = oracle.gn_stats1(x, B, T, C, groups)
    cg, n = C // groups, T * (C // groups)
    xr = x.astype(np.int64).reshape(B, T, groups, cg)
    for b in range(B):
        for g in range(groups):
            reg = xr[b, :, g, :]
            s = gs[b * groups + g]
            assert s["sum"] == reg.sum() and s["mn"] == reg.min() and s["mx"] == reg.max()
            mean = rhu(Fraction(int(reg.sum()), n))
            assert s["mean"] == mean
            m = max(int(reg.max()) - mean, mean - int(reg.min()))
            assert s["e"] == max(0, min(17, max(0, m.bit_length() - 15)) - 5)
    den = 100000
    oracle.gn_stats2(x, B, T, C, groups, den, gs)
    for b in range(B):
        for g in range(groups):
            s = gs[b * groups + g]
            e = int(s["e"])
            d = xr[b, :, g, :] - int(s["mean"])
            dd = d if e == 0 else (d + (1 << (e - 1))) >> e      # round half up of d / 2^e
            ss = int((dd * dd).sum())
            assert s["ss"] == ss
            eps = (2 ** (32 - 2 * e) + den // 2) // den
            assert s["sd"] == math.isqrt(((ss // n) + eps) << 16)


def gn_value(x, s, g, beta):
    """The applied value from its definition: the round-half-up Q24 quotient (x - mean) 2^24 / sd,
    then rshr by 16 of its product with g, plus beta, saturated."""
    yy = rhu(Fraction((int(x) - int(s["mean"])) * 2 ** (24 - int(s["e"])), int(s["sd"])))
    return sat32(rm.rshr(yy * int(g), 16) + int(beta))


def test_gn_apply_row_identity_and_shift():
    """mean 0, e 0, sd 2^24, g 2^16, beta 0 is the identity; a mean shifts; beta adds, saturating."""
    r = np.random.default_rng(5)
    B, T, C, groups = 2, 3, 64, 32
    x = r.integers(-(2**31), 2**31, (B * T, C), dtype=np.int64).astype(np.int32)
    gs = oracle.gn_records(B * groups)
    gs["mean"], gs["e"], gs["sd"] = 0, 0, 2**24
    g = np.full(C, 65536, np.int32)
    beta = np.zeros(C, np.int32)
    Y, pm = oracle.gn_apply_row(x, B, T, C, groups, gs, g, beta)
    assert np.array_equal(Y, x)
    assert np.array_equal(pm, np.abs(x.astype(np.int64)).max(1).astype(np.uint32))
    gs["mean"] = 12345
    beta[:] = r.integers(-(2**31), 2**31, C, dtype=np.int64).astype(np.int32)
    Y, _ = oracle.gn_apply_row(x, B, T, C, groups, gs, g, beta)
    want = np.clip(x.astype(np.int64) - 12345 + beta.astype(np.int64), -(2**31), 2**31 - 1)
    assert np.array_equal(Y, want.astype(np.int32))


@pytest.mark.parametrize("mode", [1, 2])
def test_gn_apply_row_against_definition(mode):
    """Random statistics as the reference's test draws them (sd = 65536 + U[0, 1e8), e = 12 and
    random g/beta in mode 2), every element against the rational definition; the SiLU tail against the
    table activation, the int16 view against quant_rows."""
    r = np.random.default_rng(20 + mode)
    B, T, C, groups = 2, 5, 64, 32
    x = make_x(r, B, T, C, mode)
    gs = oracle.gn_records(B * groups)
    gs["mean"] = r.integers(-500000, 500001, B * groups) if mode == 1 else r.integers(-(2**31), 2**31, B * groups, dtype=np.int64)
    gs["e"] = 12 if mode == 2 else 0
    gs["sd"] = 65536 + r.integers(0, 100000000, B * groups)
    g = (r.integers(-(2**31), 2**31, C, dtype=np.int64) if mode == 2 else np.full(C, 65536)).astype(np.int32)
    beta = (r.integers(-(2**31), 2**31, C, dtype=np.int64) if mode == 2 else np.zeros(C)).astype(np.int32)
    Y, pm = oracle.gn_apply_row(x, B, T, C, groups, gs, g, beta)
    cg = C // groups
    for row in range(B * T):
        for c in range(C):
            assert Y[row, c] == gn_value(x[row, c], gs[(row // T) * groups + c // cg], g[c], beta[c]), (row, c)
    L = (np.arange(2049) * 32).astype(np.int32)
    Ya, _ = oracle.gn_apply_row(x, B, T, C, groups, gs, g, beta, Lsig=L)
    assert all(Ya[i, c] == rm.gelu_dev(int(Y[i, c]), L) for i in range(B * T) for c in range(C))
    Kp = C + 16
    hi, lo, e = oracle.gn_apply_row(x, B, T, C, groups, gs, g, beta, Lsig=L, Kp=Kp)
    qh, ql, qe = oracle.quant_rows(Ya, B * T, C, C, Kp)
    assert np.array_equal(hi, qh[:B * T]) and np.array_equal(lo, ql[:B * T]) and np.array_equal(e, qe[:B * T])
    # the elementwise form with 64-bit g/beta gives the same values
    assert np.array_equal(oracle.gn_apply(x, B, T, C, groups, gs, g.astype(np.int64), beta.astype(np.int64)), Y)


def test_lnorm_closed_forms():
    """A constant row normalises to beta; a row of +-a has mean 0 and var = rshr(a, ex)^2, so its
    values are the definition's with sd = isqrt((var + eps) << 16)."""
    C, den = 64, 100000
    beta = np.arange(C, dtype=np.int64) - 7
    g = np.full(C, 65536, np.int64)
    x = np.full((1, C), 123456789, np.int32)
    assert np.array_equal(oracle.lnorm(x, 1, C, g, beta, den)[0], beta)
    for a_ in (3, 40000, 2**30):
        x = np.array([[a_ if c % 2 == 0 else -a_ for c in range(C)]], np.int32)
        ex = max(0, max(0, min(17, a_.bit_length() - 15)) - 5)
        dd = rm.rshr(a_, ex)
        eps = (2 ** (32 - 2 * ex) + den // 2) // den
        sd = math.isqrt((dd * dd + eps) << 16)
        want = [sat32(rm.rshr(rhu(Fraction(int(v) * 2 ** (24 - ex), sd)) * 65536, 16) + int(b)) for v, b in zip(x[0], beta)]
        assert list(oracle.lnorm(x, 1, C, g, beta, den)[0]) == want, a_


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("C", [4, 124, 320, 1280])
def test_lnorm_q_is_quant_rows_of_lnorm(mode, C):
    r = np.random.default_rng(mode * 10 + C)
    M, den, Kp = 9, 100000, (C + 15) // 16 * 16
    x = make_x(r, 1, M, C, mode)
    g = (r.integers(-(2**31), 2**31, C, dtype=np.int64) if mode == 2 else np.full(C, 65536)).astype(np.int32)
    beta = (r.integers(-(2**31), 2**31, C, dtype=np.int64) if mode == 2 else np.zeros(C)).astype(np.int32)
    Y = oracle.lnorm(x, M, C, g.astype(np.int64), beta.astype(np.int64), den)
    hi, lo, e = oracle.lnorm_q(x, M, C, g, beta, den, Kp)
    qh, ql, qe = oracle.quant_rows(Y, M, C, C, Kp)
    assert np.array_equal(hi, qh[:M]) and np.array_equal(lo, ql[:M]) and np.array_equal(e, qe[:M])

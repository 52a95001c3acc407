"""Pins of the oracle's integer primitives (oracle/oracle.c, restating src/intops.cuh:9-66).

Each primitive is checked against its mathematical definition (tests/refmath.py: exact rationals),
against closed forms and special cases, and on the reference's own edge lists
(src/test_attn_score.cu:14, src/test_im2col.cu:34). No GPU.
"""
import ctypes

import numpy as np
import pytest

import oracle
from tests import refmath as rm

# src/test_attn_score.cu:14
EDGES = [-32767, -32766, -32513, -256, -255, -128, -1, 0, 1, 127, 128, 255, 256, 32512, 32766, 32767]


def test_sat32_boundaries():
    L = oracle.lib()
    for v, want in [(0, 0), (2**31 - 1, 2**31 - 1), (2**31, 2**31 - 1), (-(2**31), -(2**31)), (-(2**31) - 1, -(2**31)),
                    (2**62, 2**31 - 1), (-(2**63), -(2**31)), (2**63 - 1, 2**31 - 1), (12345, 12345)]:
        assert L.orc_sat32(v) == want, v


def test_rshr_against_exact_rounding():
    r = np.random.default_rng(1)
    v = np.concatenate([r.integers(-(2**61), 2**61, 4000), r.integers(-5000, 5000, 4000),
                        np.array([0, 1, -1, 2, -2, 3, -3, 2**61, -(2**61)])])
    s = np.concatenate([r.integers(-40, 71, 8000), np.array([1, 1, 1, 1, 1, 1, 1, 62, 62])])
    got = oracle.rshr(v, s)
    want = np.array([rm.rshr(int(a), int(b)) for a, b in zip(v, s)], np.int64)
    np.testing.assert_array_equal(got, want)


def test_rshr_closed_forms():
    L = oracle.lib()
    # halves round up (towards +inf): 0.5 -> 1, -0.5 -> 0, 1.5 -> 2, -1.5 -> -1
    assert [L.orc_rshr(v, 1) for v in (1, -1, 3, -3)] == [1, 0, 2, -1]
    # s = 0 is the identity inside int32, s < 0 a saturating left shift
    assert L.orc_rshr(-77, 0) == -77 and L.orc_rshr(3, -2) == 12 and L.orc_rshr(-3, -2) == -12
    assert L.orc_rshr(1 << 20, -11) == 2**31 - 1 and L.orc_rshr(-(1 << 20), -11) == -(2**31)
    # shifts beyond 62 behave as 62 and beyond -31 as -31
    assert L.orc_rshr(2**61, 100) == L.orc_rshr(2**61, 62) == 1
    assert L.orc_rshr(1, -100) == L.orc_rshr(1, -31) == 2**31 - 1
    # the reference's int64 rounding add wraps at the top of the range (two's complement on the GPU)
    assert L.orc_rshr(2**63 - 1, 1) == -(2**31)


def test_row_exp_definitions_agree():
    """#{k in [15,32): m >= 2^k} (src/intops.cuh:36-37) equals the smallest e with m < 32768 << e
    (src/test_im2col.cu:34) and max(0, bitlen(m) - 15) below 2^32."""
    ms = [0, 1, 32767, 32768, 65535, 65536, 2**31 - 1, 2**31, 2**32 - 1, 2**32, 2**40]
    ms += [2**k + d for k in range(14, 34) for d in (-1, 0, 1)]
    ms += list(np.random.default_rng(2).integers(0, 2**33, 2000))
    got = oracle.row_exp(np.array(ms, np.int64))
    for m, g in zip(ms, got):
        m = int(m)
        assert g == rm.row_exp(m), m
        if m < 2**32:
            assert g == max(0, m.bit_length() - 15), m


def test_quant16_32_against_definition():
    r = np.random.default_rng(3)
    v = np.concatenate([r.integers(-(2**31), 2**31, 6000, dtype=np.int64),
                        np.array([0, 1, -1, 32767, -32767, -32768, 32768, 2**31 - 1, -(2**31)] * 18)]).astype(np.int32)
    e = np.concatenate([r.integers(0, 18, 6000), np.repeat(np.arange(18), 9)]).astype(np.int32)
    got = oracle.quant16_32(v, e)
    want = np.array([rm.quant16(int(a), int(b)) for a, b in zip(v, e)], np.int32)
    np.testing.assert_array_equal(got, want)
    # quant16 (int64 form) is the same function
    L = oracle.lib()
    for a, b in zip(v[:500], e[:500]):
        assert L.orc_quant16(int(a), int(b)) == rm.quant16(int(a), int(b))


def test_quant16_row_of_int16_is_identity_except_minus_32768():
    """Rows of int16 data have max |x| <= 32768 < 2^16, so e = 0 only when max |x| < 32768; with
    e = 0, q = x except -32768 -> -32767 (the clamp)."""
    x = np.arange(-32768, 32768, dtype=np.int32)
    q = oracle.quant16_32(x, 0)
    want = x.copy()
    want[0] = -32767
    np.testing.assert_array_equal(q, want)


def test_split16_exhaustive():
    """q = 256*hi + lo + 128 for every 16-bit q, both halves in int8, and 0 -> (0, -128)."""
    qs = np.arange(-32768, 32768)
    his, los = rm.split(qs)
    np.testing.assert_array_equal(256 * his.astype(np.int64) + los + 128, qs)
    for q in list(range(-32768, 32768, 97)) + EDGES + [-32768]:
        h, l = oracle.split16(q)
        assert 256 * h + l + 128 == q, q
        assert (h, l) == (int(his[q + 32768]), int(los[q + 32768]))
    assert oracle.split16(0) == (0, -128)


def test_lut16i_closed_forms():
    L = oracle.lib()
    # a linear table L[i] = c*i interpolates exactly to floor(c*z/1024), z = x + 2^20
    for c in (0, 1, 7, 32):
        tab = (c * np.arange(2049)).astype(np.int32)
        xs = np.random.default_rng(c).integers(-(1 << 20), (1 << 20) - 1, 3000)
        got = oracle.lut16i(xs, tab)
        z = xs + (1 << 20)
        np.testing.assert_array_equal(got, (c * z) // 1024)
    # grid points return the table entry; below the table 0, at or above its end 65536
    tab = np.random.default_rng(9).integers(0, 65537, 2049).astype(np.int32)
    for i in (0, 1, 1000, 2047):
        assert oracle.lut16i(np.array([i * 1024 - (1 << 20)]), tab)[0] == tab[i]
    assert oracle.lut16i(np.array([-(1 << 20) - 1, -(2**40)]), tab).tolist() == [0, 0]
    assert oracle.lut16i(np.array([1 << 20, 2**40]), tab).tolist() == [65536, 65536]
    # a monotone table interpolates monotonically
    mono = np.sort(tab)
    xs = np.arange(-(1 << 20), 1 << 20, 37)
    assert np.all(np.diff(oracle.lut16i(xs, mono)) >= 0)
    # random table against the definition
    xs = np.random.default_rng(10).integers(-(1 << 21), 1 << 21, 3000)
    np.testing.assert_array_equal(oracle.lut16i(xs, tab), [rm.lut(int(x), tab) for x in xs])


def test_epi1_against_definition():
    """epi1 = sat32(rshr((256 chi + clo + 128 wsum) * m, s - e) + b) (src/gemm_hl.cu:40-43), over the
    ranges the planes take (|chi|, |clo| <= 2^14 Kp)."""
    r = np.random.default_rng(4)
    n = 5000
    Kp = r.integers(16, 4096, n)
    chi = (r.integers(-(2**14), 2**14, n) * Kp // 64).astype(np.int32)
    clo = (r.integers(-(2**14), 2**14, n) * Kp // 64).astype(np.int32)
    m = r.integers(-(2**31), 2**31, n, dtype=np.int64)
    m[::3] = r.integers(1 << 14, 1 << 15, (n + 2) // 3)
    s = r.integers(-20, 70, n)
    b = r.integers(-(2**31), 2**31, n, dtype=np.int64)
    wsum = r.integers(-127 * 4096, 127 * 4096, n)
    er = r.integers(0, 18, n).astype(np.int32)
    cst = np.stack([m, s, b, wsum], 1).astype(np.int32)
    got = oracle.epi1(chi, clo, cst, er)
    want = []
    for i in range(n):
        acc = 256 * int(chi[i]) + int(clo[i]) + 128 * int(wsum[i])
        want.append(rm.sat32(rm.rshr(acc * int(m[i]), int(s[i]) - int(er[i])) + int(b[i])))
    np.testing.assert_array_equal(got, want)


def test_geglu_gelu_against_definition():
    r = np.random.default_rng(5)
    tab = np.sort(r.integers(0, 65537, 2049)).astype(np.int32)
    L = oracle.lib()
    tp = tab.ctypes.data_as(ctypes.c_void_p)
    vals = list(r.integers(-(2**31), 2**31, 3000, dtype=np.int64)) + [0, 1, -1, 2**31 - 1, -(2**31), 1 << 20, -(1 << 20)]
    for i, a in enumerate(vals):
        g = vals[(i * 7 + 3) % len(vals)]
        assert L.orc_geglu(int(a), int(g), tp) == rm.geglu(int(a), int(g), tab)
        assert L.orc_gelu(int(a), tp) == rm.gelu(int(a), tab)


def test_dev_forms_equal_definitions_without_wrap():
    """The wrap-aware restatements reduce to the exact-rational definitions wherever no fixed-width
    operation overflows."""
    r = np.random.default_rng(21)
    for _ in range(3000):
        v = int(r.integers(-(2**61), 2**61))
        s = int(r.integers(-40, 70))
        assert rm.rshr_dev(v, s) == rm.rshr(v, s)
    tab = r.integers(0, 65537, 2049)
    for x in r.integers(-(1 << 21), 1 << 21, 2000):
        assert rm.lut_dev(int(x), tab) == rm.lut(int(x), tab)


def test_dev_forms_known_wraps():
    """Worked values where the reference's fixed-width arithmetic wraps."""
    # rounding add: 2^63 - 1 + 2^0 wraps to -2^63, so rshr(2^63 - 1, 1) = sat32(-2^62) = INT_MIN
    assert rm.rshr_dev(2**63 - 1, 1) == -(2**31)
    # product: 2^40 * 2^24 = 2^64 wraps to 0; (2^40 + 1) * 2^24 wraps to 2^24
    assert rm.epi1_dev(2**40, 2**24, 20, 0, 7) == 7
    assert rm.epi1_dev(2**40 + 1, 2**24, 10, 0, 7) == 2**14 + 7
    # product 3 * 2^62 wraps to -2^62: rshr(-2^62, 40) = -2^22
    assert rm.epi1_dev(3 * 2**31, 2**31, 40, 0, 0) == -(2**22)
    # table: a = -2^31 + 1, b = 2^31 - 1, f = 512: b - a wraps to -2, the product to -1024, and
    # a + (-1024 >> 10) = -2^31 (the unwrapped interpolation would give 0)
    L = np.zeros(2049, np.int64)
    L[5], L[6] = -(2**31) + 1, 2**31 - 1
    x = 5 * 1024 + 512 - (1 << 20)
    assert rm.lut(x, L) == 0 and rm.lut_dev(x, L) == -(2**31)
    # (b - a) * f wraps without b - a wrapping: a = 0, b = 2^22, f = 1023 -> 2^22 * 1023 mod 2^32
    L[5], L[6] = 0, 2**22
    x = 5 * 1024 + 1023 - (1 << 20)
    assert rm.lut_dev(x, L) == rm.wrap32(2**22 * 1023) >> 10 and rm.lut(x, L) == (2**22 * 1023) >> 10


def test_epi1_wraps_like_the_reference():
    """|acc * m| >= 2^63: the int64 product of src/gemm_hl.cu:41 wraps; the oracle's epi1 agrees
    with the wrap-aware restatement on the K = 11520 extremes (|acc| up to 11520 * 32767 * 127)."""
    r = np.random.default_rng(22)
    n = 4000
    acc_target = r.integers(-(11520 * 32767 * 127), 11520 * 32767 * 127, n, dtype=np.int64)
    wsum = r.integers(-127 * 11520, 127 * 11520, n)
    # split acc = 256 chi + clo + 128 wsum into plane sums of the sizes K = 11520 produces
    rest = acc_target - 128 * wsum
    chi = (rest // 256).astype(np.int64)
    clo = rest - 256 * chi
    m = r.integers((1 << 31) - (1 << 20), 1 << 31, n, dtype=np.int64)
    s = r.integers(0, 63, n)
    b = r.integers(-(2**31), 2**31, n, dtype=np.int64)
    er = np.zeros(n, np.int32)
    cst = np.stack([m, s, b, wsum], 1).astype(np.int32)
    got = oracle.epi1(chi.astype(np.int32), clo.astype(np.int32), cst, er)
    wraps = 0
    for i in range(n):
        acc = 256 * int(chi[i]) + int(clo[i]) + 128 * int(wsum[i])
        wraps += abs(acc * int(m[i])) >= 2**63
        assert got[i] == rm.epi1_dev(acc, int(m[i]), int(s[i]), 0, int(b[i])), i
    assert wraps > n // 4


def test_lut16i_wraps_like_the_reference():
    """Tables whose entries differ by 2^21 or more: (b - a) * f (and b - a itself) wrap in int32."""
    r = np.random.default_rng(23)
    tab = r.integers(-(2**31), 2**31, 2049, dtype=np.int64).astype(np.int32)
    xs = r.integers(-(1 << 20), 1 << 20, 4000)
    got = oracle.lut16i(xs, tab)
    np.testing.assert_array_equal(got, [rm.lut_dev(int(x), tab) for x in xs])
    assert sum(rm.lut_dev(int(x), tab) != rm.lut(int(x), tab) for x in xs) > 1000
    L = oracle.lib()
    tp = tab.ctypes.data_as(ctypes.c_void_p)
    vals = list(r.integers(-(1 << 21), 1 << 21, 1500))
    for i, a in enumerate(vals):
        g = vals[(i * 5 + 1) % len(vals)]
        assert L.orc_geglu(int(a), int(g), tp) == rm.geglu_dev(int(a), int(g), tab)
        assert L.orc_gelu(int(a), tp) == rm.gelu_dev(int(a), tab)


@pytest.mark.parametrize("seed", [0, 1])
def test_attn_score_split_identity(seed):
    """src/test_attn_score.cu:14-24: on the reference's edge list and random quantised operands,
    sum(q*k) over d = 64 is recovered from the int8 halves exactly."""
    r = np.random.default_rng(seed)
    for t in range(400):
        if t < 256:
            q = np.full(64, EDGES[t // 16]); k = np.full(64, EDGES[t % 16])
        else:
            q = r.integers(-32767, 32768, 64); k = r.integers(-32767, 32768, 64)
        qh, ql = (x.astype(np.int64) for x in rm.split(q))
        kh, kl = (x.astype(np.int64) for x in rm.split(k))
        dot = int(np.dot(q.astype(np.int64), k))
        hh, hl, lh, ll = int(qh @ kh), int(qh @ kl), int(ql @ kh), int(ql @ kl)
        t_ = 256 * (hl + lh) + ll + 32768 * int(qh.sum()) + 128 * int(ql.sum()) + 128 * int(k.sum())
        assert -(2**31) <= t_ <= 2**31 - 1
        assert dot == 65536 * hh + t_

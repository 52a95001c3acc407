"""Pins of the oracle's elementwise kernels (oracle/oracle.c: orc_act, orc_geglu_n, orc_add, orc_concat,
orc_upsample2; src/kernels.cu:536-561) by their definitions: the activation and GEGLU against the
exact-rational table interpolation of tests/refmath.py (and its 32-bit wrapping form for tables
outside [0, 65536]), the saturating add against int64 clipping, the concatenation and the x2
nearest-neighbour upsampling against numpy's concatenate / repeat, and the concatenation's GroupNorm
records against a region-by-region numpy restatement of the reference's flush rule, which equals the
exact per-(sample, group) statistics when nothing saturates, with worked cases where a region's group
is all INT_MAX (dropped) or holds one value below it (kept)."""
import numpy as np
import pytest

import oracle
from tests import refmath as rm
from tests.golden import make_poisd as mp

IMAX, IMIN = 2**31 - 1, -(2**31)


def edge_values(r, n):
    base = [0, 1, -1, IMAX, IMIN, IMAX - 1, IMIN + 1, 1 << 20, -(1 << 20), (1 << 20) - 1, -(1 << 20) - 1, 1 << 16, -(1 << 16),
            1023, 1024, -1023, -1024, 65535, -65535]
    return np.array(base + [int(v) for v in r.integers(IMIN, IMAX, n)] + [int(v) for v in r.integers(-(1 << 21), 1 << 21, n)], np.int64).astype(np.int32)


TABLES = {
    "phi": mp.phi_table(),                                        # monotone Q16, within [0, 65536]
    "linear": (np.arange(2049, dtype=np.int64) * 32).astype(np.int32),
    "wild": np.random.default_rng(7).integers(IMIN, IMAX, 2049, dtype=np.int64).astype(np.int32),   # every 32-bit wrap
}


@pytest.mark.parametrize("name", list(TABLES))
def test_act_is_the_table_activation(name):
    L = TABLES[name]
    x = edge_values(np.random.default_rng(1), 600)
    got = oracle.act(x, L)
    ref = rm.gelu if name != "wild" else rm.gelu_dev
    want = np.array([ref(int(v), L) for v in x], np.int64)
    assert np.array_equal(got.astype(np.int64), want)
    if name == "linear":
        # lut is x-affine on the table's range: 65536 * (x + 2^20) / 2^21 rounded down, so y = x lut / 2^16 is a closed form
        inside = (x >= -(1 << 20)) & (x < (1 << 20))
        xs = x[inside].astype(object)
        lut = [(int(v) + (1 << 20)) // 32 for v in xs]
        closed = [rm.sat32(rm.rshr(int(v) * lv, 16)) for v, lv in zip(xs, lut)]
        assert [int(v) for v in got[inside]] == closed


@pytest.mark.parametrize("name", list(TABLES))
def test_geglu_is_the_gated_product(name):
    L = TABLES[name]
    r = np.random.default_rng(2)
    g = edge_values(r, 400)
    a_ = np.roll(edge_values(np.random.default_rng(12), 400), 5)
    got = oracle.geglu_n(a_, g, L)
    ref = rm.geglu if name != "wild" else rm.geglu_dev
    want = np.array([ref(int(x), int(y), L) for x, y in zip(a_, g)], np.int64)
    assert np.array_equal(got.astype(np.int64), want)
    # g above the table's range: lut(g) = 65536 for any table, the gate is g itself and y = sat32(rshr(a g, 16))
    big = np.full(8, 1 << 21, np.int32)
    aa = np.array([0, 1, -1, 12345, -12345, IMAX, IMIN, 99], np.int32)
    assert np.array_equal(oracle.geglu_n(aa, big, L).astype(np.int64),
                          np.array([rm.sat32(rm.rshr(int(x) * (1 << 21), 16)) for x in aa], np.int64))


def test_add_saturates():
    r = np.random.default_rng(3)
    x = edge_values(r, 500)
    y = np.roll(edge_values(r, 500), 7)
    want = np.clip(x.astype(np.int64) + y.astype(np.int64), IMIN, IMAX)
    assert np.array_equal(oracle.add(x, y).astype(np.int64), want)


def gn_regions_numpy(out, T):
    """The reference's concat statistics restated: flat regions of 256 elements, per group, flushed
    when the region's minimum of the group is not INT_MAX; region -> sample of its first row."""
    rows, Co = out.shape
    cg = Co // 32
    flat = out.reshape(-1).astype(np.int64)
    nsamp = (rows + T - 1) // T
    s = np.zeros((nsamp, 32), np.int64)
    mn = np.full((nsamp, 32), IMAX, np.int64)
    mx = np.full((nsamp, 32), IMIN, np.int64)
    for start in range(0, flat.size, 256):
        seg = flat[start:start + 256]
        grp = (np.arange(start, start + seg.size) % Co) // cg
        b = start // Co // T
        for g in np.unique(grp):
            v = seg[grp == g]
            if v.min() != IMAX:
                s[b, g] += v.sum(); mn[b, g] = min(mn[b, g], v.min()); mx[b, g] = max(mx[b, g], v.max())
    return s.reshape(-1), mn.reshape(-1), mx.reshape(-1)


@pytest.mark.parametrize("Ca,Cb,T,B", [(320, 320, 8, 3), (640, 320, 4, 2), (32, 32, 8, 2), (64, 96, 8, 2), (1280, 1280, 1, 4), (8, 24, 8, 1)])
def test_concat_and_records(Ca, Cb, T, B):
    r = np.random.default_rng(Ca + Cb + T)
    rows = B * T
    A = r.integers(-(1 << 24), 1 << 24, (rows, Ca)).astype(np.int32)
    Bm = r.integers(-(1 << 24), 1 << 24, (rows, Cb)).astype(np.int32)
    gs = oracle.gn_records(B * 32)
    out = oracle.concat(A, Ca, Bm, Cb, rows, gs, T)
    assert np.array_equal(out, np.concatenate([A, Bm], axis=1))
    s, mn, mx = gn_regions_numpy(out, T)
    assert np.array_equal(gs["sum"], s) and np.array_equal(gs["mn"], mn) and np.array_equal(gs["mx"], mx)
    # nothing saturates: the same as the exact per-(sample, group) statistics
    ex = oracle.gn_stats(out, rows, Ca + Cb, T)
    assert np.array_equal(gs["sum"], ex["sum"]) and np.array_equal(gs["mn"], ex["mn"]) and np.array_equal(gs["mx"], ex["mx"])
    # without records the concatenation alone
    assert np.array_equal(oracle.concat(A, Ca, Bm, Cb, rows), out)


def test_concat_flush_rule_worked():
    """Ca = Cb = 32, T = 8 (64 columns, groups of two columns, 4 rows per 256-element region): group 0
    of region 0 (rows 0..3, columns 0..1) all INT_MAX is dropped; group 1 of region 1 (rows 4..7,
    columns 2..3) all INT_MAX but one value is kept; INT_MIN groups always count."""
    T, rows = 8, 8
    A = np.arange(rows * 32, dtype=np.int32).reshape(rows, 32)
    Bm = -np.arange(rows * 32, dtype=np.int32).reshape(rows, 32)
    A[0:4, 0:2] = IMAX
    A[4:8, 2:4] = IMAX
    A[6, 3] = IMAX - 1
    A[0:4, 4:6] = IMIN
    gs = oracle.gn_records(32)
    out = oracle.concat(A, 32, Bm, 32, rows, gs, T)
    # group 0: only rows 4..7 (region 1) count
    assert gs["sum"][0] == int(A[4:8, 0:2].astype(np.int64).sum()) and gs["mx"][0] == int(A[4:8, 0:2].max())
    # group 1: region 0 (values 2, 3, 34, 35, ...) and region 1 with the INT_MAX - 1 present
    assert gs["sum"][1] == int(A[:, 2:4].astype(np.int64).sum()) and gs["mx"][1] == IMAX and gs["mn"][1] == 2
    assert gs["mn"][2] == IMIN
    s, mn, mx = gn_regions_numpy(out, T)
    assert np.array_equal(gs["sum"], s) and np.array_equal(gs["mn"], mn) and np.array_equal(gs["mx"], mx)


def test_concat_partial_last_region():
    """rows not a multiple of T (and rows * Co not a multiple of 256): the last region is partial and
    still flushes, into the sample of its first row."""
    Ca, Cb, T, rows = 32, 32, 8, 13
    r = np.random.default_rng(11)
    A = r.integers(-1000, 1000, (rows, Ca)).astype(np.int32)
    Bm = r.integers(-1000, 1000, (rows, Cb)).astype(np.int32)
    gs = oracle.gn_records(2 * 32)
    out = oracle.concat(A, Ca, Bm, Cb, rows, gs, T)
    s, mn, mx = gn_regions_numpy(out, T)
    assert np.array_equal(gs["sum"], s) and np.array_equal(gs["mn"], mn) and np.array_equal(gs["mx"], mx)


@pytest.mark.parametrize("B,H,W,C", [(2, 3, 5, 7), (1, 1, 1, 1), (2, 8, 8, 320), (1, 4, 2, 4)])
def test_upsample2_is_nearest_repeat(B, H, W, C):
    X = np.random.default_rng(B * H + W * C).integers(IMIN, IMAX, (B, H, W, C), dtype=np.int64).astype(np.int32)
    want = np.repeat(np.repeat(X, 2, axis=1), 2, axis=2)
    assert np.array_equal(oracle.upsample2(X, B, H, W, C), want)

"""Pins of the oracle's EPI_QKV head quantisation and GroupNorm statistics (oracle/oracle.c
orc_qkv_heads, orc_gn_accumulate) on the CPU.

Neither has a golden vector in the reference: its tests check the normalisation from supplied
statistics (src/test_normalization.cpp:18-60) and never read back the GEMM's statistics or the QKV
planes. They are pinned here by what the definitions fix:
  - the statistics against numpy reductions over a [sample, row, group, column] view (a wrong group
    index, a dropped residual row or a sample boundary off by one changes them);
  - the head quantisation by its invariants: hi/lo recombine to the 16-bit value, that value is y
    rounded to nearest (ties up) at 2^e and clamped to +-32767, e is the smallest shift with
    max|y| < 2^(15+e), the sums are the sums of the stored bytes, the row index is
    (b*heads + head)*Tp + t, and rows t >= T stay untouched.
"""
import numpy as np
import pytest

import oracle


def _y(r, M, N, scale_bits):
    """int32 values whose magnitudes spread over scale_bits (per row), with extremes planted."""
    bits = r.integers(1, scale_bits + 1, (M, 1))
    v = r.integers(-(2**31), 2**31, (M, N), dtype=np.int64) >> (32 - bits)
    return v.astype(np.int32)


@pytest.mark.parametrize("M,N,T", [(128, 320, 64), (384, 64, 192), (200, 96, 64), (1024, 1280, 256)])
def test_gn_stats_against_numpy(M, N, T):
    r = np.random.default_rng(M + N)
    Y = _y(r, M, N, 31)
    Y[0, 0], Y[-1, -1] = -(2**31), 2**31 - 1
    got = oracle.gn_stats(Y, M, N, T)
    B = -(-M // T)
    pad = np.zeros((B * T, N), np.int64)
    pad[:M] = Y
    valid = np.zeros((B * T, N), bool)
    valid[:M] = True
    v = pad.reshape(B, T, 32, N // 32)
    ok = valid.reshape(B, T, 32, N // 32)
    want_sum = np.where(ok, v, 0).sum(axis=(1, 3)).reshape(-1)
    want_mn = np.where(ok, v, 2**31 - 1).min(axis=(1, 3)).reshape(-1)
    want_mx = np.where(ok, v, -(2**31)).max(axis=(1, 3)).reshape(-1)
    np.testing.assert_array_equal(got["sum"], want_sum)
    np.testing.assert_array_equal(got["mn"], want_mn)
    np.testing.assert_array_equal(got["mx"], want_mx)


def test_gn_stats_accumulate_across_calls():
    """Two outputs added to the same records (the reference's atomics after one k_gn_init)."""
    r = np.random.default_rng(3)
    Y1, Y2 = _y(r, 128, 64, 20), _y(r, 128, 64, 20)
    a, b = oracle.gn_stats(Y1, 128, 64, 64), oracle.gn_stats(Y2, 128, 64, 64)
    s = np.zeros(64, np.int64)
    mn = np.full(64, 2**31 - 1, np.int32)
    mx = np.full(64, -(2**31), np.int32)
    for Y in (Y1, Y2):
        Yc = np.ascontiguousarray(Y)
        oracle.lib().orc_gn_accumulate(oracle.a(Yc), 128, 64, 64, 64, oracle.a(s), oracle.a(mn), oracle.a(mx))
    np.testing.assert_array_equal(s, a["sum"] + b["sum"])
    np.testing.assert_array_equal(mn, np.minimum(a["mn"], b["mn"]))
    np.testing.assert_array_equal(mx, np.maximum(a["mx"], b["mx"]))


INT_MAX, INT_MIN = 2**31 - 1, -(2**31)


@pytest.mark.parametrize("Mp,Np,Kp,src,want", [
    # src/gemm_hl.cu:352-358 with g_gemm_hl_variant = -1, case by case
    (32768, 320, 320, 0, (64, 64)),      # Kp < 2048: the small tile
    (32768, 1280, 2047, 3, (64, 64)),
    (8192, 640, 5760, 0, (64, 128)),     # deep K, Np % 128 == 0: the wide tile
    (512, 1280, 11520, 2, (64, 128)),    # ... for any source
    (32768, 320, 2880, 0, (128, 64)),    # deep K, Np % 128 != 0, Mp % 128 == 0: the tall tile (int8 planes)
    (32768, 320, 2880, 3, (128, 64)),    # int16 rows hold the same planes
    (32768, 320, 2880, 1, (64, 64)),     # register-path sources have no tall tile
    (32768, 320, 2880, 2, (64, 64)),
    (32704, 320, 2880, 0, (64, 64)),     # Mp % 128 != 0: the small tile
])
def test_gn_ref_tile(Mp, Np, Kp, src, want):
    assert oracle.gn_ref_tile(Mp, Np, Kp, src) == want


def _gn_regions(Y, M, N, T, regions):
    """Records by the flush rule, from an explicit list of regions: (sample, rows, cols) with rows
    and cols index arrays. Straight numpy, one region at a time."""
    B = -(-M // T)
    s = np.zeros(B * 32, np.int64)
    mn = np.full(B * 32, INT_MAX, np.int64)
    mx = np.full(B * 32, INT_MIN, np.int64)
    grp = np.arange(N) // (N // 32)
    for b, rows, cols in regions:
        sub = Y[np.ix_(rows, cols)].astype(np.int64)
        for g in np.unique(grp[cols]):
            v = sub[:, grp[cols] == g]
            if v.size == 0 or v.min() == INT_MAX:
                continue
            s[b * 32 + g] += v.sum()
            mn[b * 32 + g] = min(mn[b * 32 + g], v.min())
            mx[b * 32 + g] = max(mx[b * 32 + g], v.max())
    return {"sum": s, "mn": mn, "mx": mx}


def _tile_regions(M, N, T, bm, bn):
    return [(m0 // T, np.arange(m0, min(m0 + bm, M)), np.arange(n0, min(n0 + bn, N)))
            for m0 in range(0, M, bm) for n0 in range(0, N, bn)]


def _block_regions(M, N, T):
    out = []
    for e0 in range(0, M * N, 1024):
        idx = np.arange(e0, min(e0 + 1024, M * N))
        r, n = idx // N, idx % N
        for rr in np.unique(r):   # a block is a run of whole and partial rows
            out.append(((e0 // N) // T, np.array([rr]), n[r == rr]))
    return out


def _check(got, want):
    for k in ("sum", "mn", "mx"):
        np.testing.assert_array_equal(got[k], want[k], err_msg=k)


@pytest.mark.parametrize("M,N,T,tile", [(256, 320, 128, (64, 64)), (256, 320, 64, (128, 64)),
                                        (200, 1280, 64, (64, 128)), (384, 96, 192, (64, 64))])
def test_gn_tiles_without_saturation_equal_exact(M, N, T, tile):
    """No output is INT_MAX: the flush rule never fires and the statistics are the exact ones
    (when every tile lies in one sample)."""
    r = np.random.default_rng(M * N)
    Y = _y(r, M, N, 30)
    Y[0, 0] = INT_MIN
    got = oracle.gn_stats_fused(Y, M, N, T, 0, 0, 0, 0, tile=tile)
    if T % tile[0] == 0:
        _check(got, oracle.gn_stats(Y, M, N, T))
    _check(got, _gn_regions(Y, M, N, T, _tile_regions(M, N, T, *tile)))


@pytest.mark.parametrize("tile", [(64, 64), (128, 64), (64, 128)])
def test_gn_tiles_drop_saturated_tile_groups(tile):
    """A tile whose outputs of a group are all INT_MAX adds neither their sum nor their max; one
    more element below INT_MAX in that tile and group brings the whole tile-group back."""
    M, N, T = 256, 320, 128       # groups of 10 columns
    r = np.random.default_rng(7)
    Y = _y(r, M, N, 20)
    bm, bn = tile
    Y[:bm, :bn] = INT_MAX                  # tile (0, 0): groups 0..bn/10 saturated through
    Y[128:128 + bm, 0:10] = INT_MAX        # a tile of sample 1, group 0 only
    Y[128 + bm - 1, 5] = 17                # ... but one element of it is not: that tile-group counts
    Y[:, 300:310] = INT_MIN                # group 30 at INT_MIN everywhere: always counts
    got = oracle.gn_stats_fused(Y, M, N, T, 0, 0, 0, 0, tile=tile)
    _check(got, _gn_regions(Y, M, N, T, _tile_regions(M, N, T, bm, bn)))
    exact = oracle.gn_stats(Y, M, N, T)
    # group 0 of sample 0: the saturated tile (0, 0) is dropped
    assert got["sum"][0] == exact["sum"][0] - bm * 10 * INT_MAX
    assert got["sum"][32] == exact["sum"][32] and got["mx"][32] == INT_MAX
    assert got["mx"][0] < INT_MAX and exact["mx"][0] == INT_MAX
    assert got["mn"][0] == exact["mn"][0]
    assert got["mn"][30] == INT_MIN and got["sum"][30] == exact["sum"][30]


def test_gn_tiles_whole_tile_to_first_rows_sample():
    """A 128-row tile over samples of 64 rows credits all its rows to the sample of its first row."""
    M, N, T = 256, 64, 64
    Y = np.ones((M, N), np.int32)
    got = oracle.gn_stats_fused(Y, M, N, T, 0, 0, 0, 0, tile=(128, 64))
    per_group = 2     # 64 columns / 32 groups
    np.testing.assert_array_equal(got["sum"].reshape(4, 32)[:, 0], [128 * per_group, 0, 128 * per_group, 0])
    np.testing.assert_array_equal(got["mn"].reshape(4, 32)[:, 0], [1, INT_MAX, 1, INT_MAX])


@pytest.mark.parametrize("M,N,T", [(192, 128, 64), (300, 1280, 100), (512, 320, 256), (64, 32, 32)])
def test_gn_blocks_against_regions(M, N, T):
    """k_epilogue's per-1024-element blocks, with saturated groups planted inside one block."""
    r = np.random.default_rng(M + 3 * N)
    Y = _y(r, M, N, 24)
    flat = Y.reshape(-1)
    cg = N // 32
    for e in range(1024, min(2048, M * N)):      # block 1: group 0 elements saturated
        if (e % N) // cg == 0:
            flat[e] = INT_MAX
    got = oracle.gn_stats_planar(Y, M, N, T)
    _check(got, _gn_regions(Y, M, N, T, _block_regions(M, N, T)))


def test_gn_blocks_drop_saturated_block():
    """N = 1024: each block is one row. Row 1 all INT_MAX adds nothing; row 0 adds everything."""
    M, N, T = 4, 1024, 4
    Y = np.zeros((M, N), np.int32)
    Y[1] = INT_MAX
    Y[2, :] = 5
    got = oracle.gn_stats_planar(Y, M, N, T)
    np.testing.assert_array_equal(got["sum"], np.full(32, 5 * 32))
    np.testing.assert_array_equal(got["mn"], np.zeros(32))
    np.testing.assert_array_equal(got["mx"], np.full(32, 5))


def _round_half_up(y, e):
    """floor(y / 2^e + 1/2) exactly, by integer floor division."""
    y = y.astype(np.int64)
    return np.where(e == 0, y, np.floor_divide(2 * y + (np.int64(1) << e), np.int64(2) << e))


@pytest.mark.parametrize("heads,T,B", [(1, 64, 2), (5, 77, 2), (2, 130, 3)])
def test_qkv_heads_invariants(heads, T, B):
    C = 64 * heads
    M = B * T
    TpQ, TpK = -(-T // 128) * 128, -(-T // 64) * 64
    r = np.random.default_rng(heads * 100 + T)
    Y = _y(r, M, 3 * C, 31)
    Y[0, :64] = 0                          # e = 0 and all-zero bytes
    Y[1, :C] = -(2**31)                    # the largest magnitude: e = 17
    Y[2, C:C + 64] = 2**31 - 1
    Y[3, :64] = np.arange(64) - 32         # small: e = 0
    Y[4, :64] = (1 << 15)                  # exactly 2^15: e = 1
    Y[5, :64] = (1 << 15) - 1              # just below: e = 0
    out = oracle.qkv_heads(Y, M, C, heads, T, TpQ, TpK)
    np.testing.assert_array_equal(out["v"], Y[:, 2 * C:])
    for part, Tp in (("q", TpQ), ("k", TpK)):
        hi, lo, e, hs, ls, ts = out[part]
        yy = Y[:, (0 if part == "q" else C):(C if part == "q" else 2 * C)].astype(np.int64)
        yh = yy.reshape(B, T, heads, 64).transpose(0, 2, 1, 3)            # [b, head, t, d]
        rows = hi.reshape(B, heads, Tp, 64)
        live = (slice(None), slice(None), slice(0, T))
        H = rows[live].astype(np.int64)
        L = lo.reshape(B, heads, Tp, 64)[live].astype(np.int64)
        E = e.reshape(B, heads, Tp)[live].astype(np.int64)
        q = 256 * H + L + 128
        m = np.abs(yh).max(-1)
        # e: smallest shift with m < 2^(15+e), capped at 17 (row_exp counts k = 15..31)
        assert np.all(m < (np.int64(1) << (15 + E)))
        assert np.all((E == 0) | (m >= (np.int64(1) << (14 + E))))
        assert E.max() <= 17
        want_q = np.clip(_round_half_up(yh, E[..., None]), -32767, 32767)
        np.testing.assert_array_equal(q, want_q)
        np.testing.assert_array_equal(hs.reshape(B, heads, Tp)[live], H.sum(-1))
        np.testing.assert_array_equal(ls.reshape(B, heads, Tp)[live], L.sum(-1))
        np.testing.assert_array_equal(ts.reshape(B, heads, Tp)[live], q.sum(-1))
        # rows t >= T keep the fill
        pad = (slice(None), slice(None), slice(T, Tp))
        assert np.all(hi.reshape(B, heads, Tp, 64)[pad] == np.int8(0x5A))
        assert np.all(e.reshape(B, heads, Tp)[pad] == 0x5A5A5A5A)
    # the planted rows
    qh, ql, qe = out["q"][0], out["q"][1], out["q"][2]
    assert qe[0] == 0 and np.all(qh[0] == 0) and np.all(ql[0] == -128)
    assert qe[1] == 17 and np.all(256 * qh[1].astype(int) + ql[1] + 128 == -16384)
    assert qe[3] == 0 and qe[4] == 1 and qe[5] == 0
    ke = out["k"][2]
    assert ke[2] == 16                      # 2^31 - 1 < 2^31

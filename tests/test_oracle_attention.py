"""Pins of the oracle's attention (oracle/oracle.c: orc_quant_heads, orc_quant_v, orc_attention;
src/kernels.cu:611-672,799-805, src/attn.cu:1-6): the operand producers against their definitions
(row_exp, quant16 and the hi/lo split, pinned elsewhere), the score decomposition against int64 dot
products on the reference's own edge values (src/test_attn_score.cu:14-24), and the attention
against closed forms -- a single key (P clamps to 32767), identical keys (equal P from one
reciprocal), two keys a known score apart (the shift's direction and rounding), causal rows -- and
against the invariance under a permutation of the keys."""
import numpy as np
import pytest

import oracle
from tests import refmath as rm

EDGES = [-32767, -32766, -32513, -256, -255, -128, -1, 0, 1, 127, 128, 255, 256, 32512, 32766, 32767]   # src/test_attn_score.cu:14
L = oracle.exp_table()


def planes(qv):
    """int16 values [rows, 64] -> (hi, lo) planes."""
    return rm.split(np.asarray(qv, np.int64))


def test_score_split_identity():
    """S = Q.K = 65536 Shh + 256 (Shl + Slh) + Sll + 32768 qhs + 128 qls + 128 ksum on signed planes,
    the middle term inside int32 (src/test_attn_score.cu:14-24, 256 edge pairs and random rows)."""
    r = np.random.default_rng(12089)
    for test in range(256 + 400):
        if test < 256:
            q = np.full(64, EDGES[test // 16], np.int64)
            k = np.full(64, EDGES[test % 16], np.int64)
        else:
            q = r.integers(-32767, 32768, 64)
            k = r.integers(-32767, 32768, 64)
        qh, ql = (x.astype(np.int64) for x in planes(q))
        kh, kl = (x.astype(np.int64) for x in planes(k))
        hh, hl, lh, ll = (qh * kh).sum(), (qh * kl).sum(), (ql * kh).sum(), (ql * kl).sum()
        t = 256 * (hl + lh) + ll + 32768 * qh.sum() + 128 * ql.sum() + 128 * k.sum()
        assert -(2**31) <= t < 2**31
        assert 65536 * hh + t == int(q @ k)


@pytest.mark.parametrize("T,Tp", [(5, 8), (64, 64), (77, 128)])
def test_quant_heads_definition(T, Tp):
    r = np.random.default_rng(T)
    B, heads, C = 2, 3, 256
    X = r.integers(-(2**31), 2**31, (B * T, C), dtype=np.int64).astype(np.int32)
    X[0, :64] = 0
    X[1, 64:128] = r.integers(-20000, 20000, 64)
    hi, lo, e, hs, ls, ts = oracle.quant_heads(X, B, T, C, heads, Tp)
    for g in range(B * heads):
        b, h = divmod(g, heads)
        for t in range(Tp):
            w = g * Tp + t
            if t >= T:
                assert (hi[w] == 0).all() and (lo[w] == -128).all() and e[w] == 0 and hs[w] == 0 and ls[w] == -8192 and ts[w] == 0
                continue
            x = X[b * T + t, h * 64:(h + 1) * 64].astype(np.int64)
            ee = rm.row_exp(int(np.abs(x).max()))
            q = np.array([rm.quant16(int(v), ee) for v in x])
            qh, ql = planes(q)
            assert e[w] == ee and (hi[w] == qh).all() and (lo[w] == ql).all()
            assert hs[w] == qh.astype(np.int64).sum() and ls[w] == ql.astype(np.int64).sum() and ts[w] == q.sum()


@pytest.mark.parametrize("T,Tp", [(5, 8), (77, 128), (64, 64), (1, 64)])
def test_quant_heads_pad_definition(T, Tp):
    """orc_quant_heads_pad (src/kernels.cu:799-805): rows t >= T of every group become the operand of
    the value 0 -- the hi/lo split of 0 (pinned with split16), e 0, hs and ls the sums of those planes,
    tsum the sum of the quantised zeros -- equal to the pad rows orc_quant_heads writes; rows t < T are
    not touched."""
    r = np.random.default_rng(T * 131 + Tp)
    G = 5
    bufs = [r.integers(-128, 128, (G * Tp, 64)).astype(np.int8), r.integers(-128, 128, (G * Tp, 64)).astype(np.int8),
            r.integers(-1000, 1000, G * Tp).astype(np.int32)] + [r.integers(-(1 << 40), 1 << 40, G * Tp) for _ in range(3)]
    before = [b.copy() for b in bufs]
    oracle.quant_heads_pad(G, T, Tp, *bufs)
    zh, zl = (x.astype(np.int64) for x in planes(np.zeros(64, np.int64)))
    assert (zh == 0).all() and (zl == -128).all()
    X = r.integers(-(2**31), 2**31, (G * T, 64), dtype=np.int64).astype(np.int32)
    ref = oracle.quant_heads(X, G, T, 64, 1, Tp)
    for g in range(G):
        for t in range(Tp):
            w = g * Tp + t
            if t < T:
                assert all(np.array_equal(a[w], b[w]) for a, b in zip(bufs, before))
                continue
            assert (bufs[0][w] == zh).all() and (bufs[1][w] == zl).all()
            assert bufs[2][w] == 0 and bufs[3][w] == zh.sum() == 0 and bufs[4][w] == zl.sum() == -8192 and bufs[5][w] == 0
            assert all(np.array_equal(a[w], b[w]) for a, b in zip(bufs, ref))


def test_quant_v_definition():
    r = np.random.default_rng(3)
    B, heads, C, Tk, Tkp = 2, 2, 128, 77, 128
    X = r.integers(-(2**31), 2**31, (B * Tk, C), dtype=np.int64).astype(np.int32)
    X[:, 5] = r.integers(-1000, 1000, B * Tk)
    vth, vtl, ev, vs = oracle.quant_v(X, B, Tk, C, heads, Tkp)
    for g in range(B * heads):
        b, h = divmod(g, heads)
        for d in range(64):
            col = X[b * Tk:(b + 1) * Tk, h * 64 + d].astype(np.int64)
            ee = rm.row_exp(int(np.abs(col).max()))
            q = np.array([rm.quant16(int(v), ee) for v in col] + [0] * (Tkp - Tk))
            qh, ql = planes(q)
            assert ev[g * 64 + d] == ee and vs[g * 64 + d] == q.sum()
            assert (vth[g * 64 + d] == qh).all() and (vtl[g * 64 + d] == ql).all()


def operands(r, B, heads, Tq, Tqp, Tk, Tkp, C, q_scale=3000, k_scale=3000, v_scale=30000):
    Xq = r.normal(0, q_scale, (B * Tq, C)).astype(np.int32)
    Xk = r.normal(0, k_scale, (B * Tk, C)).astype(np.int32)
    Xv = r.normal(0, v_scale, (B * Tk, C)).astype(np.int32)
    q = oracle.quant_heads(Xq, B, Tq, C, heads, Tqp)
    k = oracle.quant_heads(Xk, B, Tk, C, heads, Tkp)
    v = oracle.quant_v(Xv, B, Tk, C, heads, Tkp)
    return q, k, v


def run(q, k, v, B, heads, Tq, Tqp, Tk, Tkp, C, causal=False, rowmax=None):
    return oracle.attention(q[0], q[1], q[2], k[0], k[1], k[2], v[0], v[1], v[2], B, heads, Tq, Tqp, Tk, Tkp, causal, L, C, rowmax=rowmax)


def vvals(v, g, Tkp):
    """int16 values of V [64 dims x Tkp keys] of group g."""
    return 256 * v[0][g * 64:(g + 1) * 64].astype(np.int64) + v[1][g * 64:(g + 1) * 64] + 128


def test_single_key():
    """One key: E = L[0] = 2^30, r = 2^32, P = (2^62 + 2^46) >> 47 = 32768, clamped to 32767."""
    r = np.random.default_rng(1)
    B, heads, C, Tq, Tk, Tkp = 1, 2, 128, 3, 1, 64
    q, k, v = operands(r, B, heads, Tq, 64, Tk, Tkp, C)
    out = run(q, k, v, B, heads, Tq, 64, Tk, Tkp, C)
    assert L[0] == 2**30
    for g in range(heads):
        V = vvals(v, g, Tkp)
        for qq in range(Tq):
            want = [rm.rshr(32767 * int(V[d, 0]), 15 - int(v[2][g * 64 + d])) for d in range(64)]
            assert list(out[qq, g * 64:(g + 1) * 64]) == want


def test_identical_keys():
    """Identical keys: every E = L[0], r = floor(2^62 / (Tk L[0])), every P = (L[0] r + 2^46) >> 47."""
    r = np.random.default_rng(2)
    B, heads, C, Tq, Tk, Tkp = 1, 1, 64, 4, 77, 128
    q, k, v = operands(r, B, heads, Tq, 64, Tk, Tkp, C)
    for arr in (k[0], k[1]):
        arr[1:Tk] = arr[0]
    k[2][1:Tk] = k[2][0]
    out = run(q, k, v, B, heads, Tq, 64, Tk, Tkp, C)
    rr = (1 << 62) // (Tk * int(L[0]))
    P = min(32767, (int(L[0]) * rr + (1 << 46)) >> 47)
    V = vvals(v, 0, Tkp)
    want = [rm.rshr(P * int(V[d, :Tk].sum()), 15 - int(v[2][d])) for d in range(64)]
    for qq in range(Tq):
        assert list(out[qq]) == want


@pytest.mark.parametrize("eq,ek", [(0, 0), (3, 2), (12, 9), (17, 17)])
def test_two_keys_score_shift(eq, ek):
    """Q = (a, 0, ...), K_i = (b_i, 0, ...): S_i = a b_i, s_i = rshr(S_i, 19 - eq - ek) (saturated),
    E_i = lutexp(mx - s_i), and P, O from their definitions."""
    a, b1, b2 = 20000, 30000, 29000
    Tkp, C = 64, 64
    qv = np.zeros((64, 64), np.int64); qv[0, 0] = a
    kv = np.zeros((Tkp, 64), np.int64); kv[0, 0] = b1; kv[1, 0] = b2
    qh, ql = planes(qv); kh, kl = planes(kv)
    eqa = np.full(64, eq, np.int32); eka = np.full(Tkp, ek, np.int32)
    r = np.random.default_rng(eq * 31 + ek)
    vv = np.zeros((64, Tkp), np.int64); vv[:, :2] = r.integers(-32767, 32768, (64, 2))
    vth, vtl = planes(vv)
    ev = r.integers(0, 18, 64).astype(np.int32)
    out = oracle.attention(qh, ql, eqa, kh, kl, eka, vth, vtl, ev, 1, 1, 1, 64, 2, Tkp, False, L, C)
    s = [rm.rshr(a * b, 19 - eq - ek) for b in (b1, b2)]
    mx = max(s)

    def lutexp(z):
        if z >= 1 << 20:
            return 0
        i, f = z >> 10, z & 1023
        return int(L[i]) + (((int(L[i + 1]) - int(L[i])) * f) >> 10)

    E = [lutexp((mx - x) & 0xFFFFFFFF) for x in s]
    rr = (1 << 62) // sum(E)
    P = [min(32767, ((x * rr + (1 << 46)) & (2**64 - 1)) >> 47) if x > 0 else 0 for x in E]
    want = [rm.rshr(P[0] * int(vv[d, 0]) + P[1] * int(vv[d, 1]), 15 - int(ev[d])) for d in range(64)]
    assert list(out[0]) == want


def test_causal_rows():
    """Causal: query 0 sees key 0 alone (the single-key form); every row equals the non-causal
    attention over its prefix of keys."""
    r = np.random.default_rng(4)
    B, heads, C, T, Tp = 1, 1, 64, 9, 64
    q, k, v = operands(r, B, heads, T, Tp, T, Tp, C)
    out = run(q, k, v, B, heads, T, Tp, T, Tp, C, causal=True)
    V = vvals(v, 0, Tp)
    assert list(out[0]) == [rm.rshr(32767 * int(V[d, 0]), 15 - int(v[2][d])) for d in range(64)]
    for qq in range(1, T):
        # the prefix problem: keys 0..qq only (Tk = qq + 1), rows of q moved to the front
        sub_q = tuple(x.copy() for x in q)
        for arr in sub_q:
            arr[0] = arr[qq]
        prefix = run(sub_q, k, v, B, heads, 1, Tp, qq + 1, Tp, C)
        assert (prefix[0] == out[qq]).all(), qq


def test_key_permutation_invariance():
    r = np.random.default_rng(5)
    B, heads, C, Tq, Tk, Tkp = 2, 2, 128, 7, 50, 64
    q, k, v = operands(r, B, heads, Tq, 64, Tk, Tkp, C)
    out = run(q, k, v, B, heads, Tq, 64, Tk, Tkp, C)
    perm = r.permutation(Tk)
    G = B * heads
    kp = tuple(x.copy() for x in k)
    vp = tuple(x.copy() for x in v)
    for g in range(G):
        for arr in kp[:3]:
            arr[g * Tkp:g * Tkp + Tk] = arr[g * Tkp + perm]
        for arr in vp[:2]:
            arr[g * 64:(g + 1) * 64, :Tk] = arr[g * 64:(g + 1) * 64, perm]
    assert (run(q, kp, vp, B, heads, Tq, 64, Tk, Tkp, C) == out).all()

"""GPU parity of the exact attention and its operand producers (vela_amd.attention over the C ABI)
against the oracle (orc_quant_heads, orc_quant_v, orc_attention): the producers on padded and
unpadded rows, the attention on self- and cross-attention shapes (Tq and Tk below their padded
sizes, several groups), causal masking, the reference's edge operand values with every score
shift from -15 to 19, saturating scores, the row maxima, and the chain from the QKV GEMM epilogue
(q/k head planes) and its v output through k_quant_v into the attention."""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_equal, to_np
from vela_amd import attention as va

pytestmark = pytest.mark.gpu

EDGES = [-32767, -32766, -32513, -256, -255, -128, -1, 0, 1, 127, 128, 255, 256, 32512, 32766, 32767]
L = oracle.exp_table()


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def gpu_heads(X, B, T, C, heads, Tp):
    G = B * heads
    hi = torch.full((G * Tp, 64), 0x5a, dtype=torch.int8, device="cuda")
    lo = torch.full_like(hi, 0x5a)
    e = torch.full((G * Tp,), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
    hs = torch.full((G * Tp,), 7, dtype=torch.int64, device="cuda")
    ls, ts = hs.clone(), hs.clone()
    va.k_quant_heads(dev(X), B, T, C, heads, Tp, hi, lo, e, hs, ls, ts)
    return hi, lo, e, hs, ls, ts


def gpu_v(X, B, Tk, C, heads, Tkp):
    G = B * heads
    vth = torch.full((G * 64, Tkp), 0x5a, dtype=torch.int8, device="cuda")
    vtl = torch.full_like(vth, 0x5a)
    ev = torch.full((G * 64,), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
    vs = torch.full((G * 64,), 7, dtype=torch.int64, device="cuda")
    va.k_quant_v(dev(X), B, Tk, C, heads, Tkp, vth, vtl, ev, vs)
    return vth, vtl, ev, vs


@pytest.mark.parametrize("T,Tp", [(5, 64), (77, 128), (256, 256)])
def test_quant_heads_and_v(gpu, T, Tp):
    r = np.random.default_rng(T)
    B, heads, C = 2, 5, 320
    X = r.integers(-(2**31), 2**31, (B * T, C), dtype=np.int64).astype(np.int32)
    X[0, :64] = 0
    X[1:3, 64:128] = r.integers(-3000, 3000, (2, 64))
    got = gpu_heads(X, B, T, C, heads, Tp)
    torch.cuda.synchronize()
    for gt, w, n in zip(got, oracle.quant_heads(X, B, T, C, heads, Tp), ("hi", "lo", "e", "hs", "ls", "tsum")):
        assert_equal(to_np(gt), w, f"quant_heads T={T} {n}")
    got = gpu_v(X, B, T, C, heads, Tp)
    torch.cuda.synchronize()
    for gt, w, n in zip(got, oracle.quant_v(X, B, T, C, heads, Tp), ("vthi", "vtlo", "ev", "vsum")):
        assert_equal(to_np(gt), w, f"quant_v T={T} {n}")


def test_quant_heads_pad(gpu):
    G, T, Tp = 6, 70, 128
    arrs = [torch.full((G * Tp, 64), 9, dtype=torch.int8, device="cuda") for _ in range(2)]
    e = torch.full((G * Tp,), 5, dtype=torch.int32, device="cuda")
    sums = [torch.full((G * Tp,), 3, dtype=torch.int64, device="cuda") for _ in range(3)]
    va.k_quant_heads_pad(G, T, Tp, arrs[0], arrs[1], e, *sums)
    torch.cuda.synchronize()
    want = [np.full((G * Tp, 64), 9, np.int8), np.full((G * Tp, 64), 9, np.int8), np.full(G * Tp, 5, np.int32)] + \
           [np.full(G * Tp, 3, np.int64) for _ in range(3)]
    oracle.quant_heads_pad(G, T, Tp, *want)
    for gt, w in zip(arrs + [e] + sums, want):
        assert_equal(to_np(gt), w, "quant_heads_pad")


def attend(q, k, v, B, heads, Tq, Tqp, Tk, Tkp, C, causal=False, rowmax=False):
    out = torch.full((B * Tq, C), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
    rm = torch.zeros(B * Tq, dtype=torch.int32, device="cuda") if rowmax else None
    qd = [x if isinstance(x, torch.Tensor) else dev(x) for x in q]
    kd = [x if isinstance(x, torch.Tensor) else dev(x) for x in k]
    vd = [x if isinstance(x, torch.Tensor) else dev(x) for x in v]
    va.k_fused_attention(qd[0], qd[1], qd[2], qd[3], qd[4], kd[0], kd[1], kd[2], kd[5], vd[0], vd[1], vd[2], vd[3], B, heads, Tq, Tqp, Tk, Tkp,
                         causal, dev(L), C, None, None, out, rm)
    torch.cuda.synchronize()
    return to_np(out), (to_np(rm).view(np.uint32) if rowmax else None)


def host(x):
    return [to_np(t) if isinstance(t, torch.Tensor) else t for t in x]


def check(q, k, v, B, heads, Tq, Tqp, Tk, Tkp, C, causal=False, what=""):
    got, grm = attend(q, k, v, B, heads, Tq, Tqp, Tk, Tkp, C, causal, rowmax=True)
    qh, kh, vh = host(q), host(k), host(v)
    wrm = np.zeros(B * Tq, np.uint32)
    want = oracle.attention(qh[0], qh[1], qh[2], kh[0], kh[1], kh[2], vh[0], vh[1], vh[2], B, heads, Tq, Tqp, Tk, Tkp, causal, L, C, rowmax=wrm)
    # columns of heads the call does not own stay as they were
    assert_equal(got[:, :heads * 64], want[:, :heads * 64], f"{what} out")
    assert_equal(grm, wrm, f"{what} rowmax")


@pytest.mark.parametrize("B,heads,Tq,Tk,causal", [(1, 1, 64, 64, False), (2, 5, 100, 77, False), (1, 2, 256, 300, False), (2, 3, 70, 70, True),
                                                  (1, 10, 128, 128, True), (8, 2, 33, 7, False)])
def test_attention_shapes(gpu, B, heads, Tq, Tk, causal):
    r = np.random.default_rng(Tq * 7 + Tk)
    C = heads * 64
    Tqp, Tkp = (Tq + 63) // 64 * 64, (Tk + 63) // 64 * 64
    Xq = r.normal(0, 3000, (B * Tq, C)).astype(np.int32)
    Xk = r.normal(0, 3000, (B * Tk, C)).astype(np.int32)
    Xv = r.normal(0, 30000, (B * Tk, C)).astype(np.int32)
    q = gpu_heads(Xq, B, Tq, C, heads, Tqp)
    k = gpu_heads(Xk, B, Tk, C, heads, Tkp)
    v = gpu_v(Xv, B, Tk, C, heads, Tkp)
    check(q, k, v, B, heads, Tq, Tqp, Tk, Tkp, C, causal, what=f"B{B} h{heads} {Tq}x{Tk} c{int(causal)}")


def test_attention_wide_scores(gpu):
    """Large activations (e up to 17 on both sides) and unit ones (e = 0): score shifts from -15 to
    19, saturated scores included."""
    r = np.random.default_rng(9)
    B, heads, T = 1, 4, 128
    C = heads * 64
    Xq = r.integers(-(2**31), 2**31, (B * T, C), dtype=np.int64).astype(np.int32)
    Xk = r.integers(-(2**31), 2**31, (B * T, C), dtype=np.int64).astype(np.int32)
    Xq[::3] = r.integers(-2, 3, (len(Xq[::3]), C))
    Xk[1::4] = r.integers(-40000, 40000, (len(Xk[1::4]), C))
    Xv = r.integers(-(2**31), 2**31, (B * T, C), dtype=np.int64).astype(np.int32)
    q = gpu_heads(Xq, B, T, C, heads, T)
    k = gpu_heads(Xk, B, T, C, heads, T)
    v = gpu_v(Xv, B, T, C, heads, T)
    check(q, k, v, B, heads, T, T, T, T, C, what="wide")


def test_attention_edge_operands(gpu):
    """Q and K rows made of the reference's edge values (src/test_attn_score.cu:14), each row one
    value, with eq and ek spanning 0..17 (score shifts 19 - eq - ek from -15 to 19)."""
    from tests import refmath as rm
    G, T = 1, 64
    qv = np.repeat(np.array(EDGES * 4, np.int64)[:, None], 64, axis=1)[:T]
    kv = np.repeat(np.array(EDGES[::-1] * 4, np.int64)[:, None], 64, axis=1)[:T]
    qh, ql = rm.split(qv)
    kh, kl = rm.split(kv)
    eq = (np.arange(T) % 18).astype(np.int32)
    ek = ((np.arange(T) * 7) % 18).astype(np.int32)
    qs = [qh, ql, eq, qh.astype(np.int64).sum(1), ql.astype(np.int64).sum(1)]
    ks = [kh, kl, ek, kh.astype(np.int64).sum(1), kl.astype(np.int64).sum(1), kv.sum(1)]
    r = np.random.default_rng(11)
    vv = r.integers(-32767, 32768, (64, T))
    vth, vtl = rm.split(vv)
    vs = [vth, vtl, r.integers(0, 18, 64).astype(np.int32), vv.sum(1)]
    check(qs, ks, vs, G, 1, T, T, T, T, 64, what="edges")


def test_attention_errors(gpu):
    from vela_amd._lib import VgemmError
    z8 = torch.zeros((64, 64), dtype=torch.int8, device="cuda")
    z32 = torch.zeros(64, dtype=torch.int32, device="cuda")
    z64 = torch.zeros(64, dtype=torch.int64, device="cuda")
    out = torch.zeros((64, 64), dtype=torch.int32, device="cuda")
    with pytest.raises(VgemmError, match="Tqp/Tkp alignment"):
        va.k_fused_attention(z8, z8, z32, z64, z64, z8, z8, z32, z64, z8, z8, z32, z64, 1, 1, 60, 60, 64, 64, False, dev(L), 64, None, None, out)


def test_qkv_gemm_chain(gpu):
    """The fused QKV projection (EPI_QKV: q and k head planes, v as int32), the pad rows by
    k_quant_heads_pad, k_quant_v on v, then the attention on the planes the GEMM wrote."""
    from tests.test_gpu_gemm import Case
    from tests.test_gpu_qkv_gn import run_qkv
    from vela_amd import gemm as vg
    heads, T, B = 2, 70, 2
    C, TpQ, TpK = 64 * heads, 128, 128
    c = Case(vg.SRC_I16, B * T, 3 * C, 320, seed=21)
    got = run_qkv(c, heads, T, TpQ, TpK)
    q = [dev(x) for x in got["q"]]
    k = [dev(x) for x in got["k"]]
    va.k_quant_heads_pad(B * heads, T, TpQ, *q)   # the QKV epilogue leaves rows t >= T to the caller (src/engine.cu:329-330)
    va.k_quant_heads_pad(B * heads, T, TpK, *k)
    v = gpu_v(got["v"], B, T, C, heads, TpK)
    check(q, k, v, B, heads, T, TpQ, T, TpK, C, what="qkv chain")

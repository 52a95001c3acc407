"""GPU parity of the A-operand producers, the planar-path epilogues, the Gemm::run replacement and
graph capture, each against the CPU oracle.

The im2col cases are the grid of the reference's independent oracle test src/test_im2col.cu:13-20
(B=2, H=5, W=7, C in {4..2560}, stride 1/2, zero / 16-bit / full-int32 data with INT_MIN/INT_MAX
every 19th value), compared on every output byte, shift and pad row.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_equal, to_np
from vela_amd import configs as cf
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def im2col_data(r, n, mode):
    if mode == 0:
        x = np.zeros(n, np.int32)
    elif mode == 1:
        x = (r.integers(0, 65537, n) - 32768).astype(np.int32)
    else:
        x = r.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32).view(np.int32)
        idx = np.arange(n)
        sel = idx % 19 == 0
        x[sel] = np.where(idx[sel] & 1, np.iinfo(np.int32).min, np.iinfo(np.int32).max)
    return x


@pytest.mark.parametrize("C", [4, 12, 16, 32, 320, 640, 960, 1280, 1920, 2560])
def test_pixmax_im2col3_conv_e(gpu, C):
    r = np.random.default_rng(20261021 + C)
    B, H, W = 2, 5, 7
    for stride in (1, 2):
        for mode in (0, 1, 2):
            Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
            rows = B * Ho * Wo
            Mp = (rows + 31) // 32 * 32
            Kp = cf.align(9 * C, 16)
            x = im2col_data(r, B * H * W * C, mode)
            pm_w = oracle.pixmax(x, B * H * W, C)
            hi_w, lo_w, e_w = oracle.im2col3(x, pm_w, B, H, W, C, stride, Kp)
            dx = dev(x)
            pm = torch.zeros(B * H * W, dtype=torch.int32, device="cuda")
            hi = torch.full((Mp, Kp), 0x5A, dtype=torch.int8, device="cuda")
            lo = torch.full((Mp, Kp), 0x5A, dtype=torch.int8, device="cuda")
            e = torch.zeros(Mp, dtype=torch.int32, device="cuda")
            e2 = torch.zeros(rows, dtype=torch.int32, device="cuda")
            vg.k_pixmax(dx, B * H * W, C, pm)
            vg.k_im2col3(dx, pm, B, H, W, C, stride, hi, lo, e, Kp)
            vg.k_conv_e(pm, B, H, W, stride, e2)
            torch.cuda.synchronize()
            what = f"C={C} stride={stride} mode={mode}"
            assert_equal(to_np(pm).view(np.uint32), pm_w, what + " pm")
            assert_equal(to_np(hi), hi_w, what + " hi")
            assert_equal(to_np(lo), lo_w, what + " lo")
            assert_equal(to_np(e)[:rows], e_w[:rows], what + " e")
            assert_equal(to_np(e2), oracle.conv_e(pm_w, B, H, W, stride), what + " conv_e")


@pytest.mark.parametrize("M,K,Kp", [(1, 4, 16), (77, 320, 320), (96, 1024, 1024), (33, 1280, 1296), (200, 36, 48)])
def test_quant_rows(gpu, M, K, Kp):
    r = np.random.default_rng(M * 7 + K)
    bits = r.integers(1, 32, (M, K))
    x = ((r.integers(0, 2**31, (M, K)) & ((1 << bits) - 1)) - (1 << (bits - 1))).astype(np.int32)
    x[0, 0] = np.iinfo(np.int32).min
    hi_w, lo_w, e_w = oracle.quant_rows(x, M, K, K, Kp)
    Mp = hi_w.shape[0]
    hi = torch.full((Mp, Kp), 0x33, dtype=torch.int8, device="cuda")
    lo = torch.full((Mp, Kp), 0x33, dtype=torch.int8, device="cuda")
    e = torch.zeros(Mp, dtype=torch.int32, device="cuda")
    vg.k_quant_rows(dev(x), M, K, K, hi, lo, e, Kp)
    torch.cuda.synchronize()
    assert_equal(to_np(hi), hi_w, "hi")
    assert_equal(to_np(lo), lo_w, "lo")
    assert_equal(to_np(e)[:M], e_w[:M], "e")


def _planes(r, M, N):
    Chi = r.integers(-(2**27), 2**27, (M, N)).astype(np.int32)
    Clo = r.integers(-(2**27), 2**27, (M, N)).astype(np.int32)
    return Chi, Clo


def _cst(r, N, s_lo=-4, s_hi=40):
    cst = np.zeros((N, 4), np.int32)
    cst[:, 0] = r.integers(-(2**20), 2**20, N)
    cst[:, 1] = r.integers(s_lo, s_hi, N)
    cst[:, 2] = r.integers(-50000, 50000, N)
    cst[:, 3] = r.integers(-(2**20), 2**20, N)
    return cst


def test_epilogue_and_split(gpu):
    r = np.random.default_rng(3)
    M, N = 300, 96
    Chi, Clo = _planes(r, M, N)
    cst = _cst(r, N)
    e = r.integers(0, 17, M).astype(np.int32)
    R = r.integers(-(2**31), 2**31, (M, N), dtype=np.int64).astype(np.int32)
    want = oracle.epilogue(Chi, Clo, M, N, N, cst, e, N, R)
    Y = dev(R)
    vg.k_epilogue(dev(Chi), dev(Clo), M, N, N, dev(cst), dev(e), Y, N, Y)
    Cs = 32
    Y0, Y1, Y2 = (torch.zeros((M, Cs), dtype=torch.int32, device="cuda") for _ in range(3))
    vg.k_epilogue_split(dev(Chi), dev(Clo), M, N, N, dev(cst), dev(e), Cs, Y0, Y1, Y2)
    torch.cuda.synchronize()
    assert_equal(to_np(Y), want, "epilogue")
    ws = oracle.epilogue_split(Chi, Clo, M, N, N, cst, e, Cs)
    for i, y in enumerate((Y0, Y1, Y2)):
        assert_equal(to_np(y), ws[i], f"split {i}")


def test_epilogue_geglu_q(gpu):
    r = np.random.default_rng(4)
    M, F = 130, 320
    Chi, Clo = _planes(r, M, 2 * F)
    Chi >>= 6
    Clo >>= 6
    cst = _cst(r, 2 * F, 8, 30)
    e = r.integers(0, 5, M).astype(np.int32)
    L = cf.phi_lut()
    Kp = 336
    hi_w, lo_w, eo_w = oracle.epilogue_geglu_q(Chi, Clo, M, F, 2 * F, cst, e, L, Kp)
    hi = torch.zeros((M, Kp), dtype=torch.int8, device="cuda")
    lo = torch.zeros((M, Kp), dtype=torch.int8, device="cuda")
    eo = torch.zeros(M, dtype=torch.int32, device="cuda")
    vg.k_epilogue_geglu_q(dev(Chi), dev(Clo), M, F, 2 * F, dev(cst), dev(e), dev(L), hi, lo, eo, Kp)
    torch.cuda.synchronize()
    assert_equal(to_np(hi), hi_w, "hi")
    assert_equal(to_np(lo), lo_w, "lo")
    assert_equal(to_np(eo), eo_w, "e")


@pytest.mark.parametrize("variant", [-1, 0, 1, 2, 3])
@pytest.mark.parametrize("M,N,K,batch", [(128, 128, 64, 1), (257, 100, 320, 1), (2 * 8192, 320, 16, 1), (77, 96, 64, 3)])
def test_i8gemm(gpu, variant, M, N, K, batch):
    """Gemm::run (src/gemm.cu:46-70): C = A * W^T, int32, strided batch."""
    vg.set_variant(variant)
    try:
        r = np.random.default_rng(M + N + K)
        lda, ldw, ldc = K + 16, K, N + 4
        sA, sW, sC = M * lda + 32, N * ldw + 16, M * ldc + 8
        A = r.integers(-128, 128, sA * batch).astype(np.int8)
        W = r.integers(-128, 128, sW * batch).astype(np.int8)
        want = oracle.i8gemm(A, W, M, N, K, batch, sA, sW, sC, lda, ldw, ldc)
        C = torch.zeros(max(sC * batch, M * ldc), dtype=torch.int32, device="cuda")
        g = vg.Gemm()
        g.init(32 << 20)
        g.run(dev(A), lda, sA, dev(W), ldw, sW, C, ldc, sC, M, N, K, batch)
        torch.cuda.synchronize()
        got = to_np(C)
        for b in range(batch):
            for m in range(M):
                o = b * sC + m * ldc
                assert_equal(got[o:o + N], want[o:o + N], f"batch {b} row {m}")
    finally:
        vg.set_variant(-1)


@pytest.mark.parametrize("M,N,K,ws,splits", [
    (1024, 1280, 11520, 32 << 20, 0),    # the 512-row C4 conv's stacked planes: split by the handle's workspace
    (300, 200, 4096, 32 << 20, 0),       # partial tiles in both dimensions
    (300, 200, 4096, 256 << 10, 0),      # a workspace too small for two K ranges: unsplit
    (256, 256, 2048, 32 << 20, 5),       # forced splits (uneven K ranges)
    (1024, 1280, 11520, 0, 0),           # no workspace: unsplit
])
def test_i8gemm_split_k(gpu, M, N, K, ws, splits):
    """Gemm::run on deep K with few tiles splits K into the handle's workspace (the reference's
    Gemm::init allocates it, src/gemm.cu:7-11) and sums the ranges: the same int32 C, rows and
    columns beyond M and N untouched (ldc > N)."""
    vg.set_splitk(splits)
    try:
        r = np.random.default_rng(M + N + K + splits)
        lda, ldw, ldc = K, K, N + 8
        A = r.integers(-128, 128, M * lda).astype(np.int8)
        W = r.integers(-128, 128, N * ldw).astype(np.int8)
        want = oracle.i8gemm(A, W, M, N, K, 1, 0, 0, 0, lda, ldw, ldc).reshape(M, ldc)
        C = torch.full((M + 2, ldc), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
        g = vg.Gemm()
        g.init(ws)
        for _ in range(2):   # the workspace holds the last call's partials: a repeat gives the same C
            g.run(dev(A), lda, 0, dev(W), ldw, 0, C, ldc, 0, M, N, K, 1)
        torch.cuda.synchronize()
        got = to_np(C)
        assert_equal(got[:M, :N], want[:, :N], f"split-K Gemm::run {M}x{N}x{K} ws {ws} splits {splits}")
        assert (got[:M, N:] == 0x5A5A5A5A).all() and (got[M:] == 0x5A5A5A5A).all(), "writes outside C"
    finally:
        vg.set_splitk(0)


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("M,N,K,batch", [(257, 100, 320, 1), (77, 96, 64, 3), (192, 1280, 1024, 2)])
def test_i8gemm_tile_orders(gpu, order, M, N, K, batch):
    """Gemm::run under each forced tile order over the XCDs, with strided batches."""
    vg.set_tile_order(order)
    try:
        r = np.random.default_rng(7 * M + N + K)
        lda, ldw, ldc = K, K + 32, N
        sA, sW, sC = M * lda + 16, N * ldw, M * ldc + 12
        A = r.integers(-128, 128, sA * batch).astype(np.int8)
        W = r.integers(-128, 128, sW * batch).astype(np.int8)
        want = oracle.i8gemm(A, W, M, N, K, batch, sA, sW, sC, lda, ldw, ldc)
        C = torch.zeros(max(sC * batch, M * ldc), dtype=torch.int32, device="cuda")
        g = vg.Gemm()
        g.init(0)
        g.run(dev(A), lda, sA, dev(W), ldw, sW, C, ldc, sC, M, N, K, batch)
        torch.cuda.synchronize()
        got = to_np(C)
        for b in range(batch):
            rows = got[b * sC: b * sC + M * ldc].reshape(M, ldc)[:, :N]
            wrows = want[b * sC: b * sC + M * ldc].reshape(M, ldc)[:, :N]
            assert_equal(rows, wrows, f"order {order} batch {b}")
    finally:
        vg.set_tile_order(-1)


def test_graph_replays_match_eager(gpu):
    """A captured sequence of GEMMs (with kernel-zeroed rowmax buffers) replayed several times, with
    eager work and synchronisations between replays, reproduces the eager results every time."""
    layers = [cf.Layer("g1", "linear", 512, 320, 640, seed=101), cf.Layer("g2", "linear", 384, 640, 1280, epi=cf.EPI_GEGLU, rowmax=True, seed=102),
              cf.Layer("g3", "conv", 2 * 16 * 16, 9 * 64, 128, B=2, H=16, W=16, C=64, residual=True, seed=103)]
    probs = [cf.DeviceProblem(L) for L in layers]
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        for p in probs:
            p.reset()
            p.run(stream=side)
    side.synchronize()
    eager = [(to_np(p.y).copy(), None if p.rowmax is None else to_np(p.rowmax).copy()) for p in probs]
    for (y, rm), p in zip(eager, probs):
        want, wrm = oracle.layer_reference(p.L, p.h)
        assert_equal(y, want, p.L.name)
        if wrm is not None:
            assert_equal(rm.view(np.uint32), wrm, p.L.name + " rowmax")
    graph = vg.Graph(side)
    with torch.cuda.stream(side):   # torch's copy_ and the rowmax fills must go to the captured stream
        graph.begin()
        for p in probs:
            p.reset()
            p.run(stream=side)
        graph.end()
    for rep in range(3):
        for p in probs:
            p.y.fill_(7)
        torch.cuda.synchronize()
        graph.replay()
        side.synchronize()
        for (y, rm), p in zip(eager, probs):
            assert_equal(to_np(p.y), y, f"replay {rep} {p.L.name}")
            if rm is not None:
                assert_equal(to_np(p.rowmax), rm, f"replay {rep} {p.L.name} rowmax")
    graph.destroy()

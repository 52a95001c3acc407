"""Seeded random GPU parity cases of the planar-path entry points against the CPU oracle, byte for byte.

k_quant_rows, k_pixmax + k_im2col3 + k_conv_e, k_epilogue (with and without a residual and GroupNorm
statistics), k_epilogue_split, k_epilogue_geglu_q (src/kernels.h:12-25, 68-70) and Gemm::run
(src/gemm.h:12-19) each draw shapes, leading dimensions and value ranges at random within what the
call accepts, so that combinations the structured tests do not list are also checked. Outputs start
filled with 0x5A bytes, so a byte the kernel should write and does not, or writes outside its rows
and columns, shows up. Each case prints its parameters before it runs.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_equal, to_np
from vela_amd import configs as cf
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu

FILL8 = 0x5A
FILL32 = 0x5A5A5A5A
INT_MIN, INT_MAX = -(2**31), 2**31 - 1


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def filled(shape, dtype):
    if dtype == torch.int8:
        return torch.full(shape, FILL8, dtype=torch.int8, device="cuda")
    return torch.full(shape, FILL32, dtype=torch.int32, device="cuda")


def ints(r, shape):
    """int32 values with a random bit width per element (zero rows and both extremes now and then)."""
    bits = r.integers(1, 33, shape)
    x = r.integers(0, 2**32, shape, dtype=np.uint64).astype(np.int64)
    x = (x & ((np.int64(1) << bits) - 1)) - (np.int64(1) << (bits - 1))
    x = x.astype(np.int32)
    flat = x.reshape(-1)
    if flat.size and r.integers(2):
        flat[r.integers(flat.size, size=1 + flat.size // 97)] = r.choice([INT_MIN, INT_MAX])
    if x.ndim == 2 and x.shape[0] > 1 and r.integers(3) == 0:
        x[r.integers(x.shape[0])] = 0
    return x


def log(kind, seed, **kw):
    print(f"[random {kind}] seed {seed}: " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.mark.parametrize("seed", range(24))
def test_random_quant_rows(seed):
    r = np.random.default_rng(40_000 + seed)
    M, K = int(r.integers(1, 400)), int(r.integers(1, 3000))
    Kp = K + int(r.integers(0, 64))
    Kp = (Kp + 3) // 4 * 4
    ldx = K + int(r.integers(0, 40))
    log("quant_rows", seed, M=M, K=K, ldx=ldx, Kp=Kp)
    x = ints(r, (M, ldx))
    hi_w, lo_w, e_w = oracle.quant_rows(x, M, K, ldx, Kp)
    Mp = hi_w.shape[0]
    hi, lo, e = filled((Mp, Kp), torch.int8), filled((Mp, Kp), torch.int8), filled((Mp,), torch.int32)
    vg.k_quant_rows(dev(x), M, K, ldx, hi, lo, e, Kp)
    torch.cuda.synchronize()
    assert_equal(to_np(hi), hi_w, "hi")
    assert_equal(to_np(lo), lo_w, "lo")
    assert_equal(to_np(e)[:M], e_w[:M], "e")
    assert (to_np(e)[M:] == np.int32(FILL32)).all(), "e of a pad row was written"


@pytest.mark.parametrize("seed", range(24))
def test_random_im2col3(seed):
    r = np.random.default_rng(41_000 + seed)
    B, H, W = int(r.integers(1, 4)), int(r.integers(1, 24)), int(r.integers(1, 24))
    C = 4 * int(r.integers(1, 100))
    stride = int(r.choice([1, 2, 3]))
    Kp = cf.align(9 * C, 4) + 4 * int(r.integers(0, 12))
    Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
    rows = B * Ho * Wo
    Mp = (rows + 31) // 32 * 32
    log("im2col3", seed, B=B, H=H, W=W, C=C, stride=stride, Kp=Kp)
    x = ints(r, (B * H * W, C))
    pm_w = oracle.pixmax(x, B * H * W, C)
    hi_w, lo_w, e_w = oracle.im2col3(x, pm_w, B, H, W, C, stride, Kp)
    dx = dev(x)
    pm = filled((B * H * W,), torch.int32)
    hi, lo, e = filled((Mp, Kp), torch.int8), filled((Mp, Kp), torch.int8), filled((Mp,), torch.int32)
    e2 = filled((rows,), torch.int32)
    vg.k_pixmax(dx, B * H * W, C, pm)
    vg.k_im2col3(dx, pm, B, H, W, C, stride, hi, lo, e, Kp)
    vg.k_conv_e(pm, B, H, W, stride, e2)
    torch.cuda.synchronize()
    assert_equal(to_np(pm).view(np.uint32), pm_w, "pixmax")
    assert_equal(to_np(hi), hi_w, "hi")
    assert_equal(to_np(lo), lo_w, "lo")
    assert_equal(to_np(e)[:rows], e_w[:rows], "e")
    assert (to_np(e)[rows:] == np.int32(FILL32)).all(), "e of a pad row was written"
    assert_equal(to_np(e2), oracle.conv_e(pm_w, B, H, W, stride), "conv_e")


def planes(r, M, ldc, bits):
    lim = 1 << bits
    return (r.integers(-lim, lim, (M, ldc)).astype(np.int32), r.integers(-lim, lim, (M, ldc)).astype(np.int32))


def constants(r, N):
    """Per-column (m, s, b, wsum) words over the ranges the engine's layers use and beyond."""
    s_lo, s_hi = [(16, 24), (4, 30), (-3, 8), (30, 45)][int(r.integers(4))]
    cst = np.zeros((N, 4), np.int32)
    cst[:, 0] = r.integers(-(2**20), 2**20, N)
    cst[:, 1] = r.integers(s_lo, s_hi, N)
    cst[:, 2] = r.integers(-(2**31), 2**31, N) if r.integers(4) == 0 else r.integers(-50000, 50000, N)
    cst[:, 3] = r.integers(-(2**20), 2**20, N)
    return cst


@pytest.mark.parametrize("seed", range(24))
def test_random_epilogue(seed):
    r = np.random.default_rng(42_000 + seed)
    gn = bool(r.integers(2))
    if gn:
        N = 32 * int(r.integers(1, 24))
        T = int(r.integers(1, 12))
        while (T * N) % 1024:   # the smallest multiple of the draw that keeps a block in one sample
            T += 1
        M = T * int(r.integers(1, 4)) - int(r.integers(0, min(T, 8)))
    else:
        N, T = 4 * int(r.integers(1, 200)), 0
        M = int(r.integers(1, 500))
    ldc = N + 4 * int(r.integers(0, 8))
    ldy = N + 4 * int(r.integers(0, 8))
    if gn:
        ldy = N   # statistics need ldy == N (src/kernels.cu:734 throws otherwise)
    mode = int(r.integers(3))   # 0: no residual, 1: residual aliases Y, 2: separate residual
    bits = int(r.choice([10, 20, 27, 30]))
    log("epilogue", seed, M=M, N=N, ldc=ldc, ldy=ldy, residual=mode, bits=bits, gn=gn, T=T)
    Chi, Clo = planes(r, M, ldc, bits)
    cst = constants(r, N)
    e = r.integers(0, 18, M).astype(np.int32)
    R = ints(r, (M, ldy)) if mode else None
    want = oracle.epilogue(Chi, Clo, M, N, ldc, cst, e, ldy, R)
    if mode == 1:
        Y = dev(R)
        res = Y
        want[:, N:] = R[:, N:]
    else:
        Y = filled((M, ldy), torch.int32)
        res = dev(R)
        want[:, N:] = FILL32
    gs = None
    if gn:
        cnt = -(-M // T) * 32
        gs = vg.gn_stats_alloc(cnt)
        vg.k_gn_init(gs, cnt)
    vg.k_epilogue(dev(Chi), dev(Clo), M, N, ldc, dev(cst), dev(e), Y, ldy, residual=res, gs=gs, T=T)
    torch.cuda.synchronize()
    assert_equal(to_np(Y), want, "Y")
    if gn:
        st = vg.gn_stats_read(gs, -(-M // T) * 32)
        ref = oracle.gn_stats_planar(want[:, :N], M, N, T)
        for k in ("sum", "mn", "mx"):
            assert_equal(st[k], ref[k], f"gn.{k}")


@pytest.mark.parametrize("seed", range(16))
def test_random_epilogue_split(seed):
    r = np.random.default_rng(43_000 + seed)
    Cs = int(r.integers(1, 300))
    N = int(r.integers(1, 3 * Cs + 1))
    M = int(r.integers(1, 400))
    ldc = N + int(r.integers(0, 9))
    bits = int(r.choice([10, 20, 27, 30]))
    log("epilogue_split", seed, M=M, N=N, ldc=ldc, Cs=Cs, bits=bits)
    Chi, Clo = planes(r, M, ldc, bits)
    cst = constants(r, N)
    e = r.integers(0, 18, M).astype(np.int32)
    ws = oracle.epilogue_split(Chi, Clo, M, N, ldc, cst, e, Cs)
    Ys = [filled((M, Cs), torch.int32) for _ in range(3)]
    vg.k_epilogue_split(dev(Chi), dev(Clo), M, N, ldc, dev(cst), dev(e), Cs, *Ys)
    torch.cuda.synchronize()
    for i, y in enumerate(Ys):
        # columns of a part beyond N are not produced; they keep the fill
        w = ws[i].copy()
        lo_col = i * Cs
        w[:, max(0, N - lo_col):] = FILL32
        assert_equal(to_np(y), w, f"part {i}")


@pytest.mark.parametrize("seed", range(16))
def test_random_epilogue_geglu_q(seed):
    r = np.random.default_rng(44_000 + seed)
    F = int(r.integers(1, 5121)) if r.integers(3) else int(r.integers(1, 64))
    M = int(r.integers(1, 200))
    ldc = 2 * F + int(r.integers(0, 9))
    Kp = F + int(r.integers(0, 40))
    bits = int(r.choice([12, 20, 24]))
    log("epilogue_geglu_q", seed, M=M, F=F, ldc=ldc, Kp=Kp, bits=bits)
    Chi, Clo = planes(r, M, ldc, bits)
    cst = constants(r, 2 * F)
    e = r.integers(0, 8, M).astype(np.int32)
    L = cf.phi_lut()
    hi_w, lo_w, eo_w = oracle.epilogue_geglu_q(Chi, Clo, M, F, ldc, cst, e, L, Kp)
    hi, lo, eo = filled((M, Kp), torch.int8), filled((M, Kp), torch.int8), filled((M,), torch.int32)
    vg.k_epilogue_geglu_q(dev(Chi), dev(Clo), M, F, ldc, dev(cst), dev(e), dev(L), hi, lo, eo, Kp)
    torch.cuda.synchronize()
    assert_equal(to_np(hi), hi_w, "hi")
    assert_equal(to_np(lo), lo_w, "lo")
    assert_equal(to_np(eo), eo_w, "e")


@pytest.mark.parametrize("seed", range(24))
def test_random_i8gemm(seed):
    """Gemm::run (src/gemm.cu:46-70): C = A * W^T over a strided batch, leading dimensions at random."""
    r = np.random.default_rng(45_000 + seed)
    M, N, K = int(r.integers(1, 700)), 4 * int(r.integers(1, 160)), 16 * int(r.integers(1, 80))
    batch = int(r.choice([1, 1, 2, 3]))
    lda, ldw = K + 16 * int(r.integers(0, 3)), K + 16 * int(r.integers(0, 3))
    ldc = N + int(r.integers(0, 9)) if batch == 1 else N + 4 * int(r.integers(0, 3))
    sA, sW, sC = M * lda + 16 * int(r.integers(0, 4)), N * ldw + 16 * int(r.integers(0, 4)), M * ldc + 4 * int(r.integers(0, 4))
    variant = int(r.choice([-1, -1, 0, 1, 2, 3]))
    log("i8gemm", seed, M=M, N=N, K=K, batch=batch, lda=lda, ldw=ldw, ldc=ldc, sA=sA, sW=sW, sC=sC, variant=variant)
    A = r.integers(-128, 128, sA * batch).astype(np.int8)
    W = r.integers(-128, 128, sW * batch).astype(np.int8)
    want = oracle.i8gemm(A, W, M, N, K, batch, sA, sW, sC, lda, ldw, ldc)
    size = max(sC * batch, M * ldc) if batch > 1 else M * ldc
    C = filled((size,), torch.int32)
    vg.set_variant(variant)
    try:
        g = vg.Gemm()
        g.init(32 << 20)
        g.run(dev(A), lda, sA, dev(W), ldw, sW, C, ldc, sC, M, N, K, batch)
        torch.cuda.synchronize()
    finally:
        vg.set_variant(-1)
    got = to_np(C)
    written = np.zeros(size, bool)
    for b in range(batch):
        idx = b * sC + np.arange(M)[:, None] * ldc + np.arange(N)[None, :]
        written[idx.reshape(-1)] = True
    assert_equal(got[written], want[written], "C")
    assert (got[~written] == np.int32(FILL32)).all(), "Gemm::run wrote outside the C rows and columns"

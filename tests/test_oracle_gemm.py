"""Pins of the oracle's GEMM, producers and weight preparation (oracle/oracle.c) against independent
definitions (tests/refmath.py), textbook routines and the reference's own invariants. No GPU.

  * every source (SRC_I8 planes, SRC_I16, SRC_X32, SRC_CONV32, SRC_CONV16) and epilogue (PLAIN +
    residual + rowmax, GELU, GEGLU + rowmax, SPLIT3) against one exact q.W product with rational
    rounding -- the hi/lo planes and the 128*wsum correction never appear in the checker;
  * m = 1, s = 0, b = 0, e = 0: a plain saturated integer matmul; for a 3x3 conv with C = 1, a
    direct 2-D correlation (scipy.signal.correlate2d);
  * SRC_X32 == k_quant_rows + SRC_I8 and SRC_CONV32 == k_im2col3 + SRC_I8 (src/test_gemm_hl.cu:25-41);
  * k_im2col3 on the reference's own case grid (src/test_im2col.cu:13-20) against patches cut from a
    zero-padded image;
  * the tap-major weight permutation (src/engine.cu:36) against a transpose of [N, C, 3, 3].
"""
import numpy as np
import pytest
from scipy.signal import correlate2d

import oracle
from tests import refmath as rm


def rng(seed):
    return np.random.default_rng(seed)


def align(v, a):
    return (v + a - 1) // a * a


def make_cst(r, N, w_real, m_range=(1 << 14, 1 << 15), s_range=(16, 24), b_range=(-50000, 50000), Np=None):
    Np = Np or N
    cst = np.zeros((Np, 4), np.int32)
    cst[:, 0] = 1
    cst[:N, 0] = r.integers(*m_range, N, dtype=np.int64)
    cst[:N, 1] = r.integers(s_range[0], s_range[1] + 1, N)
    cst[:N, 2] = r.integers(*b_range, N, dtype=np.int64)
    cst[:N, 3] = w_real.astype(np.int64).sum(1)
    return cst


def pad_w(w_real, Np, Kp):
    w = np.zeros((Np, Kp), np.int8)
    w[: w_real.shape[0], : w_real.shape[1]] = w_real
    return w


EPIS = [("plain", oracle.EPI_PLAIN), ("gelu", oracle.EPI_GELU), ("geglu", oracle.EPI_GEGLU)]


@pytest.mark.parametrize("epi_name,epi", EPIS)
@pytest.mark.parametrize("with_e", [False, True])
def test_i16_against_definition(epi_name, epi, with_e):
    r = rng(10 + epi + 3 * with_e)
    M, N, K = 9, 12, 40
    Kp = align(K, 16)
    q = r.integers(-32768, 32768, (M, K)).astype(np.int16)
    q[0, :16] = [-32768, -32767, -32766, -32513, -256, -255, -128, -1, 0, 1, 127, 128, 255, 256, 32766, 32767]
    w_real = r.integers(-127, 128, (N, K)).astype(np.int8)
    w_real[1] = 127
    w_real[2] = -127
    cst = make_cst(r, N, w_real, s_range=(10, 30))
    cst[3] = [2**31 - 1, 40, 0, w_real[3].astype(np.int64).sum()]          # large multiplier
    cst[4] = [12345, -3, 2**31 - 7, w_real[4].astype(np.int64).sum()]      # left shift, b near the top
    e = r.integers(0, 18, M).astype(np.int32) if with_e else None
    L = np.sort(r.integers(0, 65537, 2049)).astype(np.int32)
    res = r.integers(-(2**31), 2**31, (M, N // 2 if epi == oracle.EPI_GEGLU else N), dtype=np.int64).astype(np.int32) \
        if epi == oracle.EPI_PLAIN else None
    rmax0 = r.integers(0, 2**20, M).astype(np.uint32)
    rowmax = rmax0.copy()
    nout = N // 2 if epi == oracle.EPI_GEGLU else N
    Y = np.zeros((M, nout), np.int32) if res is None else res.copy()
    oracle.gemm(oracle.SRC_I16, Mreal=M, Nreal=N, Kp=Kp, w=pad_w(w_real, N, Kp), cst=cst, epi=epi, e=e, q16=q, K=K, Lphi=L,
                Y=Y, residual=Y if res is not None else None, rowmax=rowmax)
    want, wrm = rm.gemm(q, w_real, cst, e=e, epi=epi_name, residual=res, L=L, rowmax=rmax0)
    np.testing.assert_array_equal(Y, want)
    np.testing.assert_array_equal(rowmax, wrm)


def test_i8_planes_against_definition():
    """SRC_I8 planes carry q = 256*hi + lo + 128 (src/gemm_hl.h:1-3)."""
    r = rng(20)
    M, N, Kp = 7, 10, 48
    hi = r.integers(-128, 128, (M, Kp)).astype(np.int8)
    lo = r.integers(-128, 128, (M, Kp)).astype(np.int8)
    q = 256 * hi.astype(np.int64) + lo + 128
    w_real = r.integers(-128, 128, (N, Kp)).astype(np.int8)
    cst = make_cst(r, N, w_real)
    e = r.integers(0, 12, M).astype(np.int32)
    Y = oracle.gemm(oracle.SRC_I8, Mreal=M, Nreal=N, Kp=Kp, w=w_real, cst=cst, e=e, hi=hi, lo=lo)
    want, _ = rm.gemm(q, w_real, cst, e=e)
    np.testing.assert_array_equal(Y, want)


def test_split3_against_definition():
    r = rng(21)
    M, Cs, K = 5, 8, 32
    N = 3 * Cs
    q = r.integers(-32768, 32768, (M, K)).astype(np.int16)
    w_real = r.integers(-127, 128, (N, K)).astype(np.int8)
    cst = make_cst(r, N, w_real)
    Ys = [np.zeros((M, Cs), np.int32) for _ in range(3)]
    oracle.gemm(oracle.SRC_I16, Mreal=M, Nreal=N, Kp=K, w=w_real, cst=cst, epi=oracle.EPI_SPLIT3, q16=q, K=K, Y=Ys[0], ldy=Cs,
                Cs=Cs, Y1=Ys[1], Y2=Ys[2])
    want, _ = rm.gemm(q, w_real, cst, epi="split3", Cs=Cs)
    for g, w_ in zip(Ys, want):
        np.testing.assert_array_equal(g, w_)


def test_x32_against_definition_and_quant_rows():
    """SRC_X32: e = row_exp(max |x|) and q = quant16(x, e) (src/gemm_hl.cu:99-121); equal to
    k_quant_rows followed by SRC_I8 (src/test_gemm_hl.cu:31-41)."""
    r = rng(22)
    M, N, K = 8, 12, 36
    Kp = align(K, 16)
    bits = r.integers(1, 32, (M, 1))
    x = (r.integers(0, 2**31, (M, K), dtype=np.int64) & ((1 << bits) - 1)) - (1 << (bits - 1))
    x[0, 0] = -(2**31)
    x = x.astype(np.int32)
    xrm = np.abs(x.astype(np.int64)).max(1).astype(np.uint32)
    w_real = r.integers(-127, 128, (N, K)).astype(np.int8)
    cst = make_cst(r, N, w_real, s_range=(0, 30))
    w = pad_w(w_real, N, Kp)
    Y = oracle.gemm(oracle.SRC_X32, Mreal=M, Nreal=N, Kp=Kp, w=w, cst=cst, x=x, xrowmax=xrm, K=K)
    e = np.array([rm.row_exp(int(v)) for v in xrm], np.int32)
    want, _ = rm.gemm(rm.quant_matrix(x, e), w_real, cst, e=e)
    np.testing.assert_array_equal(Y, want)
    hi, lo, e2 = oracle.quant_rows(x, M, K, K, Kp)
    np.testing.assert_array_equal(e2[:M], e)
    assert np.all(hi[M:] == 0) and np.all(lo[M:] == -128)           # pad rows hold the value 0
    Y2 = oracle.gemm(oracle.SRC_I8, Mreal=M, Nreal=N, Kp=Kp, w=w, cst=cst, hi=hi, lo=lo, e=e2)
    np.testing.assert_array_equal(Y2, Y)


@pytest.mark.parametrize("src", [oracle.SRC_CONV32, oracle.SRC_CONV16])
@pytest.mark.parametrize("geom", [(2, 5, 7, 16, 1), (1, 6, 5, 32, 2), (2, 4, 4, 48, 1)])
def test_conv_against_definition(src, geom):
    """Implicit 3x3 / pad 1 im2col (src/gemm_hl.cu:104-114): e per output pixel from the window's
    max |x| (src/gemm_hl.cu:335-341), weights from PyTorch's [N, C, 3, 3] by the tap-major
    permutation (src/engine.cu:36)."""
    B, H, W, C, stride = geom
    r = rng(23 + C + stride)
    N = 24
    if src == oracle.SRC_CONV32:
        bits = r.integers(1, 32, (B, H, W, 1))
        img = ((r.integers(0, 2**31, (B, H, W, C), dtype=np.int64) & ((1 << bits) - 1)) - (1 << (bits - 1))).astype(np.int32)
    else:
        img = r.integers(-32768, 32768, (B, H, W, C)).astype(np.int16)
    w_nchw = r.integers(-127, 128, (N, C, 3, 3)).astype(np.int8)
    m = r.integers(1 << 14, 1 << 15, N).astype(np.int32)
    s = r.integers(16, 25, N).astype(np.int32)
    b = r.integers(-50000, 50000, N).astype(np.int32)
    K = 9 * C
    Kp = align(K, 16)
    w, cst = oracle.prep_weight(w_nchw.reshape(N, K), N, K, True, m, s, b, N, Kp)
    w_tm = rm.tapmajor_weights(w_nchw)
    np.testing.assert_array_equal(w[:, :K], w_tm)
    np.testing.assert_array_equal(cst[:, 3], w_nchw.reshape(N, -1).astype(np.int64).sum(1))
    pm = oracle.pixmax(img.astype(np.int32).reshape(-1, C), B * H * W, C)
    e = oracle.conv_e(pm, B, H, W, stride)
    e_def = rm.conv_row_exp(img, stride)
    np.testing.assert_array_equal(e, e_def)
    Mr = len(e)
    Y = oracle.gemm(src, Mreal=Mr, Nreal=N, Kp=Kp, w=w, cst=cst, e=e, img=img, H=H, W=W, C=C, stride=stride)
    q = rm.quant_matrix(rm.im2col_tapmajor(img, stride), e_def)
    want, _ = rm.gemm(q, w_tm, cst, e=e_def)
    np.testing.assert_array_equal(Y, want)
    if src == oracle.SRC_CONV32:
        # == k_pixmax + k_im2col3 + SRC_I8 (src/test_gemm_hl.cu:25-29)
        hi, lo, e3 = oracle.im2col3(img, pm, B, H, W, C, stride, Kp)
        Y3 = oracle.gemm(oracle.SRC_I8, Mreal=Mr, Nreal=N, Kp=Kp, w=w, cst=cst, hi=hi, lo=lo, e=e3)
        np.testing.assert_array_equal(Y3, Y)


def test_plain_matmul_special_case():
    """m = 1, s = 0, b = 0, e = 0: Y = sat32(q @ w.T), a textbook integer matmul; extreme operands
    drive the sums past 2^31 so saturation is exercised."""
    r = rng(30)
    M, N, K = 16, 20, 640
    q = r.integers(-32768, 32768, (M, K)).astype(np.int16)
    q[:4] = 32767
    q[4:6] = -32768
    w_real = r.integers(-128, 128, (N, K)).astype(np.int8)
    w_real[:3] = 127
    w_real[3:5] = -128
    cst = np.zeros((N, 4), np.int32)
    cst[:, 0] = 1
    cst[:, 3] = w_real.astype(np.int64).sum(1)
    Y = oracle.gemm(oracle.SRC_I16, Mreal=M, Nreal=N, Kp=K, w=w_real, cst=cst, q16=q, K=K)
    ref = np.clip(q.astype(np.int64) @ w_real.astype(np.int64).T, -(2**31), 2**31 - 1)
    assert (np.abs(ref) == 2**31 - 1).sum() + (ref == -(2**31)).sum() > 0
    np.testing.assert_array_equal(Y, ref)


def test_single_channel_conv_is_correlate2d():
    """C = 1 (padded to 16 channels of which 15 are zero), m = 1, s = b = 0: a direct 3x3
    cross-correlation with zero padding."""
    r = rng(31)
    B, H, W, C = 1, 9, 11, 16
    img = np.zeros((B, H, W, C), np.int32)
    img[..., 0] = r.integers(-30000, 30000, (H, W))
    ker = r.integers(-127, 128, (3, 3))
    w_nchw = np.zeros((1, C, 3, 3), np.int8)
    w_nchw[0, 0] = ker
    K = 9 * C
    w, cst = oracle.prep_weight(w_nchw.reshape(1, K), 1, K, True, np.ones(1), np.zeros(1), np.zeros(1), 1, K)
    Y = oracle.gemm(oracle.SRC_CONV32, Mreal=H * W, Nreal=1, Kp=K, w=w, cst=cst, e=np.zeros(H * W, np.int32), img=img, H=H,
                    W=W, C=C, stride=1)
    want = correlate2d(img[0, :, :, 0].astype(np.int64), ker, mode="same", boundary="fill")
    np.testing.assert_array_equal(Y.reshape(H, W), want)


@pytest.mark.parametrize("C", [4, 12, 16, 32, 320])
@pytest.mark.parametrize("stride", [1, 2])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_im2col3_reference_grid(C, stride, mode):
    """src/test_im2col.cu:13-45: B=2, H=5, W=7; x = 0 / random 16-bit / random 32-bit with INT_MIN
    and INT_MAX at every 19th element; pad rows (0, -128)."""
    B, H, W = 2, 5, 7
    r = rng(C * 10 + stride + mode)
    n = B * H * W * C
    if mode == 0:
        x = np.zeros(n, np.int64)
    elif mode == 1:
        x = r.integers(0, 65537, n) - 32768
    else:
        x = r.integers(-(2**31), 2**31, n, dtype=np.int64)
        idx = np.arange(0, n, 19)
        x[idx] = np.where(idx & 1, -(2**31), 2**31 - 1)
    img = x.astype(np.int32).reshape(B, H, W, C)
    Kp = align(9 * C, 16)
    pm = oracle.pixmax(img.reshape(-1, C), B * H * W, C)
    hi, lo, e = oracle.im2col3(img, pm, B, H, W, C, stride, Kp)
    rows = B * ((H - 1) // stride + 1) * ((W - 1) // stride + 1)
    e_def = rm.conv_row_exp(img, stride)
    np.testing.assert_array_equal(e[:rows], e_def)
    q = np.zeros((hi.shape[0], Kp), np.int64)
    q[:rows, : 9 * C] = rm.quant_matrix(rm.im2col_tapmajor(img, stride), e_def)
    h_def, l_def = rm.split(q)
    np.testing.assert_array_equal(hi, h_def)
    np.testing.assert_array_equal(lo, l_def)


def test_cublaslt_path_epilogues():
    """k_epilogue / k_epilogue_split / k_epilogue_geglu_q (src/kernels.cu:70-104, 499-534) on plane
    sums from a plain int8 matmul: the same values as the fused GEMM."""
    r = rng(40)
    M, K, F = 6, 64, 16
    N = 2 * F
    q = r.integers(-32768, 32768, (M, K)).astype(np.int16)
    hi, lo = rm.split(q)
    w_real = r.integers(-127, 128, (N, K)).astype(np.int8)
    Chi = oracle.i8gemm(hi, w_real, M, N, K).reshape(M, N)
    Clo = oracle.i8gemm(lo, w_real, M, N, K).reshape(M, N)
    np.testing.assert_array_equal(Chi, hi.astype(np.int64) @ w_real.astype(np.int64).T)   # textbook matmul
    cst = make_cst(r, N, w_real)
    e = r.integers(0, 4, M).astype(np.int32)
    R = r.integers(-(2**31), 2**31, (M, N), dtype=np.int64).astype(np.int32)
    Y = oracle.epilogue(Chi, Clo, M, N, N, cst, e, N, R)
    want, _ = rm.gemm(q, w_real, cst, e=e, residual=R)
    np.testing.assert_array_equal(Y, want)
    parts = oracle.epilogue_split(Chi, Clo, M, N, N, cst, e, 12)
    wparts, _ = rm.gemm(q, w_real, cst, e=e, epi="split3", Cs=12)
    for g, w_ in zip(parts, wparts):
        np.testing.assert_array_equal(g, w_)
    # geglu_q: columns [0, F) are a, [F, 2F) are g (the non-interleaved layout of k_epilogue_geglu_q)
    L = np.sort(r.integers(0, 65537, 2049)).astype(np.int32)
    Kp = 32
    qh, ql, eo = oracle.epilogue_geglu_q(Chi, Clo, M, F, N, cst, e, L, Kp)
    perm = np.empty(N, int)
    perm[0::2] = np.arange(F)
    perm[1::2] = F + np.arange(F)
    v, _ = rm.gemm(q, w_real[perm], cst[perm], e=e, epi="geglu", L=L)
    e_def = np.array([rm.row_exp(int(np.abs(v[i].astype(np.int64)).max())) for i in range(M)], np.int32)
    np.testing.assert_array_equal(eo, e_def)
    qv = np.zeros((M, Kp), np.int64)
    qv[:, :F] = rm.quant_matrix(v, e_def)
    h_def, l_def = rm.split(qv)
    np.testing.assert_array_equal(qh, h_def)
    np.testing.assert_array_equal(ql, l_def)


def test_i8gemm_strided_batch():
    """Gemm::run (src/gemm.cu:22-35): C = A W^T per batch with element strides."""
    r = rng(41)
    M, N, K, batch = 5, 8, 32, 3
    sA, sW, sC = M * K + 16, N * K + 32, M * N + 4
    A = r.integers(-128, 128, sA * batch).astype(np.int8)
    W = r.integers(-128, 128, sW * batch).astype(np.int8)
    C = oracle.i8gemm(A, W, M, N, K, batch=batch, sA=sA, sW=sW, sC=sC)
    for bt in range(batch):
        a = A[bt * sA: bt * sA + M * K].reshape(M, K).astype(np.int64)
        w = W[bt * sW: bt * sW + N * K].reshape(N, K).astype(np.int64)
        np.testing.assert_array_equal(C[bt * sC: bt * sC + M * N].reshape(M, N), a @ w.T)


def test_weight_prep_and_interleave():
    """DevModel::load padding (src/engine.cu:26-44) and mergeLins interleave (:81-88)."""
    r = rng(42)
    N, K = 5, 20
    Np, Kp = 64, 32
    w = r.integers(-127, 128, (N, K)).astype(np.int8)
    m, s, b = (r.integers(1, 1000, N).astype(np.int32) for _ in range(3))
    wout, cst = oracle.prep_weight(w, N, K, False, m, s, b, Np, Kp)
    np.testing.assert_array_equal(wout[:N, :K], w)
    assert not wout[N:].any() and not wout[:, K:].any()
    np.testing.assert_array_equal(cst[:N], np.stack([m, s, b, w.astype(np.int64).sum(1)], 1))
    np.testing.assert_array_equal(cst[N:], np.tile([1, 0, 0, 0], (Np - N, 1)))
    wa, wg = (pad_w(r.integers(-127, 128, (N, Kp)).astype(np.int8), N, Kp) for _ in range(2))
    ca, cg = (r.integers(0, 100, (N, 4)).astype(np.int32) for _ in range(2))
    wi, ci = oracle.interleave2(wa, ca, wg, cg, N, Kp)
    np.testing.assert_array_equal(wi[0:2 * N:2], wa)
    np.testing.assert_array_equal(wi[1:2 * N:2], wg)
    np.testing.assert_array_equal(ci[0:2 * N:2], ca)
    np.testing.assert_array_equal(ci[1:2 * N:2], cg)
    np.testing.assert_array_equal(ci[2 * N:], np.tile([1, 0, 0, 0], (wi.shape[0] - 2 * N, 1)))


def test_rows_are_independent():
    """Each output row depends on its own A row only: a row range gives the same rows."""
    r = rng(43)
    M, N, K = 40, 16, 64
    q = r.integers(-32768, 32768, (M, K)).astype(np.int16)
    w = r.integers(-127, 128, (N, K)).astype(np.int8)
    cst = make_cst(r, N, w)
    full = oracle.gemm(oracle.SRC_I16, Mreal=M, Nreal=N, Kp=K, w=w, cst=cst, q16=q, K=K)
    part = oracle.gemm(oracle.SRC_I16, Mreal=M, Nreal=N, Kp=K, w=w, cst=cst, q16=q, K=K, rows=(13, 29))
    np.testing.assert_array_equal(part[13:29], full[13:29])
    assert not part[:13].any() and not part[29:].any()

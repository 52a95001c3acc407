"""The GPU path (vgemm_hl2 through the C ABI) against the golden fixtures and the hand-worked case --
expected values that come from the definitions, not from the oracle."""
import numpy as np
import pytest
import torch

from tests.conftest import assert_equal, to_np
from tests.test_golden import EPI, HAND_CST, HAND_L, HAND_Q, HAND_W, load
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu


def align(v, a):
    return (v + a - 1) // a * a


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def padded_w(w, cst):
    N, K = w.shape
    Np, Kp = align(N, 64), align(K, 16)
    wp = np.zeros((Np, Kp), np.int8)
    wp[:N, :K] = w
    cp = np.zeros((Np, 4), np.int32)
    cp[:, 0] = 1
    cp[:N] = cst
    return wp, cp, Np, Kp


def run(A, M, w, cst, epi=vg.EPI_PLAIN, nout=None, residual=None, Lphi=None, rowmax=False):
    N = w.shape[0]
    wp, cp, Np, Kp = padded_w(w, cst)
    nout = nout or N
    Y = dev(residual) if residual is not None else torch.zeros((M, nout), dtype=torch.int32, device="cuda")
    rm = torch.zeros(M, dtype=torch.int32, device="cuda") if rowmax else None
    keep = [dev(wp), dev(cp)]
    E = vg.AEpi(epi=epi, Y=vg.ptr(Y), ldy=nout, rowmax=vg.ptr(rm))
    if residual is not None:
        E.residual = vg.ptr(Y)
    if Lphi is not None:
        keep.append(dev(Lphi))
        E.Lphi = vg.ptr(keep[-1])
    vg.k_gemm_hl2(A, align(M, 64), M, keep[0], Kp, Np, N, Kp, keep[1], E)
    torch.cuda.synchronize()
    return to_np(Y), (to_np(rm).view(np.uint32) if rm is not None else None)


@pytest.mark.parametrize("name", ["i16_plain_edges", "i16_geglu", "i16_gelu"])
def test_linear_fixtures_gpu(gpu, name):
    f = load(name)
    M, K = f["q16"].shape
    q, e = dev(f["q16"]), dev(f["e"])
    A = vg.ASrc(src=vg.SRC_I16, q16=vg.ptr(q), ld16=K, K=K, e=vg.ptr(e))
    epi = EPI[str(f["epi"])]
    Y, rowmax = run(A, M, f["w"], f["cst"], epi=epi, nout=f["Y"].shape[1], residual=f.get("residual"), Lphi=f["Lphi"],
                    rowmax=epi != vg.EPI_GELU)
    assert_equal(Y, f["Y"], name)
    if rowmax is not None:
        assert_equal(rowmax, f["rowmax"], name + " rowmax")


def test_x32_fixture_gpu(gpu):
    f = load("x32_rowexp")
    M, K = f["x"].shape
    x, xrm = dev(f["x"]), dev(f["xrowmax"].view(np.int32))
    A = vg.ASrc(src=vg.SRC_X32, x=vg.ptr(x), ldx=K, rowmax=vg.ptr(xrm), K=K)
    Y, _ = run(A, M, f["w"], f["cst"])
    assert_equal(Y, f["Y"], "x32")


@pytest.mark.parametrize("name,src", [("conv16_s1", vg.SRC_CONV16), ("conv32_s2", vg.SRC_CONV32)])
def test_conv_fixtures_gpu(gpu, name, src):
    f = load(name)
    B, H, W, C, stride = (int(v) for v in f["geom"])
    img, e = dev(f["img"]), dev(f["e"])
    A = vg.ASrc(src=src, e=vg.ptr(e), H=H, W=W, C=C, stride=stride, Ho=(H - 1) // stride + 1, Wo=(W - 1) // stride + 1, K=9 * C)
    if src == vg.SRC_CONV16:
        A.img16 = vg.ptr(img)
    else:
        A.img = vg.ptr(img)
    Y, _ = run(A, len(f["e"]), f["w_tapmajor"], f["cst"])
    assert_equal(Y, f["Y"], name)


def test_hand_worked_gpu(gpu):
    q = dev(HAND_Q)
    A = vg.ASrc(src=vg.SRC_I16, q16=vg.ptr(q), ld16=16, K=16)
    Y, _ = run(A, 1, HAND_W, HAND_CST)
    assert Y.tolist() == [[-3740, -15944]]
    Yg, rowmax = run(A, 1, HAND_W, HAND_CST, epi=vg.EPI_GEGLU, nout=1, Lphi=HAND_L, rowmax=True)
    assert Yg.tolist() == [[448]] and rowmax.tolist() == [448]

"""The oracle against the committed golden fixtures (tests/golden/*.npz, written from the independent
definitions by tests/golden/make_golden.py) and against one case worked by hand. No GPU."""
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
EPI = {"plain": oracle.EPI_PLAIN, "geglu": oracle.EPI_GEGLU, "gelu": oracle.EPI_GELU}


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def oracle_linear(f):
    epi = EPI[str(f["epi"])]
    M, K = f["q16"].shape
    N = f["w"].shape[0]
    nout = N // 2 if epi == oracle.EPI_GEGLU else N
    Y = f["residual"].copy() if "residual" in f else np.zeros((M, nout), np.int32)
    rowmax = np.zeros(M, np.uint32)
    oracle.gemm(oracle.SRC_I16, Mreal=M, Nreal=N, Kp=K, w=f["w"], cst=f["cst"], epi=epi, e=f["e"], q16=f["q16"], K=K,
                Lphi=f["Lphi"], Y=Y, residual=Y if "residual" in f else None, rowmax=rowmax)
    return Y, rowmax


@pytest.mark.parametrize("name", ["i16_plain_edges", "i16_geglu", "i16_gelu"])
def test_linear_fixtures(name):
    f = load(name)
    Y, rowmax = oracle_linear(f)
    np.testing.assert_array_equal(Y, f["Y"])
    np.testing.assert_array_equal(rowmax, f["rowmax"])


def test_x32_fixture():
    f = load("x32_rowexp")
    M, K = f["x"].shape
    Y = oracle.gemm(oracle.SRC_X32, Mreal=M, Nreal=f["w"].shape[0], Kp=K, w=f["w"], cst=f["cst"], x=f["x"], xrowmax=f["xrowmax"], K=K)
    np.testing.assert_array_equal(Y, f["Y"])
    assert f["e_expected"].max() == 17


@pytest.mark.parametrize("name,src", [("conv16_s1", oracle.SRC_CONV16), ("conv32_s2", oracle.SRC_CONV32)])
def test_conv_fixtures(name, src):
    f = load(name)
    B, H, W, C, stride = (int(v) for v in f["geom"])
    N = f["w_nchw"].shape[0]
    K = 9 * C
    w, _ = oracle.prep_weight(f["w_nchw"].reshape(N, K), N, K, True, f["cst"][:, 0], f["cst"][:, 1], f["cst"][:, 2], N, K)
    np.testing.assert_array_equal(w, f["w_tapmajor"])
    pm = oracle.pixmax(f["img"].astype(np.int32).reshape(-1, C), B * H * W, C)
    e = oracle.conv_e(pm, B, H, W, stride)
    np.testing.assert_array_equal(e, f["e"])
    Y = oracle.gemm(src, Mreal=len(e), Nreal=N, Kp=K, w=w, cst=f["cst"], e=e, img=f["img"], H=H, W=W, C=C, stride=stride)
    np.testing.assert_array_equal(Y, f["Y"])


# ---- worked by hand
# q = [1000, -2000, 0...] (K = 16), W rows: [3, 4, 0...] and [-1, 127, 0...]
#   acc0 = 3000 - 8000 = -5000;   acc1 = -1000 - 254000 = -255000
#   col 0: m = 3, s = 2, b = 10:  -15000 / 4 = -3750 exactly         -> -3750 + 10  = -3740
#   col 1: m = 1, s = 4, b = -7:  -255000 / 16 = -15937.5, half up    -> -15937 - 7  = -15944
# GEGLU of the pair (a = -3740, g = -15944) with L[i] = 32 i, so lut(x) = floor((x + 2^20) / 32):
#   lut(g) = floor(1032632 / 32) = 32269
#   ge = rshr(-15944 * 32269, 16) = rshr(-514496936, 16): -7850.600... -> -7851
#   v  = rshr(-3740 * -7851, 16)  = rshr(29362740, 16):  448.039...    -> 448
HAND_Q = np.zeros((1, 16), np.int16)
HAND_Q[0, :2] = [1000, -2000]
HAND_W = np.zeros((2, 16), np.int8)
HAND_W[0, :2] = [3, 4]
HAND_W[1, :2] = [-1, 127]
HAND_CST = np.array([[3, 2, 10, 7], [1, 4, -7, 126]], np.int32)
HAND_L = (32 * np.arange(2049)).astype(np.int32)


def test_hand_worked_plain_and_geglu():
    Y = oracle.gemm(oracle.SRC_I16, Mreal=1, Nreal=2, Kp=16, w=HAND_W, cst=HAND_CST, q16=HAND_Q, K=16)
    assert Y.tolist() == [[-3740, -15944]]
    rowmax = np.zeros(1, np.uint32)
    Yg = oracle.gemm(oracle.SRC_I16, Mreal=1, Nreal=2, Kp=16, w=HAND_W, cst=HAND_CST, q16=HAND_Q, K=16, epi=oracle.EPI_GEGLU,
                     Lphi=HAND_L, rowmax=rowmax)
    assert Yg.tolist() == [[448]] and rowmax.tolist() == [448]

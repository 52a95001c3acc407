"""The real-weights path on the GPU: tests/golden/tiny_model.poisd loaded by the library
(vgemm_model_open + vgemm_model_upload, i.e. Poisd::load + DevModel::load) and its prepared
linears -- 3x3 convolutions, the merged to_qkv and the alternating GEGLU projection "agi" with the
file's own lut.phi -- run through vgemm_hl2, bit-exact against the oracle over the operands the
oracle prepares from the same file (oracle/model.py)."""
import numpy as np
import pytest
import torch

import oracle
from oracle import model as om
from tests.conftest import assert_equal, to_np
from tests.golden import make_poisd as mp
from vela_amd import gemm as vg
from vela_amd.model import DevModel, Poisd

pytestmark = pytest.mark.gpu

BLOCK = mp.BLOCK


@pytest.fixture(scope="module")
def loaded(gpu):
    m = Poisd()
    m.load(mp.PATH)
    dm = DevModel()
    dm.load(0, m)
    ents = om.parse_poisd(mp.PATH.read_bytes())
    lins, _ = om.dev_model(ents)
    yield m, dm, lins, ents["lut.phi"][2].astype(np.int32)
    m.close()


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def run_conv(dm, lins, name, B, H, W, C, seed, residual=False):
    L = dm.lin(name)
    Wo, cst, N, K, conv3 = lins[name]
    assert conv3 and L.conv3 and K == 9 * C
    r = np.random.default_rng(seed)
    img = r.integers(-32767, 32768, (B, H, W, C)).astype(np.int16)
    M = B * H * W
    res = r.integers(-(2**31), 2**31, (M, N), dtype=np.int64).astype(np.int32) if residual else None
    want = np.zeros((M, N), np.int32) if res is None else res.copy()
    oracle.gemm(oracle.SRC_CONV16, Mreal=M, Nreal=N, Kp=L.Kp, w=Wo, cst=cst, img=img, H=H, W=W, C=C, Y=want,
                residual=want if res is not None else None)
    dimg = dev(img)
    Y = dev(res) if res is not None else torch.zeros((M, N), dtype=torch.int32, device="cuda")
    A = vg.ASrc(src=vg.SRC_CONV16, img16=vg.ptr(dimg), H=H, W=W, C=C, stride=1, Ho=H, Wo=W, K=9 * C)
    E = vg.AEpi(Y=vg.ptr(Y), ldy=N, residual=vg.ptr(Y) if res is not None else None)
    vg.k_gemm_hl2(A, (M + 63) // 64 * 64, M, L.w, L.Kp, L.Np, N, L.Kp, L.cst, E)
    torch.cuda.synchronize()
    assert_equal(to_np(Y), want, name)


def test_model_upload(loaded):
    m, dm, lins, _ = loaded
    assert dm.bytes >= sum(W.nbytes + c.nbytes for W, c, *_ in lins.values())
    for name in lins:
        L = dm.lin(name)
        assert L.w and L.cst and L.w % 256 == 0 and L.cst % 256 == 0, name
    p, n = dm.table("lut.phi")
    assert p and n == 2049


def test_loaded_convolutions(loaded):
    _, dm, lins, _ = loaded
    run_conv(dm, lins, mp.RESNET + ".conv1", 2, 8, 8, 64, seed=1)
    run_conv(dm, lins, mp.RESNET + ".conv2", 1, 16, 16, 64, seed=2, residual=True)
    run_conv(dm, lins, "unet.conv_in", 2, 8, 8, 8, seed=3)
    run_conv(dm, lins, "unet.conv_out", 1, 8, 8, 64, seed=4)


@pytest.mark.parametrize("name,epi", [(BLOCK + ".attn1.to_qkv", vg.EPI_PLAIN), (BLOCK + ".ff.net.0.proj.agi", vg.EPI_GEGLU),
                                      ("unet.time_embedding.linear_1", vg.EPI_PLAIN), (mp.RESNET + ".conv_shortcut", vg.EPI_PLAIN)])
def test_loaded_linears(loaded, name, epi):
    _, dm, lins, phi = loaded
    L = dm.lin(name)
    Wo, cst, N, K, _ = lins[name]
    M = 130
    r = np.random.default_rng(len(name))
    q = r.integers(-32767, 32768, (M, K)).astype(np.int16)
    nout = N // 2 if epi == vg.EPI_GEGLU else N
    want = oracle.gemm(oracle.SRC_I16, Mreal=M, Nreal=N, Kp=L.Kp, w=Wo, cst=cst, q16=q, K=K, epi=epi, Lphi=phi)
    dq = dev(q)
    Y = torch.zeros((M, nout), dtype=torch.int32, device="cuda")
    lut, _ = dm.table("lut.phi")
    A = vg.ASrc(src=vg.SRC_I16, q16=vg.ptr(dq), ld16=K, K=K)
    E = vg.AEpi(epi=epi, Y=vg.ptr(Y), ldy=nout, Lphi=lut)
    vg.k_gemm_hl2(A, (M + 63) // 64 * 64, M, L.w, L.Kp, L.Np, N, L.Kp, L.cst, E)
    torch.cuda.synchronize()
    assert_equal(to_np(Y), want, name)

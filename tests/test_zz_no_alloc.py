"""vgemm_hl2_noalloc, the allocation-free entry point, against vgemm_hl2 with a caller workspace.

The two must give the same bytes. The shapes split K (the deep 3x3 convolutions of the UNet's
lowest level and a smaller one after it), so the static workspace is really used; the second call
is smaller than the first and reuses the workspace the first call left behind. A call whose split
would need more than the static workspace is rejected with VGEMM_ERR_UNSUPPORTED.
"""
import numpy as np
import pytest
import torch

from tests.conftest import assert_equal, to_np
from tests.test_gpu_gemm import Case, dev
from vela_amd import _lib
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _knobs(gpu):
    vg.set_variant(-1)
    vg.set_splitk(0)
    yield
    vg.set_variant(-1)
    vg.set_splitk(0)


def run(c: Case, noalloc: bool):
    keep = {}
    A = c.asrc(keep)
    w, cst, lut = dev(c.w), dev(c.cst), dev(c.lut)
    Y = dev(c.res) if c.res is not None else torch.zeros((c.M, c.nout), dtype=torch.int32, device="cuda")
    rm = torch.zeros(c.M, dtype=torch.int32, device="cuda") if c.rowmax else None
    E = vg.AEpi(epi=c.epi, Y=vg.ptr(Y), ldy=c.nout, Lphi=vg.ptr(lut), rowmax=vg.ptr(rm))
    if c.res is not None:
        E.residual = vg.ptr(Y)
    ws = None
    if noalloc:
        vg.k_gemm_hl2_noalloc(A, c.Mp, c.M, w, c.Kp, c.Np, c.N, c.Kp, cst, E)
    else:
        nb = vg.workspace_bytes(c.Mp, c.M, c.Np, c.N, c.Kp, c.epi)
        assert nb <= vg.NOALLOC_WS_BYTES
        if nb:
            ws = torch.empty(nb // 4 + 16, dtype=torch.int32, device="cuda")
            E.ws, E.ws_bytes = vg.ptr(ws), nb
        vg.k_gemm_hl2(A, c.Mp, c.M, w, c.Kp, c.Np, c.N, c.Kp, cst, E)
    torch.cuda.synchronize()
    return to_np(Y), (to_np(rm) if rm is not None else None)


def _conv_case(B, H, C, N, seed, **kw):
    return Case(vg.SRC_CONV16, B * H * H, N, 9 * C, seed=seed, conv=(B, H, H, C, 1), residual=True, s_range=(18, 26), **kw)


@pytest.mark.parametrize("order", ["big-then-small", "small-plain-then-split"])
def test_noalloc_matches_workspace_entry(order):
    if order == "big-then-small":
        cases = [_conv_case(8, 8, 1280, 1280, 501), _conv_case(4, 8, 1280, 640, 502, rowmax=True)]
    else:
        cases = [Case(vg.SRC_I16, 4096, 320, 320, seed=503, rowmax=True),     # no split: no workspace use
                 _conv_case(2, 8, 640, 320, 504)]
    splits = [vg.workspace_bytes(c.Mp, c.M, c.Np, c.N, c.Kp, c.epi) > 0 for c in cases]
    assert splits == ([True, True] if order == "big-then-small" else [False, True])
    for i, c in enumerate(cases):
        want, wrm = run(c, noalloc=False)
        got, grm = run(c, noalloc=True)
        assert_equal(got, want, f"{order} call {i} Y")
        if wrm is not None:
            assert_equal(grm, wrm, f"{order} call {i} rowmax")
        ref, _ = c.reference()
        assert_equal(got, ref, f"{order} call {i} vs oracle")


def test_noalloc_rejects_a_split_beyond_the_static_workspace():
    vg.set_variant(0)
    vg.set_splitk(8)
    c = Case(vg.SRC_I16, 1088, 1024, 8192, seed=505)
    assert vg.workspace_bytes(c.Mp, c.M, c.Np, c.N, c.Kp, 0) > vg.NOALLOC_WS_BYTES
    with pytest.raises(_lib.VgemmError) as ei:
        run(c, noalloc=True)
    assert ei.value.code == -3 and "static workspace" in str(ei.value)

"""GPU parity of the elementwise kernels between the GEMMs (vela_amd.elementwise over the C ABI:
k_act, k_geglu, k_add, k_concat with and without GroupNorm records, k_upsample2) against the oracle
(oracle/oracle.c: orc_act, orc_geglu_n, orc_add, orc_concat, orc_upsample2), byte for byte: both
paths of each kernel (16-byte pieces, and single elements for odd counts or 4-byte-offset buffers),
the SiLU/GELU-shaped table and a table that exercises every 32-bit wrap of lut16i, saturating
extremes, the UNet's skip-connection concatenations with records (Co = 640, 960, 1920, 2560) and
shapes whose last 256-element region is partial."""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_equal, to_np
from tests.golden import make_poisd as mp
from tests.test_gpu_norms import check_records, records_dev, records_np
from vela_amd import elementwise as ve

pytestmark = pytest.mark.gpu

IMAX, IMIN = 2**31 - 1, -(2**31)
TABLES = {"phi": mp.phi_table(), "wild": np.random.default_rng(7).integers(IMIN, IMAX, 2049, dtype=np.int64).astype(np.int32)}


def values(r, n):
    v = np.concatenate([r.integers(IMIN, IMAX, n // 2, dtype=np.int64), r.integers(-(1 << 21), 1 << 21, n - n // 2)])
    v[: min(n, 8)] = [0, IMAX, IMIN, 1 << 20, -(1 << 20), 1023, -1024, 65536][: min(n, 8)]
    return r.permutation(v).astype(np.int32)


def on_gpu(x, offset):
    """x on the device, starting `offset` int32 into its buffer (offset 1: a 4-byte misaligned view)."""
    buf = torch.zeros(x.size + offset + 4, dtype=torch.int32, device="cuda")
    buf[offset:offset + x.size] = torch.from_numpy(np.ascontiguousarray(x).reshape(-1)).cuda()
    return buf, buf[offset:offset + x.size]


@pytest.mark.parametrize("n", [1, 7, 1000, 4096, (1 << 20) + 3])
@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("table", list(TABLES))
def test_act_geglu(n, offset, table):
    r = np.random.default_rng(n + offset)
    L = TABLES[table]
    Ld = torch.from_numpy(L).cuda()
    x, g = values(r, n), values(r, n)
    buf, xd = on_gpu(x, offset)
    ve.k_act(xd, n, Ld)
    torch.cuda.synchronize()
    assert_equal(to_np(xd), oracle.act(x, L), f"act n={n} off={offset} {table}")
    assert_equal(to_np(buf[:offset]), np.zeros(offset, np.int32), "act: nothing written before the buffer")
    assert_equal(to_np(buf[offset + n:]), np.zeros(4, np.int32), "act: nothing written after the buffer")
    _, ad = on_gpu(x, offset)
    _, gd = on_gpu(g, offset)
    ve.k_geglu(ad, gd, n, Ld)
    torch.cuda.synchronize()
    assert_equal(to_np(ad), oracle.geglu_n(x, g, L), f"geglu n={n} off={offset} {table}")


@pytest.mark.parametrize("n", [1, 6, 4096, (1 << 20) + 1])
@pytest.mark.parametrize("offset", [0, 1])
def test_add(n, offset):
    r = np.random.default_rng(n)
    x, y = values(r, n), values(r, n)
    _, xd = on_gpu(x, offset)
    _, yd = on_gpu(y, 0)
    ve.k_add(xd, yd, n)
    torch.cuda.synchronize()
    assert_equal(to_np(xd), oracle.add(x, y), f"add n={n} off={offset}")


@pytest.mark.parametrize("Ca,Cb,rows", [(320, 320, 300), (3, 5, 17), (8, 24, 100), (1280, 1280, 64), (2, 30, 9)])
def test_concat(Ca, Cb, rows):
    r = np.random.default_rng(Ca * 7 + Cb + rows)
    A = values(r, rows * Ca).reshape(rows, Ca)
    B = values(r, rows * Cb).reshape(rows, Cb)
    out = torch.full((rows, Ca + Cb), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
    ve.k_concat(torch.from_numpy(A).cuda(), Ca, torch.from_numpy(B).cuda(), Cb, rows, out)
    torch.cuda.synchronize()
    assert_equal(to_np(out), oracle.concat(A, Ca, B, Cb, rows), f"concat {Ca}+{Cb} x {rows}")


# (Ca, Cb, T, rows): the UNet's up-block skip concatenations (64x64: 640 = 320 + 320, 960 = 640 + 320;
# 32x32: 1920 = 1280 + 640; 16x16: 2560), a non-16-byte split (2 + 30), rows not a multiple of T
GN_CASES = [(320, 320, 64, 128), (640, 320, 64, 192), (1280, 640, 16, 64), (1280, 1280, 4, 16), (2, 30, 8, 24), (32, 32, 8, 13)]


@pytest.mark.parametrize("Ca,Cb,T,rows", GN_CASES)
@pytest.mark.parametrize("mode", ["random", "saturated"])
def test_concat_records(Ca, Cb, T, rows, mode):
    r = np.random.default_rng(Ca + Cb + T + rows)
    A = r.integers(-(1 << 26), 1 << 26, (rows, Ca)).astype(np.int32)
    B = r.integers(-(1 << 26), 1 << 26, (rows, Cb)).astype(np.int32)
    if mode == "saturated":
        # whole groups of whole regions at INT_MAX (dropped by the flush rule), some with one value
        # just below (kept), and INT_MIN groups (always kept)
        A[: max(1, 256 // (Ca + Cb)), :] = IMAX
        A[rows // 2:, : Ca // 2] = IMAX
        A[rows // 2, 0] = IMAX - 1
        B[:, -1] = IMIN
    nsamp = (rows + T - 1) // T
    gs0 = oracle.gn_records(nsamp * 32)
    want_gs = gs0.copy()
    want = oracle.concat(A, Ca, B, Cb, rows, want_gs, T)
    gs = records_dev(gs0)
    out = torch.zeros((rows, Ca + Cb), dtype=torch.int32, device="cuda")
    ve.k_concat(torch.from_numpy(A).cuda(), Ca, torch.from_numpy(B).cuda(), Cb, rows, out, gs, T)
    torch.cuda.synchronize()
    assert_equal(to_np(out), want, f"concat+gn {Ca}+{Cb} T={T} rows={rows}")
    check_records(records_np(gs), want_gs, f"concat records {Ca}+{Cb} {mode}", fields=("sum", "mn", "mx"))


@pytest.mark.parametrize("B,H,W,C", [(2, 3, 5, 7), (8, 8, 8, 1280), (2, 16, 16, 640), (1, 2, 2, 4), (3, 1, 1, 3)])
def test_upsample2(B, H, W, C):
    X = np.random.default_rng(B + H + W + C).integers(IMIN, IMAX, (B, H, W, C), dtype=np.int64).astype(np.int32)
    out = torch.full((B, 2 * H, 2 * W, C), 7, dtype=torch.int32, device="cuda")
    ve.k_upsample2(torch.from_numpy(X).cuda(), B, H, W, C, out)
    torch.cuda.synchronize()
    assert_equal(to_np(out), oracle.upsample2(X, B, H, W, C), f"upsample2 {B}x{H}x{W}x{C}")

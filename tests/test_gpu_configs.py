"""BASELINE.json configurations at full size on the GPU, bit-exact against the CPU oracle.

C1-C4 are compared on every output element (and rowmax). C5, the 194-GEMM UNet set, runs as one
captured hipGraph; each layer is then checked on three row blocks (first, last, seeded) -- every
output row depends on its own A row only, so sampled rows are an exact check of those rows -- and a
second replay must reproduce the first bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_equal, to_np
from vela_amd import configs as cf
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu

CONFIGS = [cf.c1(), cf.c2(cf.EPI_GEGLU), cf.c2(cf.EPI_PLAIN), cf.c3(), *cf.c4()]


@pytest.mark.parametrize("L", CONFIGS, ids=[L.name for L in CONFIGS])
def test_config_full(gpu, L):
    p = cf.DeviceProblem(L)
    p.reset()
    p.run()
    torch.cuda.synchronize()
    want, wrm = oracle.layer_reference(L, p.h)
    assert_equal(to_np(p.y), want, L.name)
    if wrm is not None:
        assert_equal(to_np(p.rowmax).view(np.uint32), wrm, L.name + " rowmax")


ORDER_CONFIGS = [cf.c1(), cf.c3(), *cf.c4()]


@pytest.mark.parametrize("L", ORDER_CONFIGS, ids=[L.name for L in ORDER_CONFIGS])
def test_config_tile_orders(gpu, L):
    """Both tile orders over the XCDs (row stripes per XCD, column groups per XCD) give the oracle's
    bits: the order only renumbers blocks, with and without split-K."""
    p = cf.DeviceProblem(L)
    want = None
    try:
        for order in (0, 1):
            vg.set_tile_order(order)
            p.reset()
            p.run()
            torch.cuda.synchronize()
            if want is None:
                want, _ = oracle.layer_reference(L, p.h)
            assert_equal(to_np(p.y), want, f"{L.name} tile order {order}")
    finally:
        vg.set_tile_order(-1)


def test_config_e_path(gpu):
    """C1 shape with per-row shifts e in [0, 17] (the int16 view of rows quantised with e > 0)."""
    L = cf.Layer("C1 with e", "linear", 4096, 320, 320, e_bits=17, seed=cf.SEED0 + 11)
    p = cf.DeviceProblem(L)
    p.reset()
    p.run()
    torch.cuda.synchronize()
    want, _ = oracle.layer_reference(L, p.h)
    assert_equal(to_np(p.y), want, L.name)


def check_layer(gs, i: int, rows_per_block: int = 16, seed: int = 0) -> None:
    """Bit-exact check of layer i of a captured GEMM set on three row blocks (first, last and one
    seeded block; every output row depends on its own A row only) against the CPU oracle."""
    p = gs.probs[i]
    L = p.L
    h = cf.make_host(L)
    r = np.random.default_rng(seed + i)
    starts = sorted({0, max(0, L.M - rows_per_block), int(r.integers(0, max(1, L.M - rows_per_block)))})
    y = to_np(p.y)
    rm = to_np(p.rowmax).view(np.uint32) if p.rowmax is not None else None
    for s0 in starts:
        rows = (s0, min(L.M, s0 + rows_per_block))
        want, wrm = oracle.layer_reference(L, h, rows=rows)
        assert_equal(y[rows[0]:rows[1]], want[rows[0]:rows[1]], f"layer {i} {L.name} rows {rows}")
        if rm is not None:
            assert_equal(rm[rows[0]:rows[1]], wrm[rows[0]:rows[1]], f"layer {i} {L.name} rowmax rows {rows}")


def test_unet_conv_in_full(gpu):
    """conv_in runs as in the reference (src/engine.cu:458, 254-280): k_pixmax, k_im2col3 and the GEMM
    on the int8 planes, all on the GPU; every output element against the oracle."""
    L = cf.unet_layers()[0]
    assert L.kind == "conv_in"
    p = cf.DeviceProblem(L)
    p.reset()
    p.run()
    torch.cuda.synchronize()
    want, _ = oracle.layer_reference(L, p.h)
    assert_equal(to_np(p.y), want, L.name)
    assert to_np(p.e_in)[:L.M].max() > 0, "the image must exercise per-row shifts"


def test_unet_gemm_set_graph(gpu):
    from vela_amd.unet import GemmSet

    gs = GemmSet()
    assert len(gs.layers) == 194
    gs.capture()
    gs.replay()
    gs.stream.synchronize()
    first = [to_np(p.y).copy() for p in gs.probs]
    for i in range(len(gs.layers)):
        check_layer(gs, i)
    gs.replay()
    gs.stream.synchronize()
    for i, p in enumerate(gs.probs):
        assert_equal(to_np(p.y), first[i], f"replay 2 layer {i}")

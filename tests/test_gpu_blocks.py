"""GPU parity of the engine blocks (vela_amd.engine over include/vgemm_engine.h: Engine::resnet,
Engine::transformer and the cross-attention K/V of setPrompt, src/engine.cu:389-454,540-560) against
their composition from the oracle (tests/oracle_blocks.py), byte for byte: the block outputs and,
with gnFuse, the GroupNorm records the last GEMM of each block gathers. Resnet A (64 -> 128 channels,
1x1 shortcut) feeds resnet B (128 -> 128, the input as residual), whose output and records feed a
transformer of 2 heads (C = 128, GEGLU width 256, a context of 77 tokens of 96 channels per sample).
Shapes: 16 x 16 (every GroupNorm record path fusable), 8 x 8 with 3 samples, 12 x 12 (T = 144: not
fusable, 144 query rows padded to 256 / 192 for the attention operands). Each block also runs as one
captured hipGraph, replayed with the inputs changed between replays, every replay checked."""
import numpy as np
import pytest
import torch

from tests.conftest import assert_equal, to_np
from tests.golden import make_poisd as mp
from tests.oracle_blocks import Act, OracleEngine
from tests.test_gpu_norms import check_records, records_np
from vela_amd import gemm as vg
from vela_amd.engine import Engine
from vela_amd.model import DevModel, Poisd

pytestmark = pytest.mark.gpu

BLOCK = mp.XF + ".transformer_blocks.0"
ARENA = 64 << 20
SHAPES = [(2, 16, 16), (3, 8, 8), (1, 12, 12)]
TC = 77


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    path = tmp_path_factory.mktemp("blocks") / "blocks.poisd"
    data = mp.encode(mp.block_tensors())
    path.write_bytes(data)
    return path, data


@pytest.fixture(scope="module")
def dev_model(model_file):
    m = Poisd()
    m.load(str(model_file[0]))
    dm = DevModel()
    dm.load(0, m)
    yield dm
    m.close()


def inputs(seed, B, T, C, scale=65536):
    r = np.random.default_rng(seed)
    return (r.standard_normal((B * T, C)) * scale).astype(np.int32)


def run_chain(eng, x_d, ctx_d, B, H, W, outs, stream=None):
    """resnet A -> resnet B -> transformer on the device (outs: yA, yB, yX and their records)."""
    yA, yB, yX, gA, gB, gX = outs
    fA = eng.resnet(x_d, B, H, W, mp.RESNET_A, yA, out_gnst=gA, stream=stream)
    fB = eng.resnet(yA, B, H, W, mp.RESNET_B, yB, out_gnst=gB, x_gnst=gA if fA else None, stream=stream)
    fX = eng.transformer(yB, B, H * W, mp.XF, mp.XF_HEADS, yX, out_gnst=gX, x_gnst=gB if fB else None, stream=stream)
    return fA, fB, fX


def oracle_chain(oe, x, ctx, B, H, W):
    T = H * W
    oe.set_context(Act(ctx, B, TC), BLOCK, mp.XF_HEADS)
    a = oe.resnet(Act(x, B, T), H, W, mp.RESNET_A)
    b = oe.resnet(a, H, W, mp.RESNET_B)
    c = oe.transformer(b, mp.XF, mp.XF_HEADS)
    return a, b, c


def alloc_outs(B, T):
    z = lambda C: torch.zeros((B * T, C), dtype=torch.int32, device="cuda")
    return (z(128), z(128), z(128), Engine.records(B), Engine.records(B), Engine.records(B))


def check_chain(got, want, fused, what):
    yA, yB, yX, gA, gB, gX = got
    for name, y, w, f, g in (("resnet A", yA, want[0], fused[0], gA), ("resnet B", yB, want[1], fused[1], gB),
                             ("transformer", yX, want[2], fused[2], gX)):
        assert_equal(to_np(y), w.d, f"{what}: {name} output")
        assert f == (w.gs is not None), f"{what}: {name} record path"
        if f:
            check_records(records_np(g), w.gs, f"{what}: {name} records", fields=("sum", "mn", "mx"))


@pytest.mark.parametrize("B,H,W", SHAPES)
@pytest.mark.parametrize("gn_fuse", [False, True])
def test_blocks_eager(dev_model, model_file, B, H, W, gn_fuse):
    T = H * W
    x = inputs(B * 100 + H, B, T, 64)
    ctx = inputs(B * 7 + 1, B, TC, mp.CTX_C)
    oe = OracleEngine(model_file[1], gn_fuse)
    want = oracle_chain(oe, x, ctx, B, H, W)
    eng = Engine(dev_model, ARENA, gn_fuse)
    eng.set_context(torch.from_numpy(ctx).cuda(), B, TC, BLOCK, mp.XF_HEADS)
    outs = alloc_outs(B, T)
    fused = run_chain(eng, torch.from_numpy(x).cuda(), None, B, H, W, outs)
    torch.cuda.synchronize()
    check_chain(outs, want, fused, f"eager B={B} {H}x{W} gn_fuse={gn_fuse}")
    assert 0 < eng.arena_peak <= ARENA
    eng.close()


@pytest.mark.parametrize("B,H,W", [(2, 16, 16), (1, 12, 12)])
@pytest.mark.parametrize("block", ["resnet", "transformer"])
def test_block_graph(dev_model, model_file, B, H, W, block):
    """One block captured as one hipGraph: replays against the oracle, with new inputs copied into the
    captured input buffer between replays and eager work of the program in between."""
    T = H * W
    gn_fuse = True
    eng = Engine(dev_model, ARENA, gn_fuse)
    oe = OracleEngine(model_file[1], gn_fuse)
    ctx = inputs(5, B, TC, mp.CTX_C)
    eng.set_context(torch.from_numpy(ctx).cuda(), B, TC, BLOCK, mp.XF_HEADS)
    oe.set_context(Act(ctx, B, TC), BLOCK, mp.XF_HEADS)
    Cin = 64 if block == "resnet" else 128
    x_d = torch.zeros((B * T, Cin), dtype=torch.int32, device="cuda")
    y_d = torch.zeros((B * T, 128), dtype=torch.int32, device="cuda")
    g_d = Engine.records(B)
    s = torch.cuda.Stream()
    g = vg.Graph(s)
    torch.cuda.synchronize()
    g.begin()
    if block == "resnet":
        fused = eng.resnet(x_d, B, H, W, mp.RESNET_A, y_d, out_gnst=g_d, stream=s)
    else:
        fused = eng.transformer(x_d, B, T, mp.XF, mp.XF_HEADS, y_d, out_gnst=g_d, stream=s)
    g.end()
    for rep in range(3):
        x = inputs(1000 + rep, B, T, Cin)
        x_d.copy_(torch.from_numpy(x).cuda())
        _ = (x_d.float() * 2).sum()   # eager work of the program between replays
        torch.cuda.synchronize()
        g.replay()
        s.synchronize()
        w = oe.resnet(Act(x, B, T), H, W, mp.RESNET_A) if block == "resnet" else oe.transformer(Act(x, B, T), mp.XF, mp.XF_HEADS)
        assert_equal(to_np(y_d), w.d, f"graph {block} replay {rep} B={B} {H}x{W}")
        assert fused == (w.gs is not None)
        if fused:
            check_records(records_np(g_d), w.gs, f"graph {block} replay {rep} records", fields=("sum", "mn", "mx"))
    g.destroy()
    eng.close()


def test_block_errors(dev_model):
    from vela_amd._lib import VgemmError
    eng = Engine(dev_model, 1 << 16, False)   # too small an arena
    x = torch.zeros((2 * 64, 64), dtype=torch.int32, device="cuda")
    y = torch.zeros((2 * 64, 128), dtype=torch.int32, device="cuda")
    with pytest.raises(VgemmError, match="arena too small"):
        eng.resnet(x, 2, 8, 8, mp.RESNET_A, y)
    eng.close()
    eng = Engine(dev_model, ARENA, False)
    with pytest.raises(VgemmError, match="no linear"):
        eng.resnet(x, 2, 8, 8, "unet.down_blocks.9.resnets.0", y)
    with pytest.raises(VgemmError, match="no cross KV"):
        eng.transformer(y, 2, 64, mp.XF, mp.XF_HEADS, torch.zeros_like(y))
    ctx = torch.zeros((1 * TC, mp.CTX_C), dtype=torch.int32, device="cuda")
    eng.set_context(ctx, 1, TC, BLOCK, mp.XF_HEADS)
    with pytest.raises(VgemmError, match="another batch"):
        eng.transformer(y, 2, 64, mp.XF, mp.XF_HEADS, torch.zeros_like(y))
    with pytest.raises(VgemmError, match="groupnormSilu: C mismatch|conv3: shape mismatch"):
        eng.resnet(y, 2, 8, 8, mp.RESNET_A, y.clone())
    torch.cuda.synchronize()
    eng.close()

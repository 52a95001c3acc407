"""Host-side logic without a GPU: the seeded input generator, the BASELINE configurations and their
algorithmic work, the 194-GEMM UNet set, and bench.py's refusal of several GPUs."""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from vela_amd import configs as cf
from vela_amd import datagen as dg

ROOT = Path(__file__).resolve().parent.parent


def test_generator_is_deterministic_and_chunked():
    """splitmix64-seeded xoshiro256** streams: a pure function of (n, seed), different per seed, and
    a call's prefix equals the shorter call (one stream per 65536-element chunk)."""
    a = dg.i32_uniform(200000, 7, -(2**31), 2**31 - 1)
    b = dg.i32_uniform(200000, 7, -(2**31), 2**31 - 1)
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, dg.i32_uniform(200000, 8, -(2**31), 2**31 - 1))
    # a prefix of a longer call is the shorter call (chunked streams)
    np.testing.assert_array_equal(dg.i32_uniform(70000, 7, -(2**31), 2**31 - 1), a[:70000])


def test_distributions():
    g = dg.i16_gauss(400000, 1, 2000.0).astype(np.float64)
    assert abs(g.mean()) < 20 and abs(g.std() - 2000) < 20
    lap = dg.i16_laplace(400000, 2, 1500.0).astype(np.float64)
    assert abs(np.abs(lap).mean() - 1500) < 20           # E|x| = b for Laplace(b)
    assert lap.min() >= -32767 and lap.max() <= 32767
    w = dg.i8_gauss(400000, 3, 40.0).astype(np.float64)
    assert abs(w.std() - 40) < 1.0 and w.min() >= -127 and w.max() <= 127
    u = dg.i8_uniform(400000, 4, -127, 127)
    assert u.min() == -127 and u.max() == 127 and abs(u.astype(np.float64).mean()) < 0.5
    c = dg.i16_gauss(100000, 5, 30000.0)
    assert c.min() == -32767 and c.max() == 32767          # clipped to +-32767
    bits = dg.i32_bits(200000, 6)
    assert np.abs(bits.astype(np.int64)).max() >= 2**29


def test_phi_lut_is_a_monotone_q16_table():
    L = cf.phi_lut()
    assert L.shape == (2049,) and L.dtype == np.int32
    assert L[0] == 0 and L[-1] == 65536 and L[1024] == 32768
    assert np.all(np.diff(L) >= 0)


def test_config_work_matches_the_published_table():
    """ops = 4 M N K and the algorithmic HBM bytes of each configuration."""
    expect = {  # name prefix: (ops in G, bytes in MB)
        "C1": (1.68, 7.97),
        "C2 GEGLU": (107.4, 189.7),
        "C2 plain": (107.4, 357.5),
        "C3": (120.8, 35.2),
    }
    layers = [cf.c1(), cf.c2(cf.EPI_GEGLU), cf.c2(cf.EPI_PLAIN), cf.c3()]
    for L in layers:
        key = next(k for k in expect if L.name.startswith(k))
        ops, mb = expect[key]
        assert L.ops / 1e9 == pytest.approx(ops, rel=0.005), L.name
        assert L.hbm_bytes / 1e6 == pytest.approx(mb, rel=0.01), L.name
    c4 = cf.c4()
    assert [(L.M, L.K, L.N) for L in c4] == [(2048, 11520, 1280), (512, 11520, 1280), (616, 1024, 1280)]


def test_unet_gemm_set():
    layers = cf.unet_layers()
    assert len(layers) == 194
    assert sum(L.ops for L in layers) / 1e12 == pytest.approx(10.787, rel=0.001)
    kinds = {}
    for L in layers:
        kinds[L.kind] = kinds.get(L.kind, 0) + 1
        assert L.Kp % 16 == 0 and L.Np % 64 == 0
        if L.kind == "conv":
            assert L.K == 9 * L.C and L.C % 8 == 0
    assert kinds["conv"] > 40 and kinds["linear"] > 100
    assert sum(L.epi == cf.EPI_GEGLU for L in layers) == 16


def test_make_host_is_deterministic_and_padded():
    L = cf.Layer("t", "linear", 100, 40, 70, seed=cf.SEED0 + 77)
    h1, h2 = cf.make_host(L), cf.make_host(L)
    for k in ("a", "w", "cst"):
        np.testing.assert_array_equal(h1[k], h2[k])
    w, cst = h1["w"], h1["cst"]
    assert w.shape == (128, 48) and not w[70:].any() and not w[:, 40:].any()
    np.testing.assert_array_equal(cst[70:], np.tile([1, 0, 0, 0], (58, 1)))
    np.testing.assert_array_equal(cst[:70, 3], w[:70].astype(np.int64).sum(1))
    assert cst[:70, 1].min() >= 16 and cst[:70, 1].max() <= 24


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr

"""Seeded random GPU parity cases of vgemm_hl2 against the CPU oracle, byte for byte.

Each case draws its A source, epilogue, shape, tile variant (including the row-stationary kernel,
variant 4), per-row shifts, residual, row maximum and requantisation ranges at random within what
the call accepts (src/gemm_hl.h:12-26; the int16 sources of this library included), so that
combinations the structured tests do not list are also checked. The draw is fixed by the seed, and
each case prints its parameters before it runs.
"""
import numpy as np
import pytest

from tests.test_gpu_gemm import Case
from vela_amd import gemm as vg

pytestmark = pytest.mark.gpu

S_RANGES = [(16, 24), (20, 29), (4, 30), (-3, 8), (30, 45)]
M_RANGES = [(1 << 14, 1 << 15), (1, 1 << 10), (1 << 20, 1 << 22), ((1 << 30), (1 << 31) - 1)]


def draw(seed):
    r = np.random.default_rng(10_000 + seed)
    src = int(r.choice([vg.SRC_I8, vg.SRC_I16, vg.SRC_X32, vg.SRC_CONV16, vg.SRC_CONV32]))
    epi = int(r.choice([vg.EPI_PLAIN, vg.EPI_PLAIN, vg.EPI_GEGLU, vg.EPI_GELU, vg.EPI_SPLIT3]))
    variant = int(r.choice([-1, -1, 0, 1, 2, 3, 4]))
    kw = dict(s_range=S_RANGES[int(r.integers(len(S_RANGES)))], m_range=M_RANGES[int(r.integers(len(M_RANGES)))])
    if int(r.integers(4)) == 0:
        kw["b_range"] = (-(2**31), 2**31)
    conv = None
    if src in (vg.SRC_CONV16, vg.SRC_CONV32):
        C = int(r.choice([16, 32, 48, 64, 128] if src == vg.SRC_CONV16 else [16, 32, 64]))
        B, H, W, stride = int(r.integers(1, 4)), int(r.integers(2, 20)), int(r.integers(2, 20)), int(r.choice([1, 1, 2]))
        conv = (B, H, W, C, stride)
        M = B * ((H - 1) // stride + 1) * ((W - 1) // stride + 1)
        K = 9 * C
    else:
        M = int(r.integers(1, 700))
        K = int(r.integers(1, 90)) * (8 if src == vg.SRC_I16 else 4 if src == vg.SRC_X32 else 1) * int(r.choice([1, 4, 8]))
        K = max(K, 8)
        if src == vg.SRC_I16:
            K = (K + 7) // 8 * 8
        elif src == vg.SRC_X32:
            K = (K + 3) // 4 * 4
    if epi == vg.EPI_SPLIT3:
        Cs = int(r.integers(1, 60)) * 4
        N = int(r.integers(1, 3 * Cs + 1))
        kw["Cs"] = Cs
    else:
        N = int(r.integers(1, 130)) * (8 if epi == vg.EPI_GEGLU else 4)
        kw["rowmax"] = bool(r.integers(2))
        kw["residual"] = epi != vg.EPI_GEGLU and bool(r.integers(2))
    if src in (vg.SRC_I8, vg.SRC_I16) and int(r.integers(2)):
        kw["e_max"] = int(r.integers(1, 12))
    splitk = int(r.choice([0, 0, 0, 2, 3, 5]))   # forced K splits (with a workspace), 0: none
    return src, epi, variant, M, N, K, conv, kw, splitk


@pytest.mark.parametrize("seed", range(128))
def test_random_case(seed):
    src, epi, variant, M, N, K, conv, kw, splitk = draw(seed)
    what = f"seed {seed}: src {src} epi {epi} variant {variant} splitk {splitk} M {M} N {N} K {K} conv {conv} {kw}"
    print(f"[random] {what}", flush=True)
    vg.set_variant(variant)
    vg.set_splitk(splitk)
    try:
        c = Case(src, M, N, K, epi=epi, seed=seed, conv=conv, **kw)
        ws = vg.workspace_bytes(c.Mp, M, c.Np, N, c.Kp, epi) if splitk else 0
        c.check(ws_bytes=ws, what=what)
    finally:
        vg.set_variant(-1)
        vg.set_splitk(0)


def draw_qkv(seed):
    r = np.random.default_rng(20_000 + seed)
    src = int(r.choice([vg.SRC_I8, vg.SRC_I16, vg.SRC_X32]))
    heads, T, B = int(r.integers(1, 7)), int(r.integers(1, 300)), int(r.integers(1, 4))
    K = int(r.integers(1, 40)) * 8 * int(r.choice([1, 4]))
    kw = dict(s_range=S_RANGES[int(r.integers(len(S_RANGES)))], m_range=M_RANGES[int(r.integers(len(M_RANGES)))])
    if src != vg.SRC_X32 and int(r.integers(2)):
        kw["e_max"] = int(r.integers(1, 12))
    return src, heads, T, B, K, int(r.choice([-1, 0, 1, 2, 3, 4])), kw


@pytest.mark.parametrize("seed", range(24))
def test_random_qkv(seed):
    from tests.test_gpu_qkv_gn import check_qkv

    src, heads, T, B, K, variant, kw = draw_qkv(seed)
    print(f"[random qkv] seed {seed}: src {src} heads {heads} T {T} B {B} K {K} variant {variant} {kw}", flush=True)
    try:
        check_qkv(src, heads, T, B=B, K=K, seed=seed, variant=variant, **kw)
    finally:
        vg.set_variant(-1)


# (B, H, W, C, stride) with Ho * Wo a multiple of 64, for the GroupNorm sample length
GN_CONV = [(2, 8, 8, 16, 1), (1, 16, 16, 32, 2), (3, 8, 16, 64, 1), (1, 16, 16, 64, 1), (2, 32, 8, 16, 1)]


def draw_gn(seed):
    r = np.random.default_rng(30_000 + seed)
    src = int(r.choice([vg.SRC_I8, vg.SRC_I16, vg.SRC_X32, vg.SRC_CONV16, vg.SRC_CONV32]))
    N = int(r.integers(1, 20)) * 32
    kw = dict(s_range=S_RANGES[int(r.integers(len(S_RANGES)))], m_range=M_RANGES[int(r.integers(len(M_RANGES)))],
              residual=bool(r.integers(2)), rowmax=bool(r.integers(2)))
    conv = None
    if src in (vg.SRC_CONV16, vg.SRC_CONV32):
        conv = GN_CONV[int(r.integers(len(GN_CONV)))]
        if src == vg.SRC_CONV32 and conv[3] % 16:
            conv = conv[:3] + (32,) + conv[4:]
        B, H, W, C, stride = conv
        T = ((H - 1) // stride + 1) * ((W - 1) // stride + 1)
        M, K = B * T, 9 * C
    else:
        T = 64 * int(r.integers(1, 6))
        M = T * int(r.integers(1, 4))
        K = int(r.integers(1, 40)) * 8 * int(r.choice([1, 4]))
        if src != vg.SRC_X32 and int(r.integers(2)):
            kw["e_max"] = int(r.integers(1, 12))
    return src, M, N, K, T, conv, int(r.choice([-1, 0, 1, 2, 3, 4])), kw


@pytest.mark.parametrize("seed", range(24))
def test_random_gnstat(seed):
    from tests.test_gpu_qkv_gn import check_gn

    src, M, N, K, T, conv, variant, kw = draw_gn(seed)
    what = f"seed {seed}: src {src} M {M} N {N} K {K} T {T} conv {conv} variant {variant} {kw}"
    print(f"[random gn] {what}", flush=True)
    vg.set_variant(variant)
    try:
        check_gn(Case(src, M, N, K, seed=seed, conv=conv, **kw), T, what)
    finally:
        vg.set_variant(-1)

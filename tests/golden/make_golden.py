"""Writes the golden fixtures of tests/golden/*.npz.

The reference holds no stored GEMM vectors (its GEMM test is differential against cuBLASLt), so the
expected outputs here come from tests/refmath.py -- the path's integer semantics restated from their
definitions with exact rationals and a single q.W product -- not from the oracle or the GPU library.
Inputs are small, seeded, and include the edge values of src/test_attn_score.cu:14, saturating
requantisation constants, a left shift, per-row shifts up to 17, and image borders.

Each .npz holds plain numeric arrays (no pickles): the inputs, `Y` (and `rowmax` where the epilogue
writes it) and the scalar parameters as 0-d arrays. Run: python -m tests.golden.make_golden
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from tests import refmath as rm  # noqa: E402

EDGES = [-32767, -32766, -32513, -256, -255, -128, -1, 0, 1, 127, 128, 255, 256, 32512, 32766, 32767]


def cst_for(r, w_real, N):
    cst = np.zeros((N, 4), np.int32)
    cst[:, 0] = r.integers(1 << 14, 1 << 15, N)
    cst[:, 1] = r.integers(16, 25, N)
    cst[:, 2] = r.integers(-50000, 50000, N)
    cst[:, 3] = w_real.astype(np.int64).sum(1)
    # requantisation corner cases on the first columns
    cst[0] = [2**31 - 1, 30, 2**31 - 1, cst[0, 3]]    # saturates high through b
    cst[1] = [-(2**31), 44, -(2**31), cst[1, 3]]      # negative multiplier, saturates low
    cst[2] = [3, -2, 0, cst[2, 3]]                    # left shift
    cst[3] = [1, 0, 0, cst[3, 3]]                     # identity requantisation
    return cst


def ramp_lut():
    """A monotone Q16 table: a clipped ramp over the 2049 grid points."""
    return np.clip((np.arange(2049) - 512) * 64, 0, 65536).astype(np.int32)


def linear_case(name, epi, K=48, M=5, N=8, e_max=0, seed=1):
    r = np.random.default_rng(seed)
    q = r.integers(-32768, 32768, (M, K)).astype(np.int16)
    q[0, :16] = EDGES
    q[1, :] = 32767
    q[2, :] = -32768
    w = r.integers(-128, 128, (N, K)).astype(np.int8)
    w[1, :] = 127
    w[2, :] = -128
    cst = cst_for(r, w, N)
    e = r.integers(0, e_max + 1, M).astype(np.int32) if e_max else np.zeros(M, np.int32)
    L = ramp_lut()
    nout = N // 2 if epi == "geglu" else N
    res = r.integers(-(2**31), 2**31, (M, nout), dtype=np.int64).astype(np.int32) if epi == "plain" else None
    rowmax0 = np.zeros(M, np.uint32)
    Y, rowmax = rm.gemm(q, w, cst, e=e, epi=epi, residual=res, L=L, rowmax=rowmax0)
    out = dict(q16=q, w=w, cst=cst, e=e, Lphi=L, Y=Y, rowmax=rowmax, K=np.array(K), epi=np.array(epi))
    if res is not None:
        out["residual"] = res
    np.savez(HERE / f"{name}.npz", **out)


def x32_case(name, seed=3):
    r = np.random.default_rng(seed)
    M, N, K = 6, 8, 32
    bits = r.integers(1, 32, (M, 1))
    bits[0] = 31
    x = ((r.integers(0, 2**31, (M, K), dtype=np.int64) & ((1 << bits) - 1)) - (1 << (bits - 1))).astype(np.int32)
    x[0, 0] = -(2**31)
    xrm = np.abs(x.astype(np.int64)).max(1).astype(np.uint32)
    w = r.integers(-127, 128, (N, K)).astype(np.int8)
    cst = cst_for(r, w, N)
    e = np.array([rm.row_exp(int(v)) for v in xrm], np.int32)
    Y, _ = rm.gemm(rm.quant_matrix(x, e), w, cst, e=e)
    np.savez(HERE / f"{name}.npz", x=x, xrowmax=xrm, w=w, cst=cst, Y=Y, e_expected=e, K=np.array(K))


def conv_case(name, src, B, H, W, C, stride, seed):
    r = np.random.default_rng(seed)
    N = 8
    if src == "conv32":
        bits = r.integers(1, 32, (B, H, W, 1))
        img = ((r.integers(0, 2**31, (B, H, W, C), dtype=np.int64) & ((1 << bits) - 1)) - (1 << (bits - 1))).astype(np.int32)
    else:
        img = r.integers(-32768, 32768, (B, H, W, C)).astype(np.int16)
        img[0, 0, 0, :4] = [-32768, 32767, 0, -1]
    w_nchw = r.integers(-127, 128, (N, C, 3, 3)).astype(np.int8)
    w_tm = rm.tapmajor_weights(w_nchw)
    cst = cst_for(r, w_tm, N)
    e = rm.conv_row_exp(img, stride)
    q = rm.quant_matrix(rm.im2col_tapmajor(img, stride), e)
    Y, _ = rm.gemm(q, w_tm, cst, e=e)
    np.savez(HERE / f"{name}.npz", img=img, w_nchw=w_nchw, w_tapmajor=w_tm, cst=cst, e=e, Y=Y,
             geom=np.array([B, H, W, C, stride]))


def main():
    linear_case("i16_plain_edges", "plain", e_max=17, seed=1)
    linear_case("i16_geglu", "geglu", seed=2)
    linear_case("i16_gelu", "gelu", K=32, seed=4)
    x32_case("x32_rowexp")
    conv_case("conv16_s1", "conv16", 1, 3, 4, 16, 1, seed=5)
    conv_case("conv32_s2", "conv32", 2, 5, 3, 16, 2, seed=6)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()

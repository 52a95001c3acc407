"""Independent statements of the path's integer semantics, from their mathematical definitions.

These checkers share no code or structure with the oracle (oracle/oracle.c): rounding is done with
exact rationals (Python integers), the GEMM is a single q.W product over the full 16-bit values (no
hi/lo planes, no column-sum correction), the 3x3 im2col is built from a zero-padded image by array
slicing, and the conv weight permutation is a transpose of PyTorch's [N, C, 3, 3] layout. A
mistake in the oracle's split, correction, shift or index arithmetic therefore shows up as a
disagreement with these definitions.

Definitions (reference file:line of the statement each one encodes):
  sat32(v)      clamp to [-2^31, 2^31 - 1]                                  src/intops.cuh:9
  rshr(v, s)    s >= 0: v / 2^min(s,62) rounded half up; s < 0: v * 2^min(-s,31); then sat32
                                                                             src/intops.cuh:10-17
  row_exp(m)    smallest e in [0, 17] with m < 32768 * 2^e (else 17)         src/test_im2col.cu:34
  quant16(v,e)  rshr(v, e) clamped to [-32767, 32767]                        src/intops.cuh:39
  lut(x, L)     linear interpolation of L at (x + 2^20) / 2^10 with the fraction floored, 0 below
                the table and 65536 at or above its end                      src/intops.cuh:42-50
  y             sat32(rshr((q . w) * m, s - e) + b), (+ residual, saturated) src/gemm_hl.h:1-3
  GEGLU         sat32(rshr(a * sat32(rshr(g * lut(g), 16)), 16))             src/gemm_hl.cu:292-293
  GELU          sat32(rshr(y * lut(y), 16))                                  src/gemm_hl.cu:280
The *_dev forms restate what the reference's fixed-width code computes where its int64 product
acc * m or its int32 table interpolation overflows: two's-complement wrapping, as the GPU executing
it does (rshr_dev, epi1_dev, lut_dev, geglu_dev, gelu_dev).
"""
from __future__ import annotations

from fractions import Fraction
import math

import numpy as np

I32_MIN, I32_MAX = -(2**31), 2**31 - 1


def sat32(v: int) -> int:
    return min(max(int(v), I32_MIN), I32_MAX)


def round_half_up(x: Fraction) -> int:
    return math.floor(x + Fraction(1, 2))


def rshr(v: int, s: int) -> int:
    """For |v| + 2^(p-1) < 2^63 (the range in which the reference's int64 add does not wrap)."""
    v, s = int(v), int(s)
    if s >= 0:
        return sat32(round_half_up(Fraction(v, 2 ** min(s, 62))))
    return sat32(v * 2 ** min(-s, 31))


def wrap64(x: int) -> int:
    """x reduced to a two's-complement int64 (what the device's 64-bit arithmetic keeps)."""
    x = int(x) & (2**64 - 1)
    return x - 2**64 if x >= 2**63 else x


def wrap32(x: int) -> int:
    x = int(x) & (2**32 - 1)
    return x - 2**32 if x >= 2**31 else x


def rshr_dev(v: int, s: int) -> int:
    """rshr as the reference's int64 code evaluates it for any int64 v: the product v arrives
    wrapped to 64 bits and the rounding add v + 2^(p-1) wraps too (src/intops.cuh:11-13); equal to
    rshr() wherever neither wraps."""
    v, s = wrap64(v), int(s)
    if s >= 0:
        p = min(s, 62)
        t = wrap64(v + ((1 << p) >> 1))
        return sat32(t >> p)          # Python's >> on ints is the arithmetic (floor) shift
    neg = min(-s, 31)
    lim = 1 << (62 - neg)
    return sat32(min(max(v, -lim), lim) << neg)


def epi1_dev(acc: int, m: int, s: int, e: int, b: int) -> int:
    """y = sat32(rshr(acc * m, s - e) + b) with the int64 product acc * m wrapping
    (src/gemm_hl.cu:40-43: `acc * c.x` on int64)."""
    return sat32(rshr_dev(wrap64(int(acc) * int(m)), int(s) - int(e)) + int(b))


def lut_dev(x: int, L) -> int:
    """lut16i as its int32 code evaluates it for any table: b - a, (b - a) * f and a + (.. >> 10)
    all wrap to 32 bits (src/intops.cuh:42-50); equal to lut() when nothing wraps."""
    z = int(x) + (16 << 16)
    if z < 0:
        return 0
    if z >= (32 << 16):
        return 65536
    i, f = z >> 10, z & 1023
    a, b = int(L[i]), int(L[i + 1])
    prod = wrap32(wrap32(b - a) * f)
    return wrap32(a + (prod >> 10))


def geglu_dev(a: int, g: int, L) -> int:
    return sat32(rshr_dev(int(a) * sat32(rshr_dev(int(g) * lut_dev(g, L), 16)), 16))


def gelu_dev(y: int, L) -> int:
    return sat32(rshr_dev(int(y) * lut_dev(y, L), 16))


def row_exp(m: int) -> int:
    e = 0
    while e < 17 and m >= (32768 << e):
        e += 1
    return e


def quant16(v: int, e: int) -> int:
    return min(max(rshr(v, e), -32767), 32767)


def lut(x: int, L) -> int:
    z = int(x) + (16 << 16)
    if z < 0:
        return 0
    if z >= (32 << 16):
        return 65536
    i, f = divmod(z, 1024)
    a, b = int(L[i]), int(L[i + 1])
    return a + math.floor(Fraction((b - a) * f, 1024))


def geglu(a: int, g: int, L) -> int:
    return sat32(rshr(a * sat32(rshr(g * lut(g, L), 16)), 16))


def gelu(y: int, L) -> int:
    return sat32(rshr(y * lut(y, L), 16))


def dot_rows(q: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact integer q @ w.T as Python integers (object array)."""
    return np.asarray(q, dtype=object) @ np.asarray(w, dtype=object).T


def requant(acc: np.ndarray, cst: np.ndarray, e: np.ndarray | None) -> np.ndarray:
    """y[r, n] = sat32(rshr(acc[r, n] * m[n], s[n] - e[r]) + b[n]) over Python integers."""
    M, N = acc.shape
    y = np.zeros((M, N), dtype=object)
    for r in range(M):
        er = 0 if e is None else int(e[r])
        for n in range(N):
            m, s, b = int(cst[n][0]), int(cst[n][1]), int(cst[n][2])
            y[r, n] = sat32(rshr(int(acc[r, n]) * m, s - er) + b)
    return y


def gemm(q: np.ndarray, w_real: np.ndarray, cst: np.ndarray, e=None, epi="plain", residual=None, L=None, rowmax=None,
         Cs=0):
    """The fused-epilogue GEMM over 16-bit activations q [M x K] and int8 weights w_real [N x K] (real
    K only). Returns the int32 output (or the three SPLIT3 parts) and the updated row max."""
    acc = dot_rows(q, w_real)
    y = requant(acc, cst, e)
    M, N = y.shape
    if epi == "geglu":
        out = np.array([[geglu(y[r, 2 * c], y[r, 2 * c + 1], L) for c in range(N // 2)] for r in range(M)], dtype=object)
    elif epi == "gelu":
        out = np.array([[gelu(y[r, n], L) for n in range(N)] for r in range(M)], dtype=object)
    else:
        out = y
    if epi == "split3":
        parts = [np.zeros((M, Cs), np.int32) for _ in range(3)]
        for n in range(N):
            parts[n // Cs][:, n % Cs] = out[:, n].astype(np.int64)
        return parts, None
    if residual is not None:
        out = np.array([[sat32(out[r, n] + int(residual[r, n])) for n in range(out.shape[1])] for r in range(M)], dtype=object)
    res = out.astype(np.int64).astype(np.int32)
    rm = None
    if rowmax is not None:
        rm = np.array(rowmax, dtype=np.uint32, copy=True)
        if res.shape[1]:
            rm = np.maximum(rm, np.abs(res.astype(np.int64)).max(axis=1).astype(np.uint32))
    return res, rm


def split(q):
    """(hi, lo) int8 planes of 16-bit values: q = 256*hi + lo + 128 (src/intops.cuh:64-66)."""
    q = np.asarray(q, np.int64)
    hi = np.floor_divide(q, 256)
    lo = q - 256 * hi - 128
    return hi.astype(np.int8), lo.astype(np.int8)


def im2col_tapmajor(img: np.ndarray, stride: int) -> np.ndarray:
    """[B*Ho*Wo x 9C] patches of an NHWC image, zero padded by 1, K index = (3*ky + kx)*C + c."""
    B, H, W, C = img.shape
    Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
    pad = np.zeros((B, H + 2, W + 2, C), np.int64)
    pad[:, 1:-1, 1:-1, :] = img
    taps = [pad[:, ky:ky + (Ho - 1) * stride + 1:stride, kx:kx + (Wo - 1) * stride + 1:stride, :]
            for ky in range(3) for kx in range(3)]
    return np.stack(taps, axis=3).reshape(B * Ho * Wo, 9 * C)


def conv_row_exp(img: np.ndarray, stride: int) -> np.ndarray:
    """Per output pixel: row_exp of the largest |x| over the in-bounds 3x3 window, all channels."""
    patches = im2col_tapmajor(np.abs(np.asarray(img, np.int64)), stride)
    return np.array([row_exp(int(m)) for m in patches.max(axis=1)], np.int32)


def tapmajor_weights(w_nchw: np.ndarray) -> np.ndarray:
    """PyTorch conv weights [N, C, 3, 3] -> [N, 9C] with K index (3*ky + kx)*C + c."""
    N, C = w_nchw.shape[:2]
    return np.ascontiguousarray(np.transpose(w_nchw, (0, 2, 3, 1)).reshape(N, 9 * C))


def quant_matrix(x: np.ndarray, e: np.ndarray) -> np.ndarray:
    return np.array([[quant16(int(v), int(e[r])) for v in row] for r, row in enumerate(np.asarray(x))], np.int64)

"""TEST INFRASTRUCTURE ONLY: ctypes wrapper of oracle/liboracle.so, the CPU restatement of the
reference's W8A16 hi/lo GEMM semantics (oracle/oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and only
to check (or time, as the CPU baseline) the product; vela_amd/ never does.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

PATH = Path(__file__).resolve().parent / "liboracle.so"
P, I, LL, SZ, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t, ctypes.c_int64

SRC_I8, SRC_X32, SRC_CONV32, SRC_I16, SRC_CONV16 = 0, 1, 2, 3, 4
EPI_PLAIN, EPI_SPLIT3, EPI_GEGLU, EPI_GELU = 0, 1, 2, 3


class OrcGemm(ctypes.Structure):
    _fields_ = [
        ("src", I),
        ("hi", P), ("lo", P), ("ld8", I),
        ("e", P),
        ("x", P), ("ldx", I), ("xrowmax", P),
        ("q16", P), ("ld16", I),
        ("img", P), ("img16", P),
        ("K", I), ("H", I), ("W", I), ("C", I), ("stride", I), ("Ho", I), ("Wo", I),
        ("Mreal", I), ("Nreal", I), ("Kp", I),
        ("w", P), ("ldw", I),
        ("cst", P),
        ("epi", I),
        ("Y", P), ("ldy", I), ("residual", P),
        ("Cs", I), ("Y1", P), ("Y2", P),
        ("Lphi", P),
        ("rowmax", P),
    ]


_SIGS = {
    "orc_set_threads": (None, [I]),
    "orc_get_threads": (I, []),
    "orc_sat32": (I64, [I64]),
    "orc_rshr": (I64, [I64, I64]),
    "orc_row_exp": (I, [I64]),
    "orc_quant16": (I64, [I64, I]),
    "orc_quant16_32": (ctypes.c_int32, [ctypes.c_int32, I]),
    "orc_lut16i": (ctypes.c_int32, [I64, P]),
    "orc_split16": (None, [I64, P, P]),
    "orc_epi1": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_int32, P, ctypes.c_int32]),
    "orc_geglu": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_int32, P]),
    "orc_gelu": (ctypes.c_int32, [ctypes.c_int32, P]),
    "orc_rshr_n": (None, [P, P, P, SZ]),
    "orc_row_exp_n": (None, [P, P, SZ]),
    "orc_quant16_32_n": (None, [P, P, P, SZ]),
    "orc_lut16i_n": (None, [P, P, P, SZ]),
    "orc_epi1_n": (None, [P, P, P, P, P, SZ]),
    "orc_quant_rows": (None, [P, I, I, I, P, P, P, I]),
    "orc_act": (None, [P, SZ, P]),
    "orc_geglu_n": (None, [P, P, SZ, P]),
    "orc_add": (None, [P, P, SZ]),
    "orc_concat": (None, [P, I, P, I, I, P, P, I]),
    "orc_upsample2": (None, [P, I, I, I, I, P]),
    "orc_pixmax": (None, [P, I, I, P]),
    "orc_im2col3": (None, [P, P, I, I, I, I, I, P, P, P, I]),
    "orc_conv_e": (None, [P, I, I, I, I, P]),
    "orc_epilogue": (None, [P, P, I, I, I, P, P, P, I, P]),
    "orc_epilogue_split": (None, [P, P, I, I, I, P, P, I, P, P, P]),
    "orc_epilogue_geglu_q": (None, [P, P, I, I, I, P, P, P, P, P, P, I]),
    "orc_a_row": (I, [ctypes.POINTER(OrcGemm), I, P, P, P]),
    "orc_gemm_hl_rows": (I, [ctypes.POINTER(OrcGemm), I, I]),
    "orc_gemm_hl": (I, [ctypes.POINTER(OrcGemm)]),
    "orc_gemm_planes": (I, [ctypes.POINTER(OrcGemm), P, P, I]),
    "orc_i8gemm": (None, [P, I, LL, P, I, LL, P, I, LL, I, I, I, I]),
    "orc_prep_weight": (None, [P, I, I, I, P, P, P, I, I, P, P]),
    "orc_interleave2": (None, [P, P, P, P, I, I, P, P]),
    "orc_gn_accumulate": (None, [P, I, I, I, I, P, P, P]),
    "orc_gn_ref_tile": (None, [I, I, I, I, P, P]),
    "orc_gn_tiles": (None, [P, I, I, I, I, I, I, P, P, P]),
    "orc_gn_blocks": (None, [P, I, I, I, I, P, P, P]),
    "orc_qkv_heads": (None, [P, I, I, I, I, I, I, I] + [P] * 13),
    "orc_floor_div": (I64, [I64, I64]),
    "orc_isqrt": (I64, [I64]),
    "orc_gn_init": (None, [P, I]),
    "orc_gn_stats1": (None, [P, I, I, I, I, P]),
    "orc_gn_fin1": (None, [P, I, I64]),
    "orc_gn_stats2": (None, [P, I, I, I, I, P]),
    "orc_gn_fin2": (None, [P, I, I64, I64]),
    "orc_gn_apply": (None, [P, I, I, I, I, P, P, P, P]),
    "orc_gn_apply_row": (None, [P, I, I, I, I, P, P, P, P, P, P, P, P, P, I]),
    "orc_lnorm": (None, [P, I, I, P, P, I64, P]),
    "orc_lnorm_q": (None, [P, I, I, P, P, I64, P, P, P, I]),
    "orc_quant_heads": (None, [P, I, I, I, I, I, P, P, P, P, P, P]),
    "orc_quant_heads_pad": (None, [I, I, I, P, P, P, P, P, P]),
    "orc_quant_v": (None, [P, I, I, I, I, I, P, P, P, P]),
    "orc_attention": (None, [P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, P, I, P, P]),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not PATH.exists():
            raise RuntimeError(f"{PATH} is not built: run `python -m vela_amd.build`")
        L = ctypes.CDLL(str(PATH))
        for name, (res, args) in _SIGS.items():
            getattr(L, name).restype = res
            getattr(L, name).argtypes = args
        _lib = L
    return _lib


def a(x):
    """Address of a C-contiguous numpy array (None -> NULL)."""
    if x is None:
        return None
    assert x.flags.c_contiguous, "oracle inputs must be C-contiguous"
    return x.ctypes.data


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


# ---------------------------------------------------------------- vectorised primitives

def rshr(v, s):
    v = np.ascontiguousarray(v, np.int64); s = np.ascontiguousarray(np.broadcast_to(s, v.shape), np.int64)
    out = np.empty_like(v); lib().orc_rshr_n(a(v), a(s), a(out), v.size); return out


def row_exp(m):
    m = np.ascontiguousarray(m, np.int64); out = np.empty(m.shape, np.int32); lib().orc_row_exp_n(a(m), a(out), m.size); return out


def quant16_32(v, e):
    v = np.ascontiguousarray(v, np.int32); e = np.ascontiguousarray(np.broadcast_to(e, v.shape), np.int32)
    out = np.empty_like(v); lib().orc_quant16_32_n(a(v), a(e), a(out), v.size); return out


def lut16i(x, L):
    x = np.ascontiguousarray(x, np.int64); L = np.ascontiguousarray(L, np.int32)
    out = np.empty(x.shape, np.int32); lib().orc_lut16i_n(a(x), a(L), a(out), x.size); return out


def split16(v):
    """(hi, lo) of one 16-bit value through orc_split16."""
    h, l = ctypes.c_int8(), ctypes.c_int8()
    lib().orc_split16(int(v), ctypes.addressof(h), ctypes.addressof(l))
    return h.value, l.value


def epi1(chi, clo, cst4, er):
    chi = np.ascontiguousarray(chi, np.int32); clo = np.ascontiguousarray(clo, np.int32)
    cst4 = np.ascontiguousarray(cst4, np.int32).reshape(-1, 4); er = np.ascontiguousarray(np.broadcast_to(er, chi.shape), np.int32)
    out = np.empty_like(chi); lib().orc_epi1_n(a(chi), a(clo), a(cst4), a(er), a(out), chi.size); return out


# ---------------------------------------------------------------- GEMM

def gemm(src, *, Mreal, Nreal, Kp, w, cst, epi=EPI_PLAIN, e=None, hi=None, lo=None, q16=None, x=None, xrowmax=None,
         img=None, K=0, H=0, W=0, C=0, stride=1, Lphi=None, residual=None, Y=None, ldy=None, Cs=0, Y1=None, Y2=None,
         rowmax=None, rows=None):
    """Run the oracle GEMM. Returns Y (allocated if not given). `rows` = (r0, r1) limits the rows."""
    g = OrcGemm()
    g.src = src
    keep = []

    def put(x_, dt):
        if x_ is None:
            return None
        y = np.ascontiguousarray(x_, dt)
        keep.append(y)
        return a(y)

    g.e = put(e, np.int32)
    if src == SRC_I8:
        g.hi, g.lo, g.ld8 = put(hi, np.int8), put(lo, np.int8), hi.shape[-1]
    elif src == SRC_I16:
        g.q16, g.ld16, g.K = put(q16, np.int16), q16.shape[-1], K or q16.shape[-1]
    elif src == SRC_X32:
        g.x, g.ldx, g.xrowmax, g.K = put(x, np.int32), x.shape[-1], put(xrowmax, np.uint32), K or x.shape[-1]
    elif src in (SRC_CONV32, SRC_CONV16):
        if src == SRC_CONV32:
            g.img = put(img, np.int32)
        else:
            g.img16 = put(img, np.int16)
        g.H, g.W, g.C, g.stride = H, W, C, stride
        g.Ho, g.Wo, g.K = (H - 1) // stride + 1, (W - 1) // stride + 1, 9 * C
    g.Mreal, g.Nreal, g.Kp = Mreal, Nreal, Kp
    g.w, g.ldw = put(w, np.int8), w.shape[-1]
    g.cst = put(cst, np.int32)
    g.epi = epi
    nout = Nreal // 2 if epi == EPI_GEGLU else Nreal
    if Y is None and epi != EPI_SPLIT3:
        Y = np.zeros((Mreal, ldy or nout), np.int32)
    if Y is not None:
        assert Y.flags.c_contiguous and Y.dtype == np.int32
        g.Y, g.ldy = a(Y), ldy or Y.shape[-1]
    g.residual = put(residual, np.int32)
    g.Cs = Cs
    if Y1 is not None:
        g.Y1 = a(Y1)
    if Y2 is not None:
        g.Y2 = a(Y2)
    g.Lphi = put(Lphi, np.int32)
    if rowmax is not None:
        assert rowmax.flags.c_contiguous and rowmax.dtype in (np.uint32, np.int32)
        g.rowmax = a(rowmax)
    r0, r1 = rows if rows is not None else (0, Mreal)
    rc = lib().orc_gemm_hl_rows(ctypes.byref(g), r0, r1)
    if rc:
        raise ValueError("oracle rejected the GEMM description")
    return Y


def planes(src, *, Mreal, Nreal, Kp, w, **kw):
    """Per-plane int32 sums Chi, Clo [Mreal x Nreal]."""
    g = OrcGemm()
    keep = []
    # reuse gemm()'s packing by building the struct the same way
    Chi = np.zeros((Mreal, Nreal), np.int32)
    Clo = np.zeros((Mreal, Nreal), np.int32)
    g.src = src
    e = kw.get("e")
    if e is not None:
        e = np.ascontiguousarray(e, np.int32); keep.append(e); g.e = a(e)
    if src == SRC_I8:
        hi = np.ascontiguousarray(kw["hi"], np.int8); lo = np.ascontiguousarray(kw["lo"], np.int8); keep += [hi, lo]
        g.hi, g.lo, g.ld8 = a(hi), a(lo), hi.shape[-1]
    elif src == SRC_I16:
        q = np.ascontiguousarray(kw["q16"], np.int16); keep.append(q)
        g.q16, g.ld16, g.K = a(q), q.shape[-1], kw.get("K") or q.shape[-1]
    else:
        raise ValueError("planes() takes SRC_I8 / SRC_I16")
    w = np.ascontiguousarray(w, np.int8); keep.append(w)
    g.w, g.ldw = a(w), w.shape[-1]
    g.Mreal, g.Nreal, g.Kp = Mreal, Nreal, Kp
    if lib().orc_gemm_planes(ctypes.byref(g), a(Chi), a(Clo), Nreal):
        raise ValueError("oracle rejected the GEMM description")
    return Chi, Clo


def i8gemm(A, W, M, N, K, batch=1, sA=0, sW=0, sC=0, lda=None, ldw=None, ldc=None):
    A = np.ascontiguousarray(A, np.int8); W = np.ascontiguousarray(W, np.int8)
    lda = lda or K; ldw = ldw or K; ldc = ldc or N
    C = np.zeros(max(sC * batch, M * ldc) if batch > 1 else M * ldc, np.int32)
    lib().orc_i8gemm(a(A), lda, sA, a(W), ldw, sW, a(C), ldc, sC, M, N, K, batch)
    return C


# ---------------------------------------------------------------- producers

def quant_rows(X, M, K, ldx, Kp):
    X = np.ascontiguousarray(X, np.int32)
    Mp = (M + 31) // 32 * 32
    hi = np.zeros((Mp, Kp), np.int8); lo = np.zeros((Mp, Kp), np.int8); e = np.zeros(Mp, np.int32)
    lib().orc_quant_rows(a(X), M, K, ldx, a(hi), a(lo), a(e), Kp)
    return hi, lo, e


def pixmax(X, rows, C):
    X = np.ascontiguousarray(X, np.int32); pm = np.zeros(rows, np.uint32)
    lib().orc_pixmax(a(X), rows, C, a(pm)); return pm


def im2col3(X, pm, B, H, W, C, stride, Kp):
    X = np.ascontiguousarray(X, np.int32); pm = np.ascontiguousarray(pm, np.uint32)
    Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
    rows = B * Ho * Wo; Mp = (rows + 31) // 32 * 32
    hi = np.zeros((Mp, Kp), np.int8); lo = np.zeros((Mp, Kp), np.int8); e = np.zeros(Mp, np.int32)
    lib().orc_im2col3(a(X), a(pm), B, H, W, C, stride, a(hi), a(lo), a(e), Kp)
    return hi, lo, e


def conv_e(pm, B, H, W, stride):
    pm = np.ascontiguousarray(pm, np.uint32)
    rows = B * ((H - 1) // stride + 1) * ((W - 1) // stride + 1)
    e = np.zeros(rows, np.int32); lib().orc_conv_e(a(pm), B, H, W, stride, a(e)); return e


def epilogue(Chi, Clo, M, N, ldc, cst, e, ldy, R=None):
    Chi = np.ascontiguousarray(Chi, np.int32); Clo = np.ascontiguousarray(Clo, np.int32)
    cst = np.ascontiguousarray(cst, np.int32); e = np.ascontiguousarray(e, np.int32)
    Y = np.zeros((M, ldy), np.int32)
    Rr = None if R is None else np.ascontiguousarray(R, np.int32)
    lib().orc_epilogue(a(Chi), a(Clo), M, N, ldc, a(cst), a(e), a(Y), ldy, a(Rr))
    return Y


def epilogue_split(Chi, Clo, M, N, ldc, cst, e, Cs):
    Chi = np.ascontiguousarray(Chi, np.int32); Clo = np.ascontiguousarray(Clo, np.int32)
    cst = np.ascontiguousarray(cst, np.int32); e = np.ascontiguousarray(e, np.int32)
    Y0, Y1, Y2 = (np.zeros((M, Cs), np.int32) for _ in range(3))
    lib().orc_epilogue_split(a(Chi), a(Clo), M, N, ldc, a(cst), a(e), Cs, a(Y0), a(Y1), a(Y2))
    return Y0, Y1, Y2


def epilogue_geglu_q(Chi, Clo, M, F, ldc, cst, e, L, Kp):
    Chi = np.ascontiguousarray(Chi, np.int32); Clo = np.ascontiguousarray(Clo, np.int32)
    cst = np.ascontiguousarray(cst, np.int32); e = np.ascontiguousarray(e, np.int32); L = np.ascontiguousarray(L, np.int32)
    hi = np.zeros((M, Kp), np.int8); lo = np.zeros((M, Kp), np.int8); eo = np.zeros(M, np.int32)
    lib().orc_epilogue_geglu_q(a(Chi), a(Clo), M, F, ldc, a(cst), a(e), a(L), a(hi), a(lo), a(eo), Kp)
    return hi, lo, eo


def gn_stats(Y, M, N, T, ldy=None):
    """GroupNorm sum/min/max records of Y [M x N] over samples of T rows and 32 column groups
    (fresh records, as after k_gn_init): dict of int64 arrays [ceil(M / T) * 32]."""
    Y = np.ascontiguousarray(Y, np.int32)
    ldy = ldy or Y.shape[1]
    cnt = (M + T - 1) // T * 32
    s = np.zeros(cnt, np.int64)
    mn = np.full(cnt, 2**31 - 1, np.int32)
    mx = np.full(cnt, -(2**31), np.int32)
    lib().orc_gn_accumulate(a(Y), M, N, ldy, T, a(s), a(mn), a(mx))
    return {"sum": s, "mn": mn.astype(np.int64), "mx": mx.astype(np.int64)}


def _gn_records(M, T):
    cnt = (M + T - 1) // T * 32
    return np.zeros(cnt, np.int64), np.full(cnt, 2**31 - 1, np.int32), np.full(cnt, -(2**31), np.int32)


def gn_ref_tile(Mp, Np, Kp, src):
    """(BMr, BNr): the reference's fused-GEMM tile for these padded sizes (src/gemm_hl.cu:352-358);
    src is a GemmSrc code (SRC_I8 = 0 and the int16 rows SRC_I16 = 3 count as int8 planes)."""
    bm, bn = ctypes.c_int(), ctypes.c_int()
    lib().orc_gn_ref_tile(Mp, Np, Kp, 1 if src in (0, 3) else 0, ctypes.addressof(bm), ctypes.addressof(bn))
    return bm.value, bn.value


def gn_stats_fused(Y, M, N, T, Mp, Np, Kp, src, ldy=None, tile=None):
    """GroupNorm records of a fused GEMM's EPI_PLAIN output by the reference's per-tile flush rule
    (fresh records): dict of int64 arrays [ceil(M / T) * 32]."""
    Y = np.ascontiguousarray(Y, np.int32)
    ldy = ldy or Y.shape[1]
    bm, bn = tile or gn_ref_tile(Mp, Np, Kp, src)
    s, mn, mx = _gn_records(M, T)
    lib().orc_gn_tiles(a(Y), M, N, ldy, T, bm, bn, a(s), a(mn), a(mx))
    return {"sum": s, "mn": mn.astype(np.int64), "mx": mx.astype(np.int64)}


def gn_stats_planar(Y, M, N, T, ldy=None):
    """GroupNorm records of k_epilogue's output by the reference's per-1024-element flush rule
    (fresh records): dict of int64 arrays [ceil(M / T) * 32]."""
    Y = np.ascontiguousarray(Y, np.int32)
    ldy = ldy or Y.shape[1]
    s, mn, mx = _gn_records(M, T)
    lib().orc_gn_blocks(a(Y), M, N, ldy, T, a(s), a(mn), a(mx))
    return {"sum": s, "mn": mn.astype(np.int64), "mx": mx.astype(np.int64)}


def qkv_heads(Y, M, C, heads, T, TpQ, TpK, fill=0x5A):
    """EPI_QKV outputs from the plain output Y [M x 3C]. Buffers start filled with `fill` bytes (rows
    t >= T are left so). Returns dict: q/k -> (hi, lo [B*heads*Tp x 64], e, hs, ls, ts), v -> [M x C]."""
    Y = np.ascontiguousarray(Y, np.int32)
    B = (M + T - 1) // T
    out = {}
    for part, Tp in (("q", TpQ), ("k", TpK)):
        G = B * heads * Tp
        f8 = np.int8(np.uint8(fill).view(np.int8))
        out[part] = (np.full((G, 64), f8, np.int8), np.full((G, 64), f8, np.int8),
                     np.full(G, np.uint32(fill * 0x01010101).view(np.int32), np.int32),
                     *(np.full(G, np.uint64(fill * 0x0101010101010101).view(np.int64), np.int64) for _ in range(3)))
    V = np.zeros((M, C), np.int32)
    q, k = out["q"], out["k"]
    lib().orc_qkv_heads(a(Y), M, Y.shape[1], C, heads, T, TpQ, TpK, *(a(x) for x in q), *(a(x) for x in k), a(V))
    out["v"] = V
    return out


def prep_weight(w, N, K, conv3, m, s, b, Np, Kp):
    w = np.ascontiguousarray(w, np.int8)
    m, s, b = (np.ascontiguousarray(v, np.int32) for v in (m, s, b))
    wout = np.zeros((Np, Kp), np.int8); cst = np.zeros((Np, 4), np.int32)
    lib().orc_prep_weight(a(w), N, K, int(conv3), a(m), a(s), a(b), Np, Kp, a(wout), a(cst))
    return wout, cst


def interleave2(wa, ca, wg, cg, N, Kp):
    wa, wg = np.ascontiguousarray(wa, np.int8), np.ascontiguousarray(wg, np.int8)
    ca, cg = np.ascontiguousarray(ca, np.int32), np.ascontiguousarray(cg, np.int32)
    Np = (2 * N + 63) // 64 * 64
    wout = np.zeros((Np, Kp), np.int8); cout = np.zeros((Np, 4), np.int32)
    lib().orc_interleave2(a(wa), a(ca), a(wg), a(cg), N, Kp, a(wout), a(cout))
    return wout, cout


# ---------------------------------------------------------------- convenience for vela_amd.configs layers

def layer_reference(L, h, rows=None, seed_y=None):
    """Oracle output of a vela_amd.configs.Layer with host inputs h (rows = (r0, r1) subset).
    Returns (Y, rowmax); rows outside the subset stay zero (or the residual seed)."""
    nout = L.Nout
    Y = np.zeros((L.M, nout), np.int32) if seed_y is None else np.array(seed_y, np.int32, copy=True)
    if L.residual:
        Y[...] = h["res"]
    rowmax = np.zeros(L.M, np.uint32) if L.rowmax else None
    kw = dict(Mreal=L.M, Nreal=L.N, Kp=L.Kp, w=h["w"], cst=h["cst"], epi=L.epi, e=h.get("e"), Lphi=h.get("lphi"),
              Y=Y, ldy=nout, residual=Y if L.residual else None, rowmax=rowmax, rows=rows)
    if L.src == SRC_CONV16:
        gemm(SRC_CONV16, img=h["img"], H=L.H, W=L.W, C=L.C, stride=L.stride, **kw)
    elif L.kind == "conv_in":
        # k_pixmax + k_im2col3, then the GEMM on the planes (src/engine.cu:254-280)
        pm = pixmax(h["img32"].reshape(-1, L.C), L.B * L.H * L.W, L.C)
        hi, lo, e = im2col3(h["img32"], pm, L.B, L.H, L.W, L.C, L.stride, L.Kp)
        kw["e"] = e
        gemm(SRC_I8, hi=hi, lo=lo, **kw)
    else:
        gemm(SRC_I16, q16=h["a"], K=h["a"].shape[1], **kw)
    return Y, rowmax


# ---------------------------------------------------------------- integer normalisations

# GnStat records (src/kernels.h:9): sum, mn, mx, mean, e, (pad), ss, sd -- 48 bytes
GN_DTYPE = np.dtype([("sum", "<i8"), ("mn", "<i4"), ("mx", "<i4"), ("mean", "<i8"), ("e", "<i4"), ("pad", "<i4"),
                     ("ss", "<i8"), ("sd", "<i8")])


def floor_div(a: int, b: int) -> int:
    return int(lib().orc_floor_div(int(a), int(b)))


def isqrt(v: int) -> int:
    return int(lib().orc_isqrt(int(v)))


def gn_records(cnt: int) -> np.ndarray:
    """cnt records as k_gn_init leaves them (src/kernels.cu:173)."""
    gs = np.zeros(cnt, GN_DTYPE)
    lib().orc_gn_init(a(gs), cnt)
    return gs


# ---------------------------------------------------------------- elementwise (src/kernels.cu:536-561)

def act(X, L):
    """k_act: a copy of X with x = sat32(rshr(x lut16i(x, L), 16))."""
    X = np.array(X, np.int32, copy=True); L = np.ascontiguousarray(L, np.int32)
    lib().orc_act(a(X), X.size, a(L)); return X


def geglu_n(A, G, L):
    """k_geglu: a copy of A with a = sat32(rshr(a sat32(rshr(g lut16i(g, L), 16)), 16))."""
    A = np.array(A, np.int32, copy=True); G = np.ascontiguousarray(G, np.int32); L = np.ascontiguousarray(L, np.int32)
    lib().orc_geglu_n(a(A), a(G), A.size, a(L)); return A


def add(X, Y):
    """k_add: a copy of X with x = sat32(x + y)."""
    X = np.array(X, np.int32, copy=True); Y = np.ascontiguousarray(Y, np.int32)
    lib().orc_add(a(X), a(Y), X.size); return X


def concat(A, Ca, B, Cb, rows, gs=None, T=0):
    """k_concat: out [rows x (Ca + Cb)]; gs (GN_DTYPE records) accumulated in place when given."""
    A = np.ascontiguousarray(A, np.int32); B = np.ascontiguousarray(B, np.int32)
    out = np.zeros((rows, Ca + Cb), np.int32)
    lib().orc_concat(a(A), Ca, a(B), Cb, rows, a(out), a(gs), T)
    return out


def upsample2(X, B, H, W, C):
    X = np.ascontiguousarray(X, np.int32)
    out = np.zeros((B, 2 * H, 2 * W, C), np.int32)
    lib().orc_upsample2(a(X), B, H, W, C, a(out)); return out


def gn_stats1(X, B, T, C, groups, gs=None):
    """k_gn_stats1 (src/kernels.cu:745-750): init, sum/min/max, fin1."""
    X = np.ascontiguousarray(X, np.int32)
    gs = gn_records(B * groups) if gs is None else gs
    lib().orc_gn_stats1(a(X), B, T, C, groups, a(gs))
    lib().orc_gn_fin1(a(gs), B * groups, T * (C // groups))
    return gs


def gn_fin1(gs, n):
    lib().orc_gn_fin1(a(gs), len(gs), int(n))
    return gs


def gn_stats2(X, B, T, C, groups, den, gs):
    """k_gn_stats2 (src/kernels.cu:751-755): ss, fin2 (in place)."""
    X = np.ascontiguousarray(X, np.int32)
    lib().orc_gn_stats2(a(X), B, T, C, groups, a(gs))
    lib().orc_gn_fin2(a(gs), B * groups, T * (C // groups), int(den))
    return gs


def gn_apply(X, B, T, C, groups, gs, g64, beta64):
    X = np.ascontiguousarray(X, np.int32)
    g64, beta64 = np.ascontiguousarray(g64, np.int64), np.ascontiguousarray(beta64, np.int64)
    Y = np.zeros((B * T, C), np.int32)
    lib().orc_gn_apply(a(X), B, T, C, groups, a(gs), a(g64), a(beta64), a(Y))
    return Y


def gn_apply_row(X, B, T, C, groups, gs, g, beta, Lsig=None, Kp=None):
    """k_gn_apply_row (src/kernels.cu:287-305, 824-830): (Y, pm), or (hi, lo, e) when Kp is given."""
    X = np.ascontiguousarray(X, np.int32)
    g, beta = np.ascontiguousarray(g, np.int32), np.ascontiguousarray(beta, np.int32)
    L = None if Lsig is None else np.ascontiguousarray(Lsig, np.int32)
    M = B * T
    if Kp is None:
        Y = np.zeros((M, C), np.int32); pm = np.zeros(M, np.uint32)
        lib().orc_gn_apply_row(a(X), B, T, C, groups, a(gs), a(g), a(beta), a(L), a(Y), a(pm), None, None, None, 0)
        return Y, pm
    hi = np.zeros((M, Kp), np.int8); lo = np.zeros((M, Kp), np.int8); e = np.zeros(M, np.int32)
    lib().orc_gn_apply_row(a(X), B, T, C, groups, a(gs), a(g), a(beta), a(L), None, None, a(hi), a(lo), a(e), Kp)
    return hi, lo, e


def lnorm(X, M, C, g64, beta64, den):
    X = np.ascontiguousarray(X, np.int32)
    g64, beta64 = np.ascontiguousarray(g64, np.int64), np.ascontiguousarray(beta64, np.int64)
    Y = np.zeros((M, C), np.int32)
    lib().orc_lnorm(a(X), M, C, a(g64), a(beta64), int(den), a(Y))
    return Y


def lnorm_q(X, M, C, g, beta, den, Kp):
    X = np.ascontiguousarray(X, np.int32)
    g, beta = np.ascontiguousarray(g, np.int32), np.ascontiguousarray(beta, np.int32)
    hi = np.zeros((M, Kp), np.int8); lo = np.zeros((M, Kp), np.int8); e = np.zeros(M, np.int32)
    lib().orc_lnorm_q(a(X), M, C, a(g), a(beta), int(den), a(hi), a(lo), a(e), Kp)
    return hi, lo, e


# ---------------------------------------------------------------- attention (src/kernels.cu:611-672,799-805; src/attn.cu)

def quant_heads(X, B, T, C, heads, Tp):
    """k_quant_heads: X[B*T, C] int32 -> (hi, lo [G*Tp, 64] int8, e [G*Tp], hs, ls, tsum [G*Tp] int64)."""
    X = np.ascontiguousarray(X, np.int32)
    G = B * heads
    hi = np.zeros((G * Tp, 64), np.int8); lo = np.zeros((G * Tp, 64), np.int8)
    e = np.zeros(G * Tp, np.int32); hs = np.zeros(G * Tp, np.int64); ls = np.zeros(G * Tp, np.int64); ts = np.zeros(G * Tp, np.int64)
    lib().orc_quant_heads(a(X), B, T, C, heads, Tp, a(hi), a(lo), a(e), a(hs), a(ls), a(ts))
    return hi, lo, e, hs, ls, ts


def quant_heads_pad(G, T, Tp, hi, lo, e, hs, ls, ts):
    """k_quant_heads_pad on the arrays (in place)."""
    lib().orc_quant_heads_pad(G, T, Tp, a(hi), a(lo), a(e), a(hs), a(ls), a(ts))


def quant_v(X, B, Tk, C, heads, Tkp):
    """k_quant_v: X[B*Tk, C] int32 -> (vthi, vtlo [G*64, Tkp] int8, ev [G*64] int32, vsum [G*64] int64)."""
    X = np.ascontiguousarray(X, np.int32)
    G = B * heads
    vth = np.zeros((G * 64, Tkp), np.int8); vtl = np.zeros((G * 64, Tkp), np.int8)
    ev = np.zeros(G * 64, np.int32); vs = np.zeros(G * 64, np.int64)
    lib().orc_quant_v(a(X), B, Tk, C, heads, Tkp, a(vth), a(vtl), a(ev), a(vs))
    return vth, vtl, ev, vs


def attention(qh, ql, eq, kh, kl, ek, vth, vtl, ev, B, heads, Tq, Tqp, Tk, Tkp, causal, Lexp, C, rowmax=None):
    """The exact attention: out [B*Tq, C] int32 (columns h*64.. of head h), and the row maxima
    folded into `rowmax` (uint32 [B*Tq], updated in place) when given."""
    arrs = [np.ascontiguousarray(x, t) for x, t in ((qh, np.int8), (ql, np.int8), (eq, np.int32), (kh, np.int8), (kl, np.int8),
                                                   (ek, np.int32), (vth, np.int8), (vtl, np.int8), (ev, np.int32))]
    L = np.ascontiguousarray(Lexp, np.int64)
    out = np.zeros((B * Tq, C), np.int32)
    rm = None if rowmax is None else rowmax
    lib().orc_attention(*[a(x) for x in arrs], B, heads, Tq, Tqp, Tk, Tkp, 1 if causal else 0, a(L), C, a(out), a(rm) if rm is not None else None)
    return out


def exp_table():
    """An exp table of the reference's shape (1025 entries, Q30 at z = 0, falling by e every 2^16 of z;
    the model's own table comes from the model file, src/engine.cu:59)."""
    z = np.arange(1025, dtype=np.float64) * 1024.0
    return np.round(np.exp(-z / 65536.0) * 2.0**30).astype(np.int64)

"""TEST INFRASTRUCTURE ONLY: CPU restatement of the reference's model-file reader and GEMM weight
preparation, the checker of libvgemm.so's vgemm_model_* (include/vgemm_model.h).

  parse_poisd    src/poisd.cpp:11-54   (POISDv1 structure, checks and error messages)
  dev_model      src/engine.cu:11-45   (which int8 ".w" tensors become linears; padding, the
                                         tap-major 3x3 permutation, wsum and cst through
                                         orc_prep_weight) and :46-56 (norms)
  merge_lins     src/engine.cu:71-101  (row-stacked or alternating merged linears)
  MERGES         src/engine.cu:62-69   (the merged projections the reference builds)

Pins (tests/test_model.py): the parser against the arrays tests/golden/make_poisd.py wrote with an
independent struct.pack writer and against hand-built malformed files (one per error message); the
preparation's permutation against a transpose of [N, C, 3, 3] (orc_prep_weight's own pin); the
merges against the GEMM invariants they exist for (a merged QKV product equals the three products
side by side; a GEGLU over the alternating a/g rows equals the GEGLU formula over separate a and g
products).
"""
from __future__ import annotations

import struct

import numpy as np

from . import prep_weight

DTYPES = {0: np.int8, 1: np.int16, 2: np.int32, 3: np.uint8}
REQUIRED = ("unet.conv_in.w", "unet.conv_out.w", "te.tok.w", "te.pos", "lut.gauss", "lut.exp", "lut.sigmoid", "lut.phi",
            "c.sig", "c.cin", "tok.vocab", "tok.merges")
CONV3_SUFFIXES = (".conv1", ".conv2", "conv_in", "conv_out", "downsamplers.0.conv", "upsamplers.0.conv")


class FormatError(ValueError):
    pass


def parse_poisd(buf: bytes) -> dict:
    """{name: (dtype, dims, data array)} of a POISDv1 file (src/poisd.cpp:20-49); raises FormatError
    with the reference's message."""
    size = len(buf)
    if size < 12 or buf[:8] != b"POISDv1\x00":
        raise FormatError("bad magic (not a POISDv1 file)")
    pos = 8

    def need(n):
        if pos + n > size:
            raise FormatError("truncated model file")

    need(4)
    (count,) = struct.unpack_from("<I", buf, pos)
    pos += 4
    out = {}
    for _ in range(count):
        need(2)
        (nl,) = struct.unpack_from("<H", buf, pos)
        pos += 2
        need(nl + 2)
        name = buf[pos:pos + nl].decode("latin-1")
        pos += nl
        dtype, nd = buf[pos], buf[pos + 1]
        pos += 2
        if dtype > 3:
            raise FormatError("bad dtype")
        need(4 * nd)
        dims = list(struct.unpack_from(f"<{nd}I", buf, pos))
        pos += 4 * nd
        cnt = int(np.prod(dims, dtype=object)) if dims else 1
        nbytes = cnt * np.dtype(DTYPES[dtype]).itemsize
        need(nbytes)
        arr = np.frombuffer(buf, dtype=np.dtype(DTYPES[dtype]).newbyteorder("<"), count=cnt, offset=pos).reshape(dims)
        pos += nbytes
        out.setdefault(name, (dtype, dims, arr.astype(DTYPES[dtype])))   # std::map::emplace keeps the first
    if pos != size:
        raise FormatError("trailing data")
    for n in REQUIRED:
        if n not in out:
            raise FormatError("missing tensor " + n)
    return out


def _i32(ents, n):
    if n not in ents:
        raise FormatError("missing tensor " + n)
    dt, _, arr = ents[n]
    if dt != 2:
        raise FormatError(n + " is not int32")
    return arr.reshape(-1).astype(np.int32)


def dev_model(ents: dict) -> tuple[dict, dict]:
    """({base: (W [Np x Kp], cst [Np x 4], N, K, conv3)}, {base: (g, beta, den)}) as DevModel::load
    builds them (src/engine.cu:19-56), merged linears included (src/engine.cu:62-69)."""
    lins = {}
    for name in sorted(ents):
        dt, dims, arr = ents[name]
        if dt != 0 or not name.endswith(".w") or len(dims) != 2:
            continue
        base = name[:-2]
        if base == "te.tok" or base + ".m" not in ents:
            continue
        N, K = dims
        Np, Kp = (N + 63) // 64 * 64, (K + 15) // 16 * 16
        conv3 = base.endswith(CONV3_SUFFIXES)
        if conv3 and K % 9:
            raise FormatError("conv weight K not multiple of 9: " + name)
        m, s, b = (_i32(ents, base + x)[:N] for x in (".m", ".s", ".b"))
        W, cst = prep_weight(arr, N, K, conv3, m, s, b, Np, Kp)
        lins[base] = (W, cst, N, K, conv3)
    norms = {}
    for name in sorted(ents):
        if not name.endswith(".g"):
            continue
        base = name[:-2]
        if base + ".beta" not in ents or base + ".eps" not in ents:
            continue
        norms[base] = (_i32(ents, name), _i32(ents, base + ".beta"), int(_i32(ents, base + ".eps")[0]))
    for name, parts, inter in MERGES:
        merged = merge_lins(lins, parts, inter)
        if merged is not None:
            lins[name] = merged
    return lins, norms


def merge_lins(lins: dict, parts: list, interleave: bool):
    """DevModel::mergeLins (src/engine.cu:71-101); None if a part is missing."""
    if any(p not in lins for p in parts):
        return None
    ls = [lins[p] for p in parts]
    K = ls[0][3]
    if any(l[3] != K for l in ls):
        raise FormatError("mergeLins: K mismatch")
    N = sum(l[2] for l in ls)
    Np, Kp = (N + 63) // 64 * 64, ls[0][0].shape[1]
    W = np.zeros((Np, Kp), np.int8)
    cst = np.zeros((Np, 4), np.int32)
    cst[:, 0] = 1
    P = len(ls)
    if interleave and any(l[2] != ls[0][2] for l in ls):
        raise FormatError("mergeLins interleave: N mismatch")
    off = 0
    for i, (Wi, ci, Ni, _, _) in enumerate(ls):
        for r in range(Ni):
            d = r * P + i if interleave else off + r
            W[d] = Wi[r]
            cst[d] = ci[r]
        off += Ni
    return W, cst, N, K, False


def _merge_table():
    blocks = [f"unet.down_blocks.{i}.attentions.{j}" for i in range(3) for j in range(2)]
    blocks.append("unet.mid_block.attentions.0")
    blocks += [f"unet.up_blocks.{i}.attentions.{j}" for i in range(1, 4) for j in range(3)]
    out = []
    for bl in blocks:
        b = bl + ".transformer_blocks.0"
        out.append((b + ".attn1.to_qkv", [b + ".attn1.to_q", b + ".attn1.to_k", b + ".attn1.to_v"], False))
        out.append((b + ".ff.net.0.proj.ag", [b + ".ff.net.0.proj.a", b + ".ff.net.0.proj.g"], False))
        out.append((b + ".ff.net.0.proj.agi", [b + ".ff.net.0.proj.a", b + ".ff.net.0.proj.g"], True))
    for l in range(23):
        p = f"te.layers.{l}"
        out.append((p + ".self_attn.qkv", [p + ".self_attn.q_proj", p + ".self_attn.k_proj", p + ".self_attn.v_proj"], False))
    return out


MERGES = _merge_table()

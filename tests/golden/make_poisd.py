"""Writes tests/golden/tiny_model.poisd, a small synthetic POISDv1 model file; `block_tensors()` gives
the arrays of a second synthetic model (written by the tests that need it) with two resnet blocks and
one transformer block at reduced width.

The real model (sd-turbo-int.poisd, 1.2 GB) is not available offline, so this file stands in for it:
every tensor the reference's reader requires (src/poisd.cpp:47-49), in miniature, plus the kinds
the weight preparation distinguishes (src/engine.cu:11-101) -- 3x3 convolutions (tap-major K), a
plain linear with N and K off the 64/16 grid, a 1x1 convolution, the to_q/to_k/to_v and
ff.net.0.proj.a/g parts of one UNet transformer block (merged into to_qkv, ag and agi), a
GroupNorm's g/beta/eps, and entries the preparation must skip (te.tok.w, a rank-3 int8 ".w", a
".w" without ".m", an int16 tensor).

The writer below follows the format as documented in include/vgemm_model.h (little-endian; magic,
u32 count, then u16 name length, name, u8 dtype, u8 rank, u32 dims, data) with struct.pack, and
shares no code with the readers it checks. `tensors()` returns the arrays written, in order.
Run: python -m tests.golden.make_poisd
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
PATH = HERE / "tiny_model.poisd"
MAGIC = b"POISDv1\x00"
CODES = {np.dtype(np.int8): 0, np.dtype(np.int16): 1, np.dtype(np.int32): 2, np.dtype(np.uint8): 3}
BLOCK = "unet.down_blocks.0.attentions.0.transformer_blocks.0"
RESNET = "unet.down_blocks.0.resnets.0"


def encode(items, magic=MAGIC, count=None) -> bytes:
    """POISDv1 bytes of [(name, array)] in the given order (count overrides the header's count)."""
    out = bytearray(magic)
    out += struct.pack("<I", len(items) if count is None else count)
    for name, arr in items:
        nb = name.encode()
        out += struct.pack("<H", len(nb)) + nb
        out += struct.pack("<BB", CODES[arr.dtype], arr.ndim)
        out += b"".join(struct.pack("<I", d) for d in arr.shape)
        out += np.ascontiguousarray(arr).astype(arr.dtype.newbyteorder("<"), copy=False).tobytes()
    return bytes(out)


def _requant(r, n):
    return [r.integers(1 << 14, 1 << 15, n).astype(np.int32), r.integers(16, 25, n).astype(np.int32),
            r.integers(-50000, 50000, n).astype(np.int32)]


def _linear(items, r, base, N, K):
    w = r.integers(-127, 128, (N, K)).astype(np.int8)
    m, s, b = _requant(r, N)
    items += [(base + ".w", w), (base + ".m", m), (base + ".s", s), (base + ".b", b)]


def phi_table() -> np.ndarray:
    """A monotone Q16 table over the 2049 grid points (a smooth step from 0 to 65536)."""
    x = (np.arange(2049) - 1024) / 256.0
    return np.round(65536.0 / (1.0 + np.exp(-1.702 * x))).astype(np.int32)


def tensors():
    r = np.random.default_rng(0x504F4953)
    items = []
    # required by the reader (src/poisd.cpp:47-49)
    _linear(items, r, "unet.conv_in", 64, 9 * 8)          # 3x3 convolution of an 8-channel image
    _linear(items, r, "unet.conv_out", 8, 9 * 64)         # 3x3 convolution, N = 8 (padded to 64)
    items += [("te.tok.w", r.integers(-127, 128, (32, 16)).astype(np.int8)),
              ("te.tok.m", r.integers(1 << 14, 1 << 15, 32).astype(np.int32)),
              ("te.pos", r.integers(-1000, 1000, (4, 16)).astype(np.int32)),
              ("lut.gauss", np.arange(257, dtype=np.int32) * 3),
              ("lut.exp", (np.arange(513, dtype=np.int32) * 7) % 65536),
              ("lut.sigmoid", phi_table()),
              ("lut.phi", phi_table()),
              ("c.sig", np.array([12345], np.int32)),
              ("c.cin", np.array([-77], np.int32)),
              ("tok.vocab", np.frombuffer(b"hello\nworld\n", np.uint8).copy()),
              ("tok.merges", np.frombuffer(b"h e\nl o\n", np.uint8).copy())]
    # a resnet: two 3x3 convolutions, a 1x1 shortcut (a plain linear), a GroupNorm
    _linear(items, r, RESNET + ".conv1", 64, 9 * 64)
    _linear(items, r, RESNET + ".conv2", 64, 9 * 64)
    _linear(items, r, RESNET + ".conv_shortcut", 64, 64)
    items += [(RESNET + ".norm1.g", r.integers(1 << 15, 1 << 17, 64).astype(np.int32)),
              (RESNET + ".norm1.beta", r.integers(-5000, 5000, 64).astype(np.int32)),
              (RESNET + ".norm1.eps", np.array([65], np.int32))]
    # a linear off the padding grid
    _linear(items, r, "unet.time_embedding.linear_1", 70, 40)
    # one transformer block's projections (merged by the preparation)
    for p in ("to_q", "to_k", "to_v"):
        _linear(items, r, f"{BLOCK}.attn1.{p}", 64, 64)
    _linear(items, r, f"{BLOCK}.ff.net.0.proj.a", 96, 64)
    _linear(items, r, f"{BLOCK}.ff.net.0.proj.g", 96, 64)
    # entries the preparation skips
    items += [("unet.rank3.w", r.integers(-127, 128, (4, 4, 4)).astype(np.int8)),
              ("unet.rank3.m", np.ones(4, np.int32)),
              ("unet.no_requant.w", r.integers(-127, 128, (8, 16)).astype(np.int8)),
              ("te.int16_table", r.integers(-30000, 30000, 10).astype(np.int16))]
    # a scalar (rank 0) and an empty tensor
    items += [("c.rank0", np.array(7, np.int32)), ("c.empty", np.zeros((0, 5), np.int32))]
    return items


# the block model (block_tensors): resnet A 64 -> 128 channels with a 1x1 shortcut, resnet B 128 -> 128,
# a transformer of XF_HEADS heads of 64 (C = 128), GEGLU width XF_F, cross-attention context width CTX_C
RESNET_A = "unet.down_blocks.1.resnets.0"
RESNET_B = "unet.down_blocks.1.resnets.1"
XF = "unet.down_blocks.1.attentions.0"
XF_HEADS, XF_C, XF_F, CTX_C = 2, 128, 256, 96


def sigmoid_table() -> np.ndarray:
    """Q16 sigmoid over the 2049 grid points of lut16i (x in [-16, 16), step 1/64)."""
    x = (np.arange(2049) - 1024) / 64.0
    return np.round(65536.0 / (1.0 + np.exp(-x))).astype(np.int32)


def exp_table32() -> np.ndarray:
    """1025 entries, 2^30 at z = 0, falling by e every 2^16 of z (grid step 1024)."""
    z = np.arange(1025, dtype=np.float64) * 1024.0
    return np.round(np.exp(-z / 65536.0) * 2.0**30).astype(np.int32)


def _linear_scaled(items, r, base, N, K):
    """A linear whose requantisation keeps the output's scale near the input's: s around
    log2(sqrt(K) * 73 * m) (73 = the standard deviation of a uniform int8 weight)."""
    w = r.integers(-127, 128, (N, K)).astype(np.int8)
    m = r.integers(1 << 14, 1 << 15, N).astype(np.int32)
    s0 = int(round(np.log2(np.sqrt(K) * 73.0 * 23170.0)))
    s = r.integers(s0 - 1, s0 + 2, N).astype(np.int32)
    b = r.integers(-20000, 20000, N).astype(np.int32)
    items += [(base + ".w", w), (base + ".m", m), (base + ".s", s), (base + ".b", b)]


def _norm(items, r, base, C):
    items += [(base + ".g", r.integers(40000, 90000, C).astype(np.int32)),
              (base + ".beta", r.integers(-6000, 6000, C).astype(np.int32)),
              (base + ".eps", np.array([100000], np.int32))]


def block_tensors():
    r = np.random.default_rng(0x424C4B53)
    items = []
    _linear(items, r, "unet.conv_in", 64, 9 * 8)
    _linear(items, r, "unet.conv_out", 8, 9 * 64)
    items += [("te.tok.w", r.integers(-127, 128, (32, 16)).astype(np.int8)),
              ("te.tok.m", r.integers(1 << 14, 1 << 15, 32).astype(np.int32)),
              ("te.pos", r.integers(-1000, 1000, (4, 16)).astype(np.int32)),
              ("lut.gauss", np.arange(257, dtype=np.int32) * 3),
              ("lut.exp", exp_table32()),
              ("lut.sigmoid", sigmoid_table()),
              ("lut.phi", phi_table()),
              ("c.sig", np.array([12345], np.int32)),
              ("c.cin", np.array([-77], np.int32)),
              ("tok.vocab", np.frombuffer(b"hello\nworld\n", np.uint8).copy()),
              ("tok.merges", np.frombuffer(b"h e\nl o\n", np.uint8).copy())]
    for base, ci, co, short in ((RESNET_A, 64, 128, True), (RESNET_B, 128, 128, False)):
        _norm(items, r, base + ".norm1", ci)
        _linear_scaled(items, r, base + ".conv1", co, 9 * ci)
        _norm(items, r, base + ".norm2", co)
        _linear_scaled(items, r, base + ".conv2", co, 9 * co)
        if short:
            _linear_scaled(items, r, base + ".conv_shortcut", co, ci)
    C, F = XF_C, XF_F
    b = XF + ".transformer_blocks.0"
    _norm(items, r, XF + ".norm", C)
    _linear_scaled(items, r, XF + ".proj_in", C, C)
    for n in ("norm1", "norm2", "norm3"):
        _norm(items, r, f"{b}.{n}", C)
    for n in ("attn1.to_q", "attn1.to_k", "attn1.to_v", "attn1.to_out.0", "attn2.to_q", "attn2.to_out.0"):
        _linear_scaled(items, r, f"{b}.{n}", C, C)
    _linear_scaled(items, r, f"{b}.attn2.to_k", C, CTX_C)
    _linear_scaled(items, r, f"{b}.attn2.to_v", C, CTX_C)
    _linear_scaled(items, r, f"{b}.ff.net.0.proj.a", F, C)
    _linear_scaled(items, r, f"{b}.ff.net.0.proj.g", F, C)
    _linear_scaled(items, r, f"{b}.ff.net.2", C, F)
    _linear_scaled(items, r, XF + ".proj_out", C, C)
    return items


def main() -> None:
    PATH.write_bytes(encode(tensors()))
    print(f"wrote {PATH} ({PATH.stat().st_size} bytes)")


if __name__ == "__main__":
    main()

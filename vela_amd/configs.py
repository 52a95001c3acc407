"""Workloads of BASELINE.json as concrete seeded layers, plus the device-side problem runner.

A `Layer` is one GEMM: a linear (SRC_I16: int16 activations [M x K] + per-row shift) or a 3x3 conv
(SRC_CONV16: NHWC int16 image, implicit im2col), int8 weights [Np x Kp] (row n = output column n;
tap-major K for convs, a/g rows interleaved for GEGLU), cst = {m, s, b, wsum} per column, and an
epilogue. `make_host` draws its inputs; `DeviceProblem` holds them in HBM and calls vgemm_hl2.

Seeds: 0x56454C41 + config index (C1..C5); C5 layer i uses the C5 seed + i. Requantisation: m in
[2^14, 2^15), s in [16, 24], b in [-50000, 50000), as the reference's GEMM test draws them
(src/test_gemm_hl.cu:63) with s narrowed to the BASELINE.json range.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

import numpy as np

from . import datagen as dg

SEED0 = 0x56454C41
EPI_PLAIN, EPI_SPLIT3, EPI_GEGLU, EPI_GELU = 0, 1, 2, 3
SRC_I8, SRC_X32, SRC_CONV32, SRC_I16, SRC_CONV16 = 0, 1, 2, 3, 4


def align(v: int, a: int) -> int:
    return (v + a - 1) // a * a


def phi_lut() -> np.ndarray:
    """A monotone Q16 table of the standard normal CDF over [-16, 16) at 2049 points (step 1/64):
    the stand-in for the model's lut.phi (src/engine.cu:57-59), which is not available offline."""
    x = -16.0 + np.arange(2049) / 64.0
    return np.array([int(round(65536.0 * 0.5 * (1.0 + math.erf(v / math.sqrt(2.0))))) for v in x], dtype=np.int32)


@dataclass
class Layer:
    name: str
    kind: str                      # "linear" | "conv" | "conv_in" (3x3 conv of an int32 image through im2col3)
    M: int                         # output rows (B*Ho*Wo for a conv)
    K: int                         # real reduction length (9C for a conv)
    N: int                         # real output columns of W (2F for GEGLU)
    epi: int = EPI_PLAIN
    residual: bool = False
    rowmax: bool = False
    B: int = 0
    H: int = 0
    W: int = 0
    C: int = 0
    stride: int = 1
    a_dist: tuple = ("gauss", 2000.0)
    w_dist: tuple = ("uniform", 127)
    seed: int = SEED0
    src: int = -1                  # default: SRC_I16 for linears, SRC_CONV16 for convs
    e_bits: int = 0                # >0: draw per-row shifts e in [0, e_bits] (e-path coverage)
    s_range: tuple = (16, 24)
    meta: dict = field(default_factory=dict)

    def __post_init__(self):
        if self.src < 0:
            self.src = {"conv": SRC_CONV16, "conv_in": SRC_I8}.get(self.kind, SRC_I16)

    @property
    def Kp(self) -> int:
        return align(self.K, 16)

    @property
    def Np(self) -> int:
        return align(self.N, 64)

    @property
    def Mp(self) -> int:
        return align(self.M, 64)

    @property
    def Ho(self) -> int:
        return (self.H - 1) // self.stride + 1

    @property
    def Wo(self) -> int:
        return (self.W - 1) // self.stride + 1

    @property
    def Nout(self) -> int:
        return self.N // 2 if self.epi == EPI_GEGLU else self.N

    @property
    def ops(self) -> int:
        """Algorithmic int8 operations: 2 planes x 2 ops per MAC over the real M, N, K."""
        return 4 * self.M * self.N * self.K

    @property
    def a_bytes(self) -> int:
        if self.kind == "conv":
            return 2 * self.B * self.H * self.W * self.C   # the NHWC image, counted once
        if self.kind == "conv_in":
            return 4 * self.B * self.H * self.W * self.C   # the int32 NHWC image, counted once
        return 2 * self.M * self.K

    @property
    def hbm_bytes(self) -> int:
        """Algorithmic HBM bytes: A + W + int32 Y + cst + per-row e/rowmax (+ residual read)."""
        b = self.a_bytes + self.N * self.K + 4 * self.M * self.Nout + 16 * self.N + 4 * self.M
        if self.residual:
            b += 4 * self.M * self.Nout
        return b


# ---------------------------------------------------------------- host inputs

def _act(shape, seed, dist):
    kind, p = dist
    if kind == "gauss":
        return dg.i16_gauss(shape, seed, p)
    if kind == "laplace":
        return dg.i16_laplace(shape, seed, p)
    if kind == "uniform16":
        return dg.i16_uniform(shape, seed)
    raise ValueError(dist)


def _weights(shape, seed, dist):
    kind, p = dist
    if kind == "uniform":
        return dg.i8_uniform(shape, seed, -p, p)
    if kind == "gauss":
        return dg.i8_gauss(shape, seed, p)
    if kind == "uniform8":
        return dg.i8_uniform(shape, seed, -128, 127)
    raise ValueError(dist)


def make_host(L: Layer) -> dict:
    """Seeded host inputs of one layer (numpy)."""
    s = L.seed * 16
    h = {}
    if L.kind == "conv":
        h["img"] = _act((L.B, L.H, L.W, L.C), s + 1, L.a_dist)
    elif L.kind == "conv_in":
        # int32 pixels: 16-bit Gaussian values times 2^k, k in [0, 6] per pixel, so that the
        # per-row shifts e of the im2col quantisation vary over the image
        base = _act((L.B, L.H, L.W, L.C), s + 1, L.a_dist).astype(np.int32)
        k = dg.i32_uniform((L.B, L.H, L.W, 1), s + 8, 0, 6)
        h["img32"] = np.ascontiguousarray(base << k)
    else:
        h["a"] = _act((L.M, L.K), s + 1, L.a_dist)
    w = np.zeros((L.Np, L.Kp), dtype=np.int8)
    w[: L.N, : L.K] = _weights((L.N, L.K), s + 2, L.w_dist)
    h["w"] = w
    cst = np.zeros((L.Np, 4), dtype=np.int32)
    cst[:, 0] = 1                                           # pad columns: m = 1, s = b = wsum = 0
    cst[: L.N, 0] = dg.i32_uniform(L.N, s + 3, 1 << 14, (1 << 15) - 1)
    cst[: L.N, 1] = dg.i32_uniform(L.N, s + 4, L.s_range[0], L.s_range[1])
    cst[: L.N, 2] = dg.i32_uniform(L.N, s + 5, -50000, 49999)
    cst[: L.N, 3] = w[: L.N].astype(np.int64).sum(axis=1).astype(np.int32)
    h["cst"] = cst
    h["e"] = dg.i32_uniform(L.M, s + 6, 0, L.e_bits) if L.e_bits > 0 else None
    if L.residual:
        h["res"] = dg.i32_uniform((L.M, L.Nout), s + 7, -(2**31), 2**31 - 1)
    if L.epi in (EPI_GEGLU, EPI_GELU):
        h["lphi"] = phi_lut()
    return h


# ---------------------------------------------------------------- the BASELINE.json configurations

def c1() -> Layer:
    return Layer("C1 linear 4096x320x320", "linear", 4096, 320, 320, a_dist=("gauss", 2000.0), seed=SEED0 + 1)


def c2(epi: int = EPI_GEGLU) -> Layer:
    name = "C2 GEGLU up-proj 32768x320x2560" if epi == EPI_GEGLU else "C2 plain 32768x320x2560"
    return Layer(name, "linear", 32768, 320, 2560, epi=epi, rowmax=epi == EPI_GEGLU,
                 a_dist=("laplace", 1500.0), w_dist=("gauss", 40.0), seed=SEED0 + 2)


def c3() -> Layer:
    return Layer("C3 conv3x3 [8,32,32,640]->640", "conv", 8 * 32 * 32, 9 * 640, 640, B=8, H=32, W=32, C=640,
                 a_dist=("gauss", 3000.0), seed=SEED0 + 3)


def c4() -> list[Layer]:
    return [
        Layer("C4 conv3x3 [8,16,16,1280]->1280", "conv", 8 * 16 * 16, 9 * 1280, 1280, B=8, H=16, W=16, C=1280,
              a_dist=("gauss", 3000.0), seed=SEED0 + 4),
        Layer("C4 conv3x3 [8,8,8,1280]->1280", "conv", 8 * 8 * 8, 9 * 1280, 1280, B=8, H=8, W=8, C=1280,
              a_dist=("gauss", 3000.0), seed=SEED0 + 4 + 1000),
        Layer("C4 cross-attn K/V 616x1024x1280", "linear", 8 * 77, 1024, 1280, a_dist=("gauss", 2000.0), seed=SEED0 + 4 + 2000),
    ]


def unet_layers(B: int = 8) -> list[Layer]:
    """The 194 linear/conv GEMMs of the SD-turbo-sized UNet forward at batch B, in forward order
    (src/engine.cu:455-490 with resnet :389-405 and transformer :406-454; widths 320/640/1280/1280,
    64x64 latent). QKV is one PLAIN GEMM with N = 3C; ff.net.0.proj is the interleaved GEGLU GEMM
    (+ rowmax, as gegluX at :447); ff.net.2 writes rowmax; residual adds as at :400-401, :431, :440,
    :447, :451. conv_in (C = 4, an int32 image) runs as the reference runs it (src/engine.cu:458 ->
    :254-280): pixel maxima, a materialised im2col3 operand (K = 36 padded to 48, e per row), then the
    GEMM on those int8 planes."""
    L: list[Layer] = []
    seed = SEED0 + 5

    def add(layer: Layer):
        L.append(replace(layer, seed=seed * 1000 + len(L)))

    def conv(name, cin, cout, H, stride=1, residual=False):
        Ho = (H - 1) // stride + 1
        add(Layer(name, "conv", B * Ho * Ho, 9 * cin, cout, residual=residual, B=B, H=H, W=H, C=cin, stride=stride,
                  a_dist=("gauss", 3000.0)))

    def lin(name, M, K, N, epi=EPI_PLAIN, residual=False, rowmax=False):
        add(Layer(name, "linear", M, K, N, epi=epi, residual=residual, rowmax=rowmax, a_dist=("gauss", 2000.0)))

    def resnet(p, cin, cout, H):
        conv(p + ".conv1", cin, cout, H)
        if cin != cout:
            lin(p + ".conv_shortcut", B * H * H, cin, cout)
        conv(p + ".conv2", cout, cout, H, residual=True)

    def transformer(p, C, H):
        M = B * H * H
        lin(p + ".proj_in", M, C, C)
        lin(p + ".attn1.to_qkv", M, C, 3 * C)
        lin(p + ".attn1.to_out.0", M, C, C, residual=True)
        lin(p + ".attn2.to_q", M, C, C)
        lin(p + ".attn2.to_out.0", M, C, C, residual=True)
        lin(p + ".ff.net.0.proj", M, C, 8 * C, epi=EPI_GEGLU, rowmax=True)
        lin(p + ".ff.net.2", M, 4 * C, C, residual=True, rowmax=True)
        lin(p + ".proj_out", M, C, C, residual=True)

    ch = [320, 640, 1280, 1280]
    H = 64
    add(Layer("conv_in", "conv_in", B * H * H, 36, 320, B=B, H=H, W=H, C=4, a_dist=("gauss", 3000.0)))
    skips = [320]
    cin = 320
    for i in range(4):
        for j in range(2):
            resnet(f"down_blocks.{i}.resnets.{j}", cin, ch[i], H)
            cin = ch[i]
            if i < 3:
                transformer(f"down_blocks.{i}.attentions.{j}", ch[i], H)
            skips.append(ch[i])
        if i < 3:
            conv(f"down_blocks.{i}.downsamplers.0.conv", ch[i], ch[i], H, stride=2)
            H //= 2
            skips.append(ch[i])
    resnet("mid_block.resnets.0", cin, cin, H)
    transformer("mid_block.attentions.0", cin, H)
    resnet("mid_block.resnets.1", cin, cin, H)
    for i in range(4):
        cout = ch[3 - i]
        for j in range(3):
            s = skips.pop()
            resnet(f"up_blocks.{i}.resnets.{j}", cin + s, cout, H)
            cin = cout
            if i > 0:
                transformer(f"up_blocks.{i}.attentions.{j}", cout, H)
        if i < 3:
            H *= 2
            conv(f"up_blocks.{i}.upsamplers.0.conv", cin, cin, H)
    conv("conv_out", cin, 4, H)
    return L


# ---------------------------------------------------------------- device problem

class DeviceProblem:
    """One layer's inputs and outputs resident in HBM, callable through the C ABI."""

    def __init__(self, L: Layer, h: dict | None = None, device: str = "cuda", with_ws: bool = True):
        import torch

        from . import gemm as vg

        self.L = L
        self.h = h if h is not None else make_host(L)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)   # noqa: E731
        if L.kind == "conv_in":
            # k_pixmax + k_im2col3 outputs: pixel maxima, int8 planes [Mp x Kp] and row shifts
            self.img32 = t(self.h["img32"])
            self.pm = torch.zeros(L.B * L.H * L.W, dtype=torch.int32, device=device)
            self.hi = torch.zeros((L.Mp, L.Kp), dtype=torch.int8, device=device)
            self.lo = torch.zeros((L.Mp, L.Kp), dtype=torch.int8, device=device)
            self.e_in = torch.zeros(L.Mp, dtype=torch.int32, device=device)
        self.w = t(self.h["w"])
        self.cst = t(self.h["cst"])
        self.e = t(self.h["e"]) if self.h.get("e") is not None else None
        self.img = t(self.h["img"]) if "img" in self.h else None
        self.a = t(self.h["a"]) if "a" in self.h else None
        self.res = t(self.h["res"]) if "res" in self.h else None
        self.lphi = t(self.h["lphi"]) if "lphi" in self.h else None
        self.y = torch.zeros((L.M, L.Nout), dtype=torch.int32, device=device)
        self.rowmax = torch.zeros(L.M, dtype=torch.int32, device=device) if L.rowmax else None
        self.ws = None
        if with_ws:
            nb = vg.workspace_bytes(L.Mp, L.M, L.Np, L.N, L.Kp, L.epi)
            if nb:
                self.ws = torch.empty(nb // 4 + 64, dtype=torch.int32, device=device)
        self._build_args()

    def _build_args(self):
        from . import gemm as vg

        L = self.L
        A = vg.ASrc(src=L.src)
        A.e = vg.ptr(self.e)
        if L.src == SRC_CONV16:
            A.img16 = vg.ptr(self.img)
            A.H, A.W, A.C, A.stride, A.Ho, A.Wo, A.K = L.H, L.W, L.C, L.stride, L.Ho, L.Wo, L.K
        elif L.src == SRC_I16:
            A.q16 = vg.ptr(self.a)
            A.ld16 = self.a.shape[1]
            A.K = self.a.shape[1]
        elif L.kind == "conv_in":
            A.hi, A.lo, A.ld8, A.e = vg.ptr(self.hi), vg.ptr(self.lo), L.Kp, vg.ptr(self.e_in)
        else:
            raise ValueError("DeviceProblem drives the int16 sources")
        E = vg.AEpi(epi=L.epi, Y=vg.ptr(self.y), ldy=L.Nout)
        # residual aliases Y as at src/engine.cu:431 (the caller re-seeds Y before each checked call)
        E.residual = vg.ptr(self.y) if L.residual else None
        E.Lphi = vg.ptr(self.lphi)
        E.rowmax = vg.ptr(self.rowmax)
        if self.ws is not None:
            E.ws = vg.ptr(self.ws)
            E.ws_bytes = self.ws.numel() * 4
        self.A, self.E = A, E

    def reset(self):
        """Y <- residual input (or 0) and rowmax <- 0, by kernels (capture-safe)."""
        if self.res is not None:
            self.y.copy_(self.res)
        if self.rowmax is not None:
            from . import gemm as vg
            vg.fill_u32(self.rowmax, 0)

    def run(self, stream=None):
        from . import gemm as vg

        L = self.L
        if L.kind == "conv_in":
            vg.k_pixmax(self.img32, L.B * L.H * L.W, L.C, self.pm, stream=stream)
            vg.k_im2col3(self.img32, self.pm, L.B, L.H, L.W, L.C, L.stride, self.hi, self.lo, self.e_in, L.Kp, stream=stream)
        vg.k_gemm_hl2(self.A, L.Mp, L.M, self.w, self.w.shape[1], L.Np, L.N, L.Kp, self.cst, self.E, stream=stream)

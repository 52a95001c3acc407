"""Python mirror of the reference's GEMM call surface over the C ABI of libvgemm.so.

Names, argument order and meaning follow meow:: in src/gemm_hl.h:8-35, src/gemm.h:12-23 and
src/kernels.h:11-21,68-70 of the reference; a failed shape check raises (VgemmError, a RuntimeError)
where the reference throws std::runtime_error. Tensor arguments are torch CUDA tensors (or raw device
addresses as ints, or None for a null pointer); `stream` defaults to torch's current stream.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import GNSTAT_BYTES, GNSTAT_OFFSETS, AEpi, ASrc, VgemmError, View, check, load

EPI_PLAIN, EPI_SPLIT3, EPI_GEGLU, EPI_GELU, EPI_QKV = 0, 1, 2, 3, 4
SRC_I8, SRC_X32, SRC_CONV32, SRC_I16, SRC_CONV16 = 0, 1, 2, 3, 4

__all__ = [
    "ASrc", "AEpi", "View", "VgemmError", "k_gemm_hl2_view", "EPI_PLAIN", "EPI_SPLIT3", "EPI_GEGLU", "EPI_GELU", "EPI_QKV",
    "SRC_I8", "SRC_X32", "SRC_CONV32", "SRC_I16", "SRC_CONV16", "k_gemm_hl2", "k_gemm_hl", "k_conv_e",
    "gemm_hl_supported", "set_variant", "get_variant", "set_splitk", "set_stream_workspaces", "set_tile_order", "conv16_halo_rows", "workspace_bytes", "view_workspace_bytes", "Gemm",
    "k_quant_rows", "k_epilogue", "k_pixmax", "k_im2col3", "k_epilogue_split", "k_epilogue_geglu_q",
    "fill_u32", "Graph", "ptr", "stream_ptr", "GNSTAT_BYTES", "gn_stats_alloc", "k_gn_init", "gn_stats_read",
]


def ptr(t) -> int | None:
    """Device address of a tensor (None/0 -> null)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t or None
    if isinstance(t, torch.Tensor):
        if not t.is_cuda:
            raise ValueError("vgemm takes device tensors")
        return t.data_ptr()
    raise TypeError(f"cannot take a device address of {type(t)}")


def stream_ptr(stream=None) -> int | None:
    if stream is None:
        stream = torch.cuda.current_stream()
    if isinstance(stream, int):
        return stream or None
    return stream.cuda_stream or None


def k_gemm_hl2(A: ASrc, Mp: int, Mreal: int, W, ldw: int, Np: int, Nreal: int, Kp: int, cst, E: AEpi, stream=None) -> None:
    """meow::k_gemm_hl2 (src/gemm_hl.h:27)."""
    check(load().vgemm_hl2(stream_ptr(stream), ctypes.byref(A), Mp, Mreal, ptr(W), ldw, Np, Nreal, Kp, ptr(cst), ctypes.byref(E)))


NOALLOC_WS_BYTES = 64 << 20


def set_stream_workspaces(on: bool) -> None:
    """vgemm_set_stream_workspaces: split-K workspaces for calls without AEpi.ws (default on)."""
    load().vgemm_set_stream_workspaces(1 if on else 0)


def k_gemm_hl2_view(A: ASrc, Mp: int, Mreal: int, W, ldw: int, Np: int, Nreal: int, Kp: int, cst, E: AEpi, hi, lo, e, ld: int,
                    stream=None) -> None:
    """vgemm_hl2_view: the int16 view of the output (planes hi/lo [Mreal x ld], e per row) instead of Y;
    E.ws must hold view_workspace_bytes()."""
    V = View(hi=ptr(hi), lo=ptr(lo), e=ptr(e), ld=ld)
    check(load().vgemm_hl2_view(stream_ptr(stream), ctypes.byref(A), Mp, Mreal, ptr(W), ldw, Np, Nreal, Kp, ptr(cst), ctypes.byref(E),
                                ctypes.byref(V)))


def k_gemm_hl2_noalloc(A: ASrc, Mp: int, Mreal: int, W, ldw: int, Np: int, Nreal: int, Kp: int, cst, E: AEpi, stream=None) -> None:
    """vgemm_hl2 with the split-K partials in the library's static device workspace (no allocation;
    AEpi.ws is ignored; calls that overlap on one GPU race)."""
    check(load().vgemm_hl2_noalloc(stream_ptr(stream), ctypes.byref(A), Mp, Mreal, ptr(W), ldw, Np, Nreal, Kp, ptr(cst),
                                   ctypes.byref(E)))


def k_gemm_hl(Ahi, Alo, lda: int, Mp: int, Mreal: int, W, ldw: int, Np: int, Nreal: int, Kp: int, cst, e, Y, ldy: int,
              residual=None, epi: int = EPI_PLAIN, Cs: int = 0, Y1=None, Y2=None, Lphi=None, stream=None) -> None:
    """meow::k_gemm_hl (src/gemm_hl.h:30-33)."""
    check(load().vgemm_hl(stream_ptr(stream), ptr(Ahi), ptr(Alo), lda, Mp, Mreal, ptr(W), ldw, Np, Nreal, Kp, ptr(cst), ptr(e),
                          ptr(Y), ldy, ptr(residual), epi, Cs, ptr(Y1), ptr(Y2), ptr(Lphi)))


def k_conv_e(pm, B: int, H: int, W: int, stride: int, e, stream=None) -> None:
    """meow::k_conv_e (src/gemm_hl.h:29)."""
    check(load().vgemm_conv_e(stream_ptr(stream), ptr(pm), B, H, W, stride, ptr(e)))


def gemm_hl_supported(Mp: int, Np: int, Kp: int) -> bool:
    """meow::gemm_hl_supported (src/gemm_hl.h:34)."""
    return bool(load().vgemm_supported(Mp, Np, Kp))


def set_variant(v: int) -> None:
    """Write meow::g_gemm_hl_variant (src/gemm_hl.h:35): -1 auto, 0 128x128, 1 64x128, 2 128x64,
    3 128x256, 4 row-stationary, 5 K split over the waves of 64x64 tiles."""
    load().vgemm_set_variant(v)


def get_variant() -> int:
    return load().vgemm_get_variant()


def set_splitk(s: int) -> None:
    """Force the split-K partition count for calls with a workspace (0 = automatic)."""
    load().vgemm_set_splitk(s)


def set_tile_order(order: int) -> None:
    """Tile order over the XCDs: -1 automatic, 0 row stripes per XCD, 1 column groups per XCD."""
    load().vgemm_set_tile_order(order)


def conv16_halo_rows(H: int, W: int, C: int, stride: int, epi: int = EPI_PLAIN) -> int:
    """Rows per tile of the halo-reuse 3x3 kernel for this SRC_CONV16 geometry (0: not used)."""
    return int(load().vgemm_conv16_halo_rows(H, W, C, stride, epi))


def workspace_bytes(Mp: int, Mreal: int, Np: int, Nreal: int, Kp: int, epi: int = EPI_PLAIN) -> int:
    return int(load().vgemm_workspace_bytes(Mp, Mreal, Np, Nreal, Kp, epi))


def view_workspace_bytes(Mreal: int, Nreal: int, Kp: int, epi: int = EPI_PLAIN) -> int:
    """Workspace bytes of the int16 view (k_gemm_hl2_view) for an Mreal x Nreal x Kp call."""
    return int(load().vgemm_view_workspace_bytes(Mreal, Nreal, Kp, epi))


class Gemm:
    """meow::Gemm (src/gemm.h:12-23): C[M,N] = A[M,K] * W[N,K]^T, int8 -> int32, strided batch."""

    def __init__(self):
        self._h = ctypes.c_void_p()

    def init(self, ws_bytes: int = 0) -> None:
        check(load().vgemm_i8_create(ws_bytes, ctypes.byref(self._h)))

    def run(self, A, lda: int, strideA: int, W, ldw: int, strideW: int, C, ldc: int, strideC: int, M: int, N: int, K: int,
            batch: int = 1, stream=None) -> None:
        if not self._h:
            raise VgemmError(-1, "Gemm::run before init")
        check(load().vgemm_i8_run(self._h, stream_ptr(stream), ptr(A), lda, strideA, ptr(W), ldw, strideW, ptr(C), ldc, strideC,
                                  M, N, K, batch))

    def __del__(self):
        if getattr(self, "_h", None):
            try:
                load().vgemm_i8_destroy(self._h)
            except Exception:
                pass


def k_quant_rows(X, M: int, K: int, ldx: int, hi, lo, e, Kp: int, stream=None) -> None:
    """meow::k_quant_rows (src/kernels.h:12-13)."""
    check(load().vgemm_quant_rows(stream_ptr(stream), ptr(X), M, K, ldx, ptr(hi), ptr(lo), ptr(e), Kp))


def k_epilogue(Chi, Clo, M: int, N: int, ldc: int, cst, e, Y, ldy: int, residual=None, gs=None, T: int = 0, stream=None) -> None:
    """meow::k_epilogue (src/kernels.h:14-17); gs: GroupNorm statistics records (gn_stats_alloc)."""
    check(load().vgemm_epilogue(stream_ptr(stream), ptr(Chi), ptr(Clo), M, N, ldc, ptr(cst), ptr(e), ptr(Y), ldy, ptr(residual),
                                ptr(gs), T))


def k_pixmax(X, rows: int, C: int, pm, stream=None) -> None:
    """meow::k_pixmax (src/kernels.h:18-19)."""
    check(load().vgemm_pixmax(stream_ptr(stream), ptr(X), rows, C, ptr(pm)))


def k_im2col3(X, pm, B: int, H: int, W: int, C: int, stride: int, hi, lo, e, Kp: int, stream=None) -> None:
    """meow::k_im2col3 (src/kernels.h:20-21)."""
    check(load().vgemm_im2col3(stream_ptr(stream), ptr(X), ptr(pm), B, H, W, C, stride, ptr(hi), ptr(lo), ptr(e), Kp))


def k_epilogue_split(Chi, Clo, M: int, N: int, ldc: int, cst, e, Cs: int, Y0, Y1, Y2, stream=None) -> None:
    """meow::k_epilogue_split (src/kernels.h:68-69)."""
    check(load().vgemm_epilogue_split(stream_ptr(stream), ptr(Chi), ptr(Clo), M, N, ldc, ptr(cst), ptr(e), Cs, ptr(Y0), ptr(Y1), ptr(Y2)))


def k_epilogue_geglu_q(Chi, Clo, M: int, F: int, ldc: int, cst, e, Lphi, hi, lo, eo, Kp: int, stream=None) -> None:
    """meow::k_epilogue_geglu_q (src/kernels.h:70)."""
    check(load().vgemm_epilogue_geglu_q(stream_ptr(stream), ptr(Chi), ptr(Clo), M, F, ldc, ptr(cst), ptr(e), ptr(Lphi), ptr(hi), ptr(lo),
                                        ptr(eo), Kp))


def gn_stats_alloc(count: int, device="cuda") -> torch.Tensor:
    """Device memory for `count` GnStat records (48 bytes each, 16-byte aligned), as a uint8 tensor."""
    return torch.empty(count * GNSTAT_BYTES, dtype=torch.uint8, device=device)


def k_gn_init(gs, count: int, stream=None) -> None:
    """meow::k_gn_init (src/kernels.h:25): sum = ss = 0, mn = INT_MAX, mx = INT_MIN."""
    check(load().vgemm_gn_init(stream_ptr(stream), ptr(gs), count))


def gn_stats_read(gs, count: int) -> dict:
    """The sum, mn and mx fields of `count` records as int64 numpy arrays (a host copy)."""
    raw = gs[: count * GNSTAT_BYTES].cpu().numpy().reshape(count, GNSTAT_BYTES)
    out = {}
    for name, dt in (("sum", "<i8"), ("mn", "<i4"), ("mx", "<i4")):
        o = GNSTAT_OFFSETS[name]
        w = 8 if dt == "<i8" else 4
        out[name] = raw[:, o:o + w].copy().view(dt).reshape(count).astype("int64")
    return out


def fill_u32(t, value: int = 0, stream=None) -> None:
    """Fill a uint32/int32 tensor by a kernel (capture-safe; no hipMemsetAsync)."""
    check(load().vgemm_fill_u32(stream_ptr(stream), ptr(t), t.numel() * t.element_size() // 4, value & 0xFFFFFFFF))


class Graph:
    """A captured GEMM sequence (src/engine.cu:625-630): capture() on a non-default stream, then replay()."""

    def __init__(self, stream: torch.cuda.Stream):
        self.stream = stream
        self._exec = ctypes.c_void_p()

    def begin(self) -> None:
        check(load().vgemm_graph_begin(stream_ptr(self.stream)))

    def end(self) -> None:
        check(load().vgemm_graph_end(stream_ptr(self.stream), ctypes.byref(self._exec)))

    def replay(self) -> None:
        check(load().vgemm_graph_launch(self._exec, stream_ptr(self.stream)))

    def destroy(self) -> None:
        if self._exec:
            check(load().vgemm_graph_destroy(self._exec))
            self._exec = ctypes.c_void_p()

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

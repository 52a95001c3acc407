"""Python mirror of the reference's elementwise launchers between the GEMMs over the C ABI of
libvgemm.so: meow::k_act / k_geglu / k_add / k_concat / k_upsample2 (src/kernels.h:31-35), same
argument order and meaning; a failed check raises VgemmError where the reference throws.
"""
from __future__ import annotations

from ._lib import check, load
from .gemm import ptr, stream_ptr

__all__ = ["k_act", "k_geglu", "k_add", "k_concat", "k_upsample2"]


def k_act(X, n: int, L, stream=None) -> None:
    """meow::k_act: x = sat32(rshr(x lut16i(x, L), 16)) in place (SiLU with lut.sigmoid, GELU with lut.phi)."""
    check(load().vgemm_act(stream_ptr(stream), ptr(X), n, ptr(L)))


def k_geglu(A, G, n: int, L, stream=None) -> None:
    """meow::k_geglu: a = sat32(rshr(a sat32(rshr(g lut16i(g, L), 16)), 16)) in place."""
    check(load().vgemm_geglu(stream_ptr(stream), ptr(A), ptr(G), n, ptr(L)))


def k_add(X, Y, n: int, stream=None) -> None:
    """meow::k_add: x = sat32(x + y) in place."""
    check(load().vgemm_add(stream_ptr(stream), ptr(X), ptr(Y), n))


def k_concat(A, Ca: int, B, Cb: int, rows: int, out, gs=None, T: int = 0, stream=None) -> None:
    """meow::k_concat: out[r] = [A[r] | B[r]], with the GroupNorm records of out when gs is given."""
    check(load().vgemm_concat(stream_ptr(stream), ptr(A), Ca, ptr(B), Cb, rows, ptr(out), ptr(gs), T))


def k_upsample2(X, B: int, H: int, W: int, C: int, out, stream=None) -> None:
    """meow::k_upsample2: nearest-neighbour x2 of the NHWC image X into out [B, 2H, 2W, C]."""
    check(load().vgemm_upsample2(stream_ptr(stream), ptr(X), B, H, W, C, ptr(out)))

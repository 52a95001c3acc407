"""Python mirror of the reference's attention launchers over the C ABI of libvgemm.so:
meow::k_quant_heads / k_quant_heads_pad / k_quant_v / k_fused_attention (src/kernels.h:42-50,61,73-77),
same argument order and meaning. Heads of 64 values; a failed check raises VgemmError where the
reference throws ("fused attention: Tqp/Tkp alignment").
"""
from __future__ import annotations

from ._lib import check, load
from .gemm import ptr, stream_ptr

__all__ = ["k_quant_heads", "k_quant_heads_pad", "k_quant_v", "k_fused_attention"]


def k_quant_heads(X, B: int, T: int, C: int, heads: int, Tp: int, hi, lo, e, hs, ls, tsum, stream=None) -> None:
    """meow::k_quant_heads: X[B, T, C] -> planes [B*heads*Tp x 64], e / hs / ls / tsum per row (rows t >= T: value 0)."""
    check(load().vgemm_quant_heads(stream_ptr(stream), ptr(X), B, T, C, heads, Tp, ptr(hi), ptr(lo), ptr(e), ptr(hs), ptr(ls), ptr(tsum)))


def k_quant_heads_pad(G: int, T: int, Tp: int, hi, lo, e, hs, ls, tsum, stream=None) -> None:
    """meow::k_quant_heads_pad: rows t in [T, Tp) of every group take the value 0."""
    check(load().vgemm_quant_heads_pad(stream_ptr(stream), G, T, Tp, ptr(hi), ptr(lo), ptr(e), ptr(hs), ptr(ls), ptr(tsum)))


def k_quant_v(X, B: int, Tk: int, C: int, heads: int, Tkp: int, vthi, vtlo, ev, vsum, scratch=None, stream=None) -> None:
    """meow::k_quant_v: X[B, Tk, C] -> transposed planes [B*heads*64 x Tkp], ev and vsum per (g, d)."""
    check(load().vgemm_quant_v(stream_ptr(stream), ptr(X), B, Tk, C, heads, Tkp, ptr(vthi), ptr(vtlo), ptr(ev), ptr(vsum), ptr(scratch)))


def k_fused_attention(qhi, qlo, eq, qhs, qls, khi, klo, ek, ksum, vthi, vtlo, ev, vsum, B: int, heads: int, Tq: int, Tqp: int, Tk: int,
                      Tkp: int, causal: bool, Lexp, C: int, gmx, gr, out, rowmax=None, stream=None) -> None:
    """meow::k_fused_attention: out[B, Tq, C] (head h at columns h*64..), rowmax[b*Tq + q] = max |out| (optional)."""
    check(load().vgemm_fused_attention(stream_ptr(stream), ptr(qhi), ptr(qlo), ptr(eq), ptr(qhs), ptr(qls), ptr(khi), ptr(klo), ptr(ek),
                                       ptr(ksum), ptr(vthi), ptr(vtlo), ptr(ev), ptr(vsum), B, heads, Tq, Tqp, Tk, Tkp, 1 if causal else 0,
                                       ptr(Lexp), C, ptr(gmx), ptr(gr), ptr(out), ptr(rowmax)))

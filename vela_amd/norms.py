"""Python mirror of the reference's integer normalisation launchers over the C ABI of libvgemm.so:
meow::k_gn_stats1 / k_gn_fin1 / k_gn_stats2 / k_gn_apply / k_gn_apply_row / k_lnorm / k_lnorm_q
(src/kernels.h:21-24,59-63,66-67), same argument order and meaning. Records are GnStat (48 bytes,
vela_amd.gemm.gn_stats_alloc); a failed check raises VgemmError where the reference throws.
"""
from __future__ import annotations

from ._lib import check, load
from .gemm import ptr, stream_ptr

__all__ = ["k_gn_stats1", "k_gn_fin1", "k_gn_stats2", "k_gn_apply", "k_gn_apply_row", "k_lnorm", "k_lnorm_q"]


def k_gn_stats1(X, B: int, T: int, C: int, groups: int, gs, stream=None) -> None:
    """meow::k_gn_stats1: init the B*groups records, gather sum/min/max, then fin1."""
    check(load().vgemm_gn_stats1(stream_ptr(stream), ptr(X), B, T, C, groups, ptr(gs)))


def k_gn_fin1(gs, cnt: int, n: int, stream=None) -> None:
    """meow::k_gn_fin1: mean and shift e of records whose sum/min/max a GEMM epilogue gathered."""
    check(load().vgemm_gn_fin1(stream_ptr(stream), ptr(gs), cnt, n))


def k_gn_stats2(X, B: int, T: int, C: int, groups: int, den: int, gs, stream=None) -> None:
    """meow::k_gn_stats2: squared deviations, then fin2 (sd)."""
    check(load().vgemm_gn_stats2(stream_ptr(stream), ptr(X), B, T, C, groups, den, ptr(gs)))


def k_gn_apply(X, B: int, T: int, C: int, groups: int, gs, g64, beta64, Y, stream=None) -> None:
    """meow::k_gn_apply (64-bit g, beta)."""
    check(load().vgemm_gn_apply(stream_ptr(stream), ptr(X), B, T, C, groups, ptr(gs), ptr(g64), ptr(beta64), ptr(Y)))


def k_gn_apply_row(X, B: int, T: int, C: int, groups: int, gs, g, beta, Lsig, Y, pm, hi, lo, e, Kp: int, stream=None) -> None:
    """meow::k_gn_apply_row: + SiLU (Lsig), int32 Y plus the row maxima pm, or the int16 view."""
    check(load().vgemm_gn_apply_row(stream_ptr(stream), ptr(X), B, T, C, groups, ptr(gs), ptr(g), ptr(beta), ptr(Lsig), ptr(Y), ptr(pm),
                                    ptr(hi), ptr(lo), ptr(e), Kp))


def k_lnorm(X, M: int, C: int, g64, beta64, den: int, Y, stream=None) -> None:
    """meow::k_lnorm (64-bit g, beta)."""
    check(load().vgemm_lnorm(stream_ptr(stream), ptr(X), M, C, ptr(g64), ptr(beta64), den, ptr(Y)))


def k_lnorm_q(X, M: int, C: int, g, beta, den: int, hi, lo, e, Kp: int, stream=None) -> None:
    """meow::k_lnorm_q: the int16 view of the normalised row."""
    check(load().vgemm_lnorm_q(stream_ptr(stream), ptr(X), M, C, ptr(g), ptr(beta), den, ptr(hi), ptr(lo), ptr(e), Kp))

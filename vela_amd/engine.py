"""Python mirror of the reference engine's blocks over the C ABI of libvgemm.so (include/vgemm_engine.h).

  Engine       meow::Engine (src/engine.h:58-116) for an uploaded DevModel: an arena of device memory
               allocated once; resnet (src/engine.cu:389-405), transformer (src/engine.cu:406-454) and the
               cross-attention K/V of setPrompt (src/engine.cu:540-560) for one block and a context of
               B samples. gn_fuse = EngineConfig::gnFuse; fusedAttention, fusedLoader and customGemmMaxK
               stay at the reference's defaults.

Activations are torch int32 CUDA tensors [B * T, C] (NHWC rows); GroupNorm records are uint8 CUDA
tensors of B * 32 VgemmGnStat records (48 bytes each). A failed check raises VgemmError where the
reference throws std::runtime_error.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import GNSTAT_BYTES, Activation, check, load
from .gemm import ptr, stream_ptr
from .model import DevModel

__all__ = ["Engine"]


def _act(x: torch.Tensor | None, B: int, T: int, C: int, rowmax=None, gnst=None) -> Activation:
    a = Activation()
    a.d = ptr(x)
    a.B, a.T, a.C = B, T, C
    a.rowmax = ptr(rowmax)
    a.gnst = ptr(gnst)
    return a


class Engine:
    """meow::Engine's blocks on one uploaded model (DevModel.load first)."""

    def __init__(self, dm: DevModel, arena_bytes: int, gn_fuse: bool = False):
        if dm.model is None or dm.device < 0:
            raise ValueError("Engine: the DevModel must be loaded onto a device first")
        self.dm = dm
        self._h = ctypes.c_void_p()
        check(load().vgemm_engine_create(dm.model.handle, arena_bytes, 1 if gn_fuse else 0, ctypes.byref(self._h)))

    def close(self) -> None:
        if self._h:
            load().vgemm_engine_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def arena_peak(self) -> int:
        """Engine::arenaPeak (src/engine.h:69): the arena's high-water mark so far, in bytes."""
        return int(load().vgemm_engine_arena_peak(self._h))

    @staticmethod
    def records(B: int, device="cuda") -> torch.Tensor:
        """Device memory for the GroupNorm records of a B-sample activation."""
        return torch.zeros(B * 32 * GNSTAT_BYTES, dtype=torch.uint8, device=device)

    def resnet(self, x: torch.Tensor, B: int, H: int, W: int, prefix: str, out: torch.Tensor, out_gnst=None, x_gnst=None,
               stream=None) -> bool:
        """Engine::resnet of "<prefix>" on x [B * H * W, C] into out [B * H * W, N]; True when out_gnst
        received the output's GroupNorm records (gn_fuse and a fusable shape)."""
        a = _act(x, B, H * W, x.shape[1], gnst=x_gnst)
        o = _act(out, B, H * W, out.shape[1], gnst=out_gnst)
        check(load().vgemm_engine_resnet(self._h, stream_ptr(stream), ctypes.byref(a), H, W, prefix.encode(), ctypes.byref(o)))
        return bool(o.gnst)

    def set_context(self, ctx: torch.Tensor, B: int, Tc: int, block: str, heads: int, stream=None) -> None:
        """The cross-attention K/V of "<block>" (…transformer_blocks.0) from ctx [B * Tc, Cc]."""
        a = _act(ctx, B, Tc, ctx.shape[1])
        check(load().vgemm_engine_set_context(self._h, stream_ptr(stream), ctypes.byref(a), block.encode(), heads))

    def transformer(self, x: torch.Tensor, B: int, T: int, prefix: str, heads: int, out: torch.Tensor, out_gnst=None, x_gnst=None,
                    stream=None) -> bool:
        """Engine::transformer of "<prefix>" on x [B * T, C] into out [B * T, C]; True when out_gnst
        received the output's GroupNorm records."""
        a = _act(x, B, T, x.shape[1], gnst=x_gnst)
        o = _act(out, B, T, out.shape[1], gnst=out_gnst)
        check(load().vgemm_engine_transformer(self._h, stream_ptr(stream), ctypes.byref(a), prefix.encode(), heads, ctypes.byref(o)))
        return bool(o.gnst)

"""The UNet GEMM set: the 194 linear/conv GEMMs of an SD-turbo-sized UNet
forward at batch 8, every input seeded and resident in HBM, captured once into one hipGraph and
replayed (the reference captures its whole forward the same way, src/engine.cu:625-630, 661-667).

All layers share one split-K workspace: they run in order on one stream, so the workspace is never
used by two GEMMs at once.
"""
from __future__ import annotations

import torch

from . import configs as cf
from . import gemm as vg


class GemmSet:
    def __init__(self, layers: list[cf.Layer] | None = None, device: str = "cuda", keep_host: bool = False):
        self.layers = layers if layers is not None else cf.unet_layers()
        ws_bytes = max(vg.workspace_bytes(L.Mp, L.M, L.Np, L.N, L.Kp, L.epi) for L in self.layers)
        self.ws = torch.empty(max(ws_bytes // 4, 1) + 64, dtype=torch.int32, device=device) if ws_bytes else None
        self.probs: list[cf.DeviceProblem] = []
        for L in self.layers:
            p = cf.DeviceProblem(L, device=device, with_ws=False)
            if self.ws is not None and vg.workspace_bytes(L.Mp, L.M, L.Np, L.N, L.Kp, L.epi):
                p.E.ws = vg.ptr(self.ws)
                p.E.ws_bytes = self.ws.numel() * 4
            if not keep_host:
                p.h = None   # regenerated from the seed when checked
            self.probs.append(p)
        self.stream = torch.cuda.Stream(device=device)
        self.graph: vg.Graph | None = None

    @property
    def ops(self) -> int:
        return sum(L.ops for L in self.layers)

    def _enqueue(self, reseed: bool = True):
        for p in self.probs:
            if reseed:
                p.reset()
            elif p.rowmax is not None:
                vg.fill_u32(p.rowmax, 0)
            p.run(stream=self.stream)

    def run_eager(self):
        with torch.cuda.stream(self.stream):
            self._enqueue()

    def capture(self, reseed: bool = True):
        """Capture the whole set into one graph: for each layer in forward order, rowmax zeroing by a
        kernel (the engine clears every rowmax buffer it allocates, src/engine.cu:161) and the GEMM.
        With reseed, residual layers first copy their seeded residual back into Y, so that every
        replay computes the same bytes (the parity tests); without it, Y accumulates in place from
        replay to replay as the forward's residual stream does, and the graph holds only the GEMMs,
        the rowmax fills and conv_in's pixel-max and im2col3 passes (the timed C5 set)."""
        self.run_eager()                      # first calls outside capture
        self.stream.synchronize()
        self.graph = vg.Graph(self.stream)
        with torch.cuda.stream(self.stream):
            self.graph.begin()
            self._enqueue(reseed)
            self.graph.end()

    def replay(self):
        self.graph.replay()

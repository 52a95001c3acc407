"""Python mirror of the reference's model-file reader and device model over the C ABI of libvgemm.so
(include/vgemm_model.h).

  Poisd     meow::Poisd (src/poisd.h:10-36, src/poisd.cpp:11-64): load, entries, has, get, i8, i32v,
            i32s, blob. load raises VgemmError with the reference's message where Poisd::load returns
            false with it.
  DevModel  meow::DevModel (src/engine.h:16-37, src/engine.cu:11-104): load(device, model) prepares
            every linear (padding, tap-major 3x3 convolutions, wsum, cst) and the merged projections
            and copies them to the device; lin / has_lin / norm as the reference's accessors.

Device pointers are returned as ints (valid until the Poisd is closed); host arrays are copies.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from ._lib import Lin as _Lin, Norm as _Norm, Tensor as _Tensor, VgemmError, check, load

DTYPES = {0: np.int8, 1: np.int16, 2: np.int32, 3: np.uint8}

__all__ = ["Poisd", "PoisdTensor", "DevModel", "Lin", "Norm", "DTYPES"]


@dataclass
class PoisdTensor:
    """meow::PoisdTensor (src/poisd.h:10-16)."""

    dtype: int
    dims: list
    off: int
    count: int

    def bytes(self) -> int:
        return self.count * np.dtype(DTYPES[self.dtype]).itemsize


class Poisd:
    """meow::Poisd over vgemm_model_open: the file is mapped, not read into memory."""

    def __init__(self):
        self._h = ctypes.c_void_p()

    def load(self, path: str) -> None:
        self.close()
        check(load().vgemm_model_open(str(path).encode(), ctypes.byref(self._h)))

    def close(self) -> None:
        if self._h:
            load().vgemm_model_close(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        if not self._h:
            raise VgemmError(-1, "model not loaded")
        return self._h

    def names(self) -> list[str]:
        lib = load()
        return [lib.vgemm_model_name(self.handle, i).decode() for i in range(lib.vgemm_model_count(self.handle))]

    def _tensor(self, name: str) -> _Tensor:
        t = _Tensor()
        check(load().vgemm_model_tensor(self.handle, name.encode(), ctypes.byref(t)))
        return t

    def get(self, name: str) -> PoisdTensor:
        t = self._tensor(name)
        return PoisdTensor(t.dtype, [int(t.dims[d]) for d in range(min(t.rank, 8))], int(t.offset), int(t.count))

    def entries(self) -> dict:
        return {n: self.get(n) for n in self.names()}

    def has(self, name: str) -> bool:
        return name in set(self.names())

    def array(self, name: str) -> np.ndarray:
        """The tensor's data with its dtype and dims (a copy)."""
        t = self._tensor(name)
        raw = ctypes.string_at(t.data, t.bytes) if t.bytes else b""
        dims = [int(t.dims[d]) for d in range(min(t.rank, 8))]
        return np.frombuffer(raw, dtype=np.dtype(DTYPES[t.dtype]).newbyteorder("<")).reshape(dims).copy()

    def i8(self, name: str) -> np.ndarray:
        if self.get(name).dtype != 0:
            raise VgemmError(-4, f"{name} is not int8")
        return self.array(name)

    def i32v(self, name: str) -> np.ndarray:
        """int32 tensor widened to int64, flat (src/poisd.cpp:60-63)."""
        if self.get(name).dtype != 2:
            raise VgemmError(-4, f"{name} is not int32")
        return self.array(name).reshape(-1).astype(np.int64)

    def i32s(self, name: str) -> int:
        return int(self.i32v(name)[0])

    def blob(self, name: str) -> bytes:
        t = self._tensor(name)
        return ctypes.string_at(t.data, t.bytes) if t.bytes else b""


@dataclass
class Lin:
    """meow::Lin (src/engine.h:12): w / cst device addresses (0 before upload), host copies."""

    N: int
    K: int
    Np: int
    Kp: int
    conv3: bool
    w: int
    cst: int
    w_host: np.ndarray
    cst_host: np.ndarray


@dataclass
class Norm:
    """meow::Norm (src/engine.h:13): Q16 g / beta [C] and den."""

    C: int
    den: int
    g: int
    beta: int
    g_host: np.ndarray
    beta_host: np.ndarray


def _host(addr, n, dtype):
    if not addr or n == 0:
        return np.zeros(0, dtype)
    return np.frombuffer(ctypes.string_at(addr, n * np.dtype(dtype).itemsize), dtype=dtype).copy()


class DevModel:
    """meow::DevModel: the prepared GEMM operands of one model on one device."""

    def __init__(self):
        self.model: Poisd | None = None
        self.device = -1

    def prepare(self, model: Poisd) -> None:
        """The host half of DevModel::load only (no device work)."""
        check(load().vgemm_model_prepare(model.handle))
        self.model = model

    def load(self, device: int, model: Poisd) -> None:
        """DevModel::load (src/engine.cu:11-70): prepare and copy to `device`."""
        check(load().vgemm_model_upload(model.handle, device))
        self.model, self.device = model, device

    @property
    def bytes(self) -> int:
        return int(load().vgemm_model_device_bytes(self.model.handle)) if self.model else 0

    def lin_names(self) -> list[str]:
        lib = load()
        h = self.model.handle
        return [lib.vgemm_model_lin_name(h, i).decode() for i in range(lib.vgemm_model_lin_count(h))]

    def has_lin(self, name: str) -> bool:
        return name in set(self.lin_names())

    def lin(self, name: str) -> Lin:
        L = _Lin()
        check(load().vgemm_model_lin(self.model.handle, name.encode(), ctypes.byref(L)))
        return Lin(L.N, L.K, L.Np, L.Kp, bool(L.conv3), L.w or 0, L.cst or 0,
                   _host(L.w_host, L.Np * L.Kp, np.int8).reshape(L.Np, L.Kp), _host(L.cst_host, L.Np * 4, np.int32).reshape(L.Np, 4))

    def norm(self, name: str) -> Norm:
        n = _Norm()
        check(load().vgemm_model_norm(self.model.handle, name.encode(), ctypes.byref(n)))
        return Norm(n.C, n.den, n.g or 0, n.beta or 0, _host(n.g_host, n.C, np.int32), _host(n.beta_host, n.C, np.int32))

    def table(self, name: str) -> tuple[int, int]:
        """(device address, count) of an int32 table: "lut.phi" (DevModel::lutPhi32) or "lut.sigmoid"."""
        p, c = ctypes.c_void_p(), ctypes.c_int()
        check(load().vgemm_model_table(self.model.handle, name.encode(), ctypes.byref(p), ctypes.byref(c)))
        return int(p.value or 0), int(c.value)

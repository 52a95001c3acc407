"""Seeded synthetic inputs (numpy arrays) from libvela_datagen.so (vela_amd/csrc/datagen.c).

Every generator is a pure function of (n, seed, distribution parameters): splitmix64-seeded
xoshiro256** streams per 65536-element chunk, independent of the thread count.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_PATH = Path(__file__).resolve().parent / "libvela_datagen.so"
_lib = None

_D, _I, _LL, _SZ, _U64, _P = ctypes.c_double, ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_void_p
_SIGS = {
    "vdg_i16_gauss": [_P, _SZ, _U64, _D, _I, _I],
    "vdg_i8_gauss": [_P, _SZ, _U64, _D, _I, _I],
    "vdg_i32_gauss": [_P, _SZ, _U64, _D, _LL, _LL],
    "vdg_i16_laplace": [_P, _SZ, _U64, _D, _I, _I],
    "vdg_i8_uniform": [_P, _SZ, _U64, _I, _I],
    "vdg_i16_uniform": [_P, _SZ, _U64, _I, _I],
    "vdg_i32_uniform": [_P, _SZ, _U64, _LL, _LL],
    "vdg_i32_bits": [_P, _SZ, _U64, _I],
}


def _load():
    global _lib
    if _lib is None:
        if not _PATH.exists():
            raise RuntimeError(f"{_PATH} is not built: run `python -m vela_amd.build`")
        lib = ctypes.CDLL(str(_PATH))
        for name, args in _SIGS.items():
            getattr(lib, name).restype = None
            getattr(lib, name).argtypes = args
        _lib = lib
    return _lib


def _fill(name, dtype, shape, seed, *args):
    out = np.empty(shape, dtype=dtype)
    getattr(_load(), name)(out.ctypes.data, out.size, seed & 0xFFFFFFFFFFFFFFFF, *args)
    return out


def i16_gauss(shape, seed, sigma, lo=-32767, hi=32767):
    return _fill("vdg_i16_gauss", np.int16, shape, seed, float(sigma), lo, hi)


def i16_laplace(shape, seed, b, lo=-32767, hi=32767):
    return _fill("vdg_i16_laplace", np.int16, shape, seed, float(b), lo, hi)


def i16_uniform(shape, seed, lo=-32768, hi=32767):
    return _fill("vdg_i16_uniform", np.int16, shape, seed, lo, hi)


def i8_uniform(shape, seed, lo=-127, hi=127):
    return _fill("vdg_i8_uniform", np.int8, shape, seed, lo, hi)


def i8_gauss(shape, seed, sigma, lo=-127, hi=127):
    return _fill("vdg_i8_gauss", np.int8, shape, seed, float(sigma), lo, hi)


def i32_uniform(shape, seed, lo, hi):
    return _fill("vdg_i32_uniform", np.int32, shape, seed, int(lo), int(hi))


def i32_gauss(shape, seed, sigma, lo=-(2**31), hi=2**31 - 1):
    return _fill("vdg_i32_gauss", np.int32, shape, seed, float(sigma), int(lo), int(hi))


def i32_bits(shape, seed, maxbits=31):
    """Signed values of a uniformly drawn bit width in [1, maxbits] (saturation and e up to 17)."""
    return _fill("vdg_i32_bits", np.int32, shape, seed, int(maxbits))

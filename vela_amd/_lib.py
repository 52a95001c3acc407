"""Loader for the in-tree libvgemm.so (the HIP kernels behind the C ABI of include/vgemm.h).

torch is imported first so that the HIP runtime torch ships (SONAME libamdhip64.so.7) is the one
libvgemm.so binds to: device pointers and streams from torch are then valid in the library. There is
no fallback: if the library is missing or does not load, every call raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the dlopen below)

LIB_PATH = Path(__file__).resolve().parent / "libvgemm.so"

P = ctypes.c_void_p
I = ctypes.c_int
LL = ctypes.c_longlong
SZ = ctypes.c_size_t
U32 = ctypes.c_uint32


class ASrc(ctypes.Structure):
    """VgemmASrc (include/vgemm.h) == meow::ASrc (src/gemm_hl.h:12-17) plus the int16 sources."""

    _fields_ = [
        ("src", I),
        ("hi", P), ("lo", P), ("ld8", I), ("e", P),
        ("x", P), ("ldx", I), ("rowmax", P), ("K", I),
        ("img", P), ("H", I), ("W", I), ("C", I), ("stride", I), ("Ho", I), ("Wo", I),
        ("q16", P), ("ld16", I),
        ("img16", P),
    ]

    def __init__(self, **kw):
        super().__init__()
        self.src = 0
        self.stride = 1
        for k, v in kw.items():
            setattr(self, k, v)


class GnStat(ctypes.Structure):
    """VgemmGnStat (include/vgemm.h) == meow::GnStat (src/kernels.h:9), 48 bytes."""

    _fields_ = [("sum", LL), ("mn", I), ("mx", I), ("mean", LL), ("e", I), ("ss", LL), ("sd", LL)]


GNSTAT_BYTES = ctypes.sizeof(GnStat)
# field offsets, for reading records out of a device buffer viewed as bytes
GNSTAT_OFFSETS = {name: getattr(GnStat, name).offset for name, _ in GnStat._fields_}


class AEpi(ctypes.Structure):
    """VgemmAEpi (include/vgemm.h) == meow::AEpi (src/gemm_hl.h:18-26) plus the split-K workspace."""

    _fields_ = [
        ("epi", I), ("Y", P), ("ldy", I), ("residual", P),
        ("Cs", I), ("Y1", P), ("Y2", P), ("Lphi", P),
        ("rowmax", P),
        ("gnstat", P), ("gnT", I),
        ("heads", I), ("T", I), ("TpQ", I), ("TpK", I), ("C", I),
        ("qhi", P), ("qlo", P), ("khi", P), ("klo", P), ("qe", P), ("ke", P),
        ("qhs", P), ("qls", P), ("qts", P), ("khs", P), ("kls", P), ("kts", P),
        ("ws", P), ("ws_bytes", SZ),
    ]

    def __init__(self, **kw):
        super().__init__()
        for k, v in kw.items():
            setattr(self, k, v)


class View(ctypes.Structure):
    """VgemmView (include/vgemm.h): the int16 view of a GEMM's output (vgemm_hl2_view)."""

    _fields_ = [("hi", P), ("lo", P), ("e", P), ("ld", I)]

    def __init__(self, **kw):
        super().__init__()
        for k, v in kw.items():
            setattr(self, k, v)


class Tensor(ctypes.Structure):
    """VgemmTensor (include/vgemm_model.h) == meow::PoisdTensor (src/poisd.h:10-16) plus a host pointer."""

    _fields_ = [("dtype", I), ("rank", I), ("dims", ctypes.c_uint32 * 8), ("count", SZ), ("offset", SZ), ("bytes", SZ),
                ("data", P)]


class Lin(ctypes.Structure):
    """VgemmLin (include/vgemm_model.h) == meow::Lin (src/engine.h:12)."""

    _fields_ = [("N", I), ("K", I), ("Np", I), ("Kp", I), ("conv3", I), ("w_host", P), ("cst_host", P), ("w", P), ("cst", P)]


class Norm(ctypes.Structure):
    """VgemmNorm (include/vgemm_model.h) == meow::Norm (src/engine.h:13)."""

    _fields_ = [("C", I), ("den", LL), ("g_host", P), ("beta_host", P), ("g", P), ("beta", P)]


class Activation(ctypes.Structure):
    """VgemmActivation (include/vgemm_engine.h) == meow::Tensor (src/engine.h:36)."""

    _fields_ = [("d", P), ("B", I), ("T", I), ("C", I), ("rowmax", P), ("gnst", P)]


# (name, restype, argtypes) of every entry point declared in include/vgemm.h, include/vgemm_model.h and
# include/vgemm_engine.h
SIGNATURES = [
    ("vgemm_asrc_init", None, [ctypes.POINTER(ASrc)]),
    ("vgemm_aepi_init", None, [ctypes.POINTER(AEpi)]),
    ("vgemm_hl2", I, [P, ctypes.POINTER(ASrc), I, I, P, I, I, I, I, P, ctypes.POINTER(AEpi)]),
    ("vgemm_hl2_noalloc", I, [P, ctypes.POINTER(ASrc), I, I, P, I, I, I, I, P, ctypes.POINTER(AEpi)]),
    ("vgemm_hl2_view", I, [P, ctypes.POINTER(ASrc), I, I, P, I, I, I, I, P, ctypes.POINTER(AEpi), ctypes.POINTER(View)]),
    ("vgemm_hl", I, [P, P, P, I, I, I, P, I, I, I, I, P, P, P, I, P, I, I, P, P, P]),
    ("vgemm_conv_e", I, [P, P, I, I, I, I, P]),
    ("vgemm_supported", I, [I, I, I]),
    ("vgemm_set_variant", None, [I]),
    ("vgemm_get_variant", I, []),
    ("vgemm_set_splitk", None, [I]),
    ("vgemm_set_tile_order", None, [I]),
    ("vgemm_conv16_halo_rows", I, [I, I, I, I, I]),
    ("vgemm_workspace_bytes", SZ, [I, I, I, I, I, I]),
    ("vgemm_view_workspace_bytes", SZ, [I, I, I, I]),
    ("vgemm_i8_create", I, [SZ, ctypes.POINTER(P)]),
    ("vgemm_i8_destroy", I, [P]),
    ("vgemm_i8_run", I, [P, P, P, I, LL, P, I, LL, P, I, LL, I, I, I, I]),
    ("vgemm_quant_rows", I, [P, P, I, I, I, P, P, P, I]),
    ("vgemm_epilogue", I, [P, P, P, I, I, I, P, P, P, I, P, P, I]),
    ("vgemm_pixmax", I, [P, P, I, I, P]),
    ("vgemm_im2col3", I, [P, P, P, I, I, I, I, I, P, P, P, I]),
    ("vgemm_epilogue_split", I, [P, P, P, I, I, I, P, P, I, P, P, P]),
    ("vgemm_epilogue_geglu_q", I, [P, P, P, I, I, I, P, P, P, P, P, P, I]),
    ("vgemm_graph_begin", I, [P]),
    ("vgemm_graph_end", I, [P, ctypes.POINTER(P)]),
    ("vgemm_graph_launch", I, [P, P]),
    ("vgemm_graph_destroy", I, [P]),
    ("vgemm_fill_u32", I, [P, P, SZ, U32]),
    ("vgemm_gn_init", I, [P, P, I]),
    ("vgemm_gn_stats1", I, [P, P, I, I, I, I, P]),
    ("vgemm_gn_fin1", I, [P, P, I, LL]),
    ("vgemm_gn_stats2", I, [P, P, I, I, I, I, LL, P]),
    ("vgemm_gn_apply", I, [P, P, I, I, I, I, P, P, P, P]),
    ("vgemm_gn_apply_row", I, [P, P, I, I, I, I, P, P, P, P, P, P, P, P, P, I]),
    ("vgemm_lnorm", I, [P, P, I, I, P, P, LL, P]),
    ("vgemm_lnorm_q", I, [P, P, I, I, P, P, LL, P, P, P, I]),
    ("vgemm_quant_heads", I, [P, P, I, I, I, I, I, P, P, P, P, P, P]),
    ("vgemm_quant_heads_pad", I, [P, I, I, I, P, P, P, P, P, P]),
    ("vgemm_quant_v", I, [P, P, I, I, I, I, I, P, P, P, P, P]),
    ("vgemm_fused_attention", I, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, P, I, P, P, P, P]),
    ("vgemm_model_open", I, [ctypes.c_char_p, ctypes.POINTER(P)]),
    ("vgemm_model_close", None, [P]),
    ("vgemm_model_count", I, [P]),
    ("vgemm_model_name", ctypes.c_char_p, [P, I]),
    ("vgemm_model_tensor", I, [P, ctypes.c_char_p, ctypes.POINTER(Tensor)]),
    ("vgemm_model_prepare", I, [P]),
    ("vgemm_model_upload", I, [P, I]),
    ("vgemm_model_device_bytes", SZ, [P]),
    ("vgemm_model_lin", I, [P, ctypes.c_char_p, ctypes.POINTER(Lin)]),
    ("vgemm_model_lin_count", I, [P]),
    ("vgemm_model_lin_name", ctypes.c_char_p, [P, I]),
    ("vgemm_model_norm", I, [P, ctypes.c_char_p, ctypes.POINTER(Norm)]),
    ("vgemm_model_table", I, [P, ctypes.c_char_p, ctypes.POINTER(P), ctypes.POINTER(I)]),
    ("vgemm_last_error", ctypes.c_char_p, []),
    ("vgemm_version", ctypes.c_char_p, []),
    ("vgemm_act", I, [P, P, SZ, P]),
    ("vgemm_geglu", I, [P, P, P, SZ, P]),
    ("vgemm_add", I, [P, P, P, SZ]),
    ("vgemm_concat", I, [P, P, I, P, I, I, P, P, I]),
    ("vgemm_upsample2", I, [P, P, I, I, I, I, P]),
    ("vgemm_set_stream_workspaces", None, [I]),
    ("vgemm_engine_create", I, [P, SZ, I, ctypes.POINTER(P)]),
    ("vgemm_engine_destroy", None, [P]),
    ("vgemm_engine_arena_peak", SZ, [P]),
    ("vgemm_engine_resnet", I, [P, P, ctypes.POINTER(Activation), I, I, ctypes.c_char_p, ctypes.POINTER(Activation)]),
    ("vgemm_engine_set_context", I, [P, P, ctypes.POINTER(Activation), ctypes.c_char_p, I]),
    ("vgemm_engine_transformer", I, [P, P, ctypes.POINTER(Activation), ctypes.c_char_p, I, ctypes.POINTER(Activation)]),
]

_lib = None


def load() -> ctypes.CDLL:
    """Load libvgemm.so (once) and set every prototype; raise if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m vela_amd.build` (there is no fallback path)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES:
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class VgemmError(RuntimeError):
    """A non-zero vgemm return code (the reference throws std::runtime_error at these points)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"vgemm error {code}: {msg}")
        self.code = code


def check(rc: int) -> None:
    if rc != 0:
        raise VgemmError(rc, load().vgemm_last_error().decode())

"""The C ABI of libvgemm.so without a GPU: the library loads, exports every entry point that
include/vgemm.h, include/vgemm_model.h and include/vgemm_engine.h declare, the ctypes mirror of VgemmASrc / VgemmAEpi / VgemmGnStat has the C layout (checked
against a gcc-compiled probe of the header), and argument checks fail the way the reference throws
(src/gemm_hl.cu:351,357; src/gemm.cu:41) before any device work."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from vela_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADERS = [ROOT / "include" / "vgemm.h", ROOT / "include" / "vgemm_model.h", ROOT / "include" / "vgemm_engine.h"]


def declared():
    text = re.sub(r"/\*.*?\*/", "", "\n".join(h.read_text() for h in HEADERS), flags=re.S)
    out = {}
    for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(vgemm_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    decl = declared()
    assert len(decl) >= 26
    sigs = {name: args for name, _, args in _lib.SIGNATURES}
    for name, nargs in decl.items():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in sigs, f"{name} has no ctypes prototype"
        assert len(sigs[name]) == nargs, f"{name}: {len(sigs[name])} ctypes args, header has {nargs}"
    assert set(sigs) == set(decl)


PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#include "vgemm.h"
#include "vgemm_model.h"
#include "vgemm_engine.h"
#define F(T, f) printf(#T " " #f " %zu\n", offsetof(T, f));
int main(void) {
    printf("VgemmASrc sizeof %zu\nVgemmAEpi sizeof %zu\nVgemmGnStat sizeof %zu\n", sizeof(VgemmASrc), sizeof(VgemmAEpi),
           sizeof(VgemmGnStat));
    printf("VgemmTensor sizeof %zu\nVgemmLin sizeof %zu\nVgemmNorm sizeof %zu\n", sizeof(VgemmTensor), sizeof(VgemmLin),
           sizeof(VgemmNorm));
    printf("VgemmActivation sizeof %zu\nVgemmView sizeof %zu\n", sizeof(VgemmActivation), sizeof(VgemmView));
    %FIELDS%
    return 0;
}
"""


STRUCTS = (("VgemmASrc", _lib.ASrc), ("VgemmAEpi", _lib.AEpi), ("VgemmGnStat", _lib.GnStat), ("VgemmTensor", _lib.Tensor),
           ("VgemmLin", _lib.Lin), ("VgemmNorm", _lib.Norm), ("VgemmActivation", _lib.Activation),
           ("VgemmView", _lib.View))


def test_struct_layout_matches_c(tmp_path):
    lines = []
    for T, cls in STRUCTS:
        for f, _ in cls._fields_:
            lines.append(f"F({T}, {f})")
    src = tmp_path / "probe.c"
    src.write_text(PROBE.replace("%FIELDS%", "\n    ".join(lines)))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        T, f, v = line.split()
        got[(T, f)] = int(v)
    for T, cls in STRUCTS:
        assert got[(T, "sizeof")] == ctypes.sizeof(cls), T
        for f, _ in cls._fields_:
            assert got[(T, f)] == getattr(cls, f).offset, f"{T}.{f}"


def test_init_defaults():
    lib = _lib.load()
    a = _lib.ASrc(src=3, K=99)
    lib.vgemm_asrc_init(ctypes.byref(a))
    assert (a.src, a.stride, a.K, a.hi) == (0, 1, 0, None)
    e = _lib.AEpi(epi=2, ldy=5)
    lib.vgemm_aepi_init(ctypes.byref(e))
    assert (e.epi, e.ldy, e.ws_bytes) == (0, 0, 0)


def test_supported_shapes():
    lib = _lib.load()
    assert lib.vgemm_supported(64, 64, 16) == 1
    assert lib.vgemm_supported(32768, 2560, 320) == 1
    for shape in [(63, 64, 16), (64, 65, 16), (64, 64, 8), (0, 64, 16), (64, 64, 0)]:
        assert lib.vgemm_supported(*shape) == 0, shape


FAKE = 1 << 40   # a 16-byte aligned address that is never dereferenced: every case fails validation first


def call_hl2(A, E, Mp=64, Mreal=64, ldw=64, Np=64, Nreal=64, Kp=64):
    lib = _lib.load()
    rc = lib.vgemm_hl2(None, ctypes.byref(A), Mp, Mreal, FAKE, ldw, Np, Nreal, Kp, FAKE, ctypes.byref(E))
    return rc, lib.vgemm_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(Mp=65), -1, "unsupported shape"),
    (dict(Kp=8), -1, "unsupported shape"),
    (dict(Mreal=65), -1, "Mreal/Nreal"),
    (dict(ldw=48), -1, "ldw"),
])
def test_hl2_shape_errors(kw, code, msg):
    A = _lib.ASrc(src=0, hi=FAKE, lo=FAKE, ld8=64)
    E = _lib.AEpi(Y=FAKE, ldy=64)
    rc, err = call_hl2(A, E, **kw)
    assert rc == code and msg in err, err


@pytest.mark.parametrize("asrc,aepi,code,msg", [
    (dict(src=2, img=FAKE, C=12, K=108, H=4, W=4, Ho=4, Wo=4), {}, -1, "conv source"),
    (dict(src=4, img16=FAKE, C=4, K=36, H=4, W=4, Ho=4, Wo=4), {}, -1, "C % 8"),
    (dict(src=4, img16=FAKE, C=8, K=72, H=4, W=4, Ho=3, Wo=4), {}, -1, "Ho/Wo"),
    (dict(src=4, img16=FAKE, C=16, K=144, H=4, W=4, Ho=4, Wo=4), {}, -1, "H/W/stride/Kp"),
    (dict(src=3, q16=FAKE, K=60, ld16=64), {}, -1, "SRC_I16"),
    (dict(src=1, x=FAKE, K=64, ldx=64), {}, -1, "SRC_X32"),
    (dict(src=9), {}, -1, "unknown A source"),
    (dict(src=0, hi=FAKE, lo=FAKE, ld8=64), dict(epi=4), -1, "EPI_QKV needs C = 64*heads"),
    (dict(src=0, hi=FAKE, lo=FAKE, ld8=64), dict(epi=4, heads=1, C=64, T=8, TpQ=8, TpK=8), -1, "Nreal = 3C"),
    (dict(src=0, hi=FAKE, lo=FAKE, ld8=64), dict(gnstat=FAKE), -1, "GroupNorm statistics need"),
    (dict(src=0, hi=FAKE, lo=FAKE, ld8=64), dict(gnstat=FAKE, gnT=96), -1, "gnT % 64"),
    (dict(src=0, hi=FAKE, lo=FAKE, ld8=64), dict(epi=2), -1, "Lphi"),
    (dict(src=0, hi=FAKE, lo=FAKE, ld8=64), dict(epi=1, Cs=30), -1, "SPLIT3"),
    (dict(src=0, hi=FAKE, lo=FAKE, ld8=64), dict(Y=None), -1, "null Y"),
])
def test_hl2_argument_errors(asrc, aepi, code, msg):
    A = _lib.ASrc(**asrc)
    E = _lib.AEpi(**{"Y": FAKE, "ldy": 64, **aepi})
    Kp = 80 if asrc.get("K") == 72 else 64
    rc, err = call_hl2(A, E, Kp=Kp, ldw=Kp)
    assert rc == code and msg in err, err


QKV = dict(epi=4, heads=1, C=64, T=40, TpQ=128, TpK=64, Y2=FAKE, qhi=FAKE, qlo=FAKE, khi=FAKE, klo=FAKE, qe=FAKE, ke=FAKE,
           qhs=FAKE, qls=FAKE, qts=FAKE, khs=FAKE, kls=FAKE, kts=FAKE)


@pytest.mark.parametrize("aepi,msg", [
    (dict(QKV, TpK=32), "TpK >= T"),
    (dict(QKV, T=0), "T > 0"),
    (dict(QKV, kts=None), "every q/k output"),
    (dict(QKV, Y2=FAKE + 4), "16-byte aligned Y2"),
    (dict(QKV, qlo=FAKE + 2), "4-byte aligned"),
])
def test_hl2_qkv_errors(aepi, msg):
    """EPI_QKV (src/gemm_hl.cu:179-241) needs N = 3C with C = 64 heads and every q/k output."""
    A = _lib.ASrc(src=0, hi=FAKE, lo=FAKE, ld8=64)
    E = _lib.AEpi(**{"Y": None, "ldy": 0, **aepi})
    rc, err = call_hl2(A, E, Np=192, Nreal=192)
    assert rc == -1 and msg in err, err


def test_epilogue_and_gn_init_errors():
    """k_epilogue with statistics needs 32 whole groups and whole 1024-element blocks per sample."""
    lib = _lib.load()
    base = [None, FAKE, FAKE, 64, 128, 128, FAKE, FAKE, FAKE, 128, None]
    assert lib.vgemm_epilogue(*base, FAKE, 0) == -1
    assert "GN stats: shape" in lib.vgemm_last_error().decode()
    # ldy != N with statistics: the reference throws "epilogue GN stats: shape" (src/kernels.cu:734)
    assert lib.vgemm_epilogue(*base[:9], 132, None, FAKE, 64) == -1
    assert "GN stats: shape" in lib.vgemm_last_error().decode()
    assert lib.vgemm_epilogue(*base[:4], 96, 96, *base[6:9], 96, None, FAKE, 48) == -1   # 96 * 48 % 1024 != 0
    assert lib.vgemm_epilogue(*base[:4], 100, 100, *base[6:9], 100, None, FAKE, 64) == -1  # N % 4
    assert lib.vgemm_gn_init(None, None, 4) == -1
    assert lib.vgemm_gn_init(None, FAKE, 0) == -1


def test_empty_problem_is_a_no_op():
    """Mreal = 0 or Nreal = 0 returns before any launch (no device needed)."""
    A = _lib.ASrc(src=0, hi=FAKE, lo=FAKE, ld8=64)
    E = _lib.AEpi(Y=FAKE, ldy=64)
    assert call_hl2(A, E, Mreal=0)[0] == 0
    assert call_hl2(A, E, Nreal=0)[0] == 0


def test_i8gemm_errors():
    lib = _lib.load()
    h = ctypes.c_void_p()
    assert lib.vgemm_i8_create(0, ctypes.byref(h)) == 0
    try:
        rc = lib.vgemm_i8_run(h, None, FAKE, 64, 0, FAKE, 64, 0, FAKE, 64, 0, 0, 64, 64, 1)
        assert rc == -1 and "no int8 GEMM" in lib.vgemm_last_error().decode()
        rc = lib.vgemm_i8_run(h, None, FAKE, 64, 0, FAKE, 64, 0, FAKE, 64, 0, 64, 64, 40, 1)
        assert rc == -1 and "K % 16" in lib.vgemm_last_error().decode()
    finally:
        lib.vgemm_i8_destroy(h)


def test_workspace_heuristic():
    """Split-K only for deep K whose tiles leave CUs idle (C4 conv at M = 512), none for C2."""
    lib = _lib.load()
    lib.vgemm_set_variant(-1)
    lib.vgemm_set_splitk(0)
    assert lib.vgemm_workspace_bytes(32768, 32768, 2560, 2560, 320, 2) == 0
    assert lib.vgemm_workspace_bytes(512, 512, 1280, 1280, 11520, 0) > 0
    lib.vgemm_set_variant(1)
    assert lib.vgemm_get_variant() == 1
    lib.vgemm_set_variant(-1)


@pytest.mark.parametrize("geom,epi,rows", [
    ((16, 16, 1280, 1), 0, 128),   # eight output rows per tile
    ((16, 16, 1280, 1), 1, 128),   # SPLIT3
    ((16, 16, 1280, 1), 4, 0),     # QKV runs on the 128 x 128 tile kernels
    ((16, 8, 64, 1), 0, 128),      # sixteen rows of 8 pixels
    ((32, 4, 64, 1), 0, 128),      # 32 rows of 4 pixels: a 34 x 6 patch
    ((64, 2, 64, 1), 0, 0),        # 64 rows of 2 pixels: a 66 x 4 patch does not fit
    ((32, 32, 640, 1), 0, 0),      # four rows per tile: the tile kernels measured faster
    ((64, 64, 320, 1), 0, 0),
    ((8, 8, 1280, 1), 0, 0),       # a tile would span two images
    ((12, 16, 64, 1), 0, 0),       # 12 rows are not a multiple of 8
    ((16, 16, 1280, 1), 2, 0),     # GEGLU keeps its table on the tile kernels
    ((16, 16, 1280, 1), 3, 0),     # GELU likewise
    ((16, 16, 1280, 2), 0, 0),     # stride 2
    ((16, 16, 32, 1), 0, 0),       # C % 64 != 0
])
def test_conv16_halo_rows(geom, epi, rows):
    """Selection of the halo-reuse 3x3 kernel: stride 1, C % 64, at least eight whole output rows per
    128-row tile, a patch of at most 208 pixels, no GELU table."""
    H, W, C, stride = geom
    assert _lib.load().vgemm_conv16_halo_rows(H, W, C, stride, epi) == rows


def test_version():
    assert b"gfx950" in _lib.load().vgemm_version()


def test_elementwise_errors():
    """The elementwise entry points' checks (src/kernels.cu:763-771): empty work is a no-op, null
    pointers and negative sizes fail, and concat with GroupNorm records needs Co % 32 == 0 and
    (T Co) % 256 == 0 (the reference's "concat GN stats: shape")."""
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    assert lib.vgemm_act(None, None, 0, None) == 0
    assert lib.vgemm_add(None, None, None, 0) == 0
    assert lib.vgemm_act(None, None, 5, fake) != 0
    assert lib.vgemm_geglu(None, fake, None, 5, fake) != 0
    assert lib.vgemm_add(None, fake, None, 5) != 0
    rc = lib.vgemm_concat(None, fake, 40, fake, 8, 4, fake, fake, 8)
    assert rc != 0 and b"concat GN stats: shape" in lib.vgemm_last_error()
    rc = lib.vgemm_concat(None, fake, 32, fake, 32, 4, fake, fake, 2)   # T Co = 128
    assert rc != 0 and b"concat GN stats: shape" in lib.vgemm_last_error()
    assert lib.vgemm_concat(None, fake, -1, fake, 8, 4, fake, None, 0) != 0
    assert lib.vgemm_concat(None, fake, 8, fake, 8, 0, fake, None, 0) == 0
    assert lib.vgemm_upsample2(None, fake, 1, 2, 2, -4, fake) != 0
    assert lib.vgemm_upsample2(None, None, 0, 2, 2, 4, None) == 0


def test_engine_argument_errors():
    """The engine entry points' checks before any device work: a model and an arena size are needed,
    a null engine or malformed activation fails, and destroy / arena_peak take a null engine."""
    lib = _lib.load()
    h = ctypes.c_void_p()
    assert lib.vgemm_engine_create(None, 1 << 20, 0, ctypes.byref(h)) == -1 and not h.value
    assert b"a model and an arena size" in lib.vgemm_last_error()
    assert lib.vgemm_engine_create(None, 1 << 20, 0, None) == -1
    lib.vgemm_engine_destroy(None)
    assert lib.vgemm_engine_arena_peak(None) == 0
    x = _lib.Activation(d=0x1000, B=2, T=64, C=64)
    out = _lib.Activation(d=0x2000, B=2, T=64, C=128)
    assert lib.vgemm_engine_resnet(None, None, ctypes.byref(x), 8, 8, b"p", ctypes.byref(out)) == -1
    assert b"null engine" in lib.vgemm_last_error()
    assert lib.vgemm_engine_resnet(None, None, ctypes.byref(x), 8, 7, b"p", ctypes.byref(out)) == -1   # T != H W
    assert b"resnet: bad arguments" in lib.vgemm_last_error()
    bad = _lib.Activation(d=0, B=2, T=64, C=64)
    assert lib.vgemm_engine_transformer(None, None, ctypes.byref(bad), b"p", 2, ctypes.byref(out)) == -1
    assert lib.vgemm_engine_set_context(None, None, ctypes.byref(x), b"b", 0) == -1


def test_norm_argument_errors():
    """The integer norms' checks: groups divide C and are at most 64 (32 for the row kernel, whose
    reference caches 32 records per row), C % 4 and C <= 2560, 16-byte aligned rows, the int16 view's
    planes with Kp >= C and Kp % 4 == 0."""
    lib = _lib.load()
    ok_args = (None, FAKE, 2, 8, 128)
    assert lib.vgemm_gn_stats1(*ok_args, 96, FAKE) == -1   # 128 % 96
    assert b"groups must divide C" in lib.vgemm_last_error()
    assert lib.vgemm_gn_stats1(None, FAKE, 2, 8, 256, 128, FAKE) == -1   # more than 64 groups
    assert lib.vgemm_gn_stats2(None, FAKE, 2, 8, 128, 32, 0, FAKE) == -1   # den
    assert lib.vgemm_gn_stats1(None, FAKE, 2, 8, 2564, 4, FAKE) == -1   # C > 2560
    assert lib.vgemm_gn_stats1(None, FAKE + 4, 2, 8, 128, 32, FAKE) == -1   # alignment
    rc = lib.vgemm_gn_apply_row(None, FAKE, 2, 8, 128, 64, FAKE, FAKE, FAKE, None, FAKE, None, None, None, None, 0)
    assert rc == -1 and b"at most 32 groups" in lib.vgemm_last_error()
    rc = lib.vgemm_gn_apply_row(None, FAKE, 2, 8, 128, 32, FAKE, FAKE, FAKE, None, None, None, FAKE, FAKE, FAKE, 126)
    assert rc == -1 and b"Kp >= C" in lib.vgemm_last_error()
    rc = lib.vgemm_lnorm_q(None, FAKE, 4, 128, FAKE, FAKE, 100000, FAKE, FAKE, FAKE, 130)
    assert rc == -1 and b"Kp % 4 == 0" in lib.vgemm_last_error()

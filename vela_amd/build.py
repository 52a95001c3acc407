"""Build the in-tree shared libraries.

  vela_amd/libvgemm.so         the HIP kernels and the C ABI (hipcc, gfx950)
  vela_amd/libvela_datagen.so  seeded synthetic inputs (gcc, OpenMP)
  oracle/liboracle.so          the CPU oracle (gcc, OpenMP) -- test infrastructure, built here so the
                               GPU box receives it prebuilt
  tests/cpp/dropin_test        the C++ drop-in check (hipcc; host code against include/vela/*.h)

Run as ``python -m vela_amd.build``. Objects go to vela_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "vela_amd"
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
ORACLE = ROOT / "oracle"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-mcode-object-version=5",
    # no packed-FP32 instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-but-set-variable",
]
# AVX2 baseline so the CPU libraries run on any x86-64-v3 host (this container and the GPU box)
C_FLAGS = ["-O3", "-march=x86-64-v3", "-fPIC", "-fopenmp", "-Wall", "-Wextra", "-Wno-unused-parameter", "-std=gnu11"]

HIP_SOURCES = ["gemm_src_i8.hip", "gemm_src_i16.hip", "gemm_src_x32.hip", "gemm_src_conv32.hip",
               "gemm_src_conv16.hip", "gemm_stripe.hip", "gemm_stripe16.hip", "gemm_kwave.hip", "gemm_raw.hip", "producers.hip", "elementwise.hip", "norms.hip", "attn.hip", "capi.hip", "model.cpp", "engine.cpp"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip() != "1 warning generated.")
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}")
    if out.strip():
        print(out, file=sys.stderr)


def _hip_object(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    _run([HIPCC, *HIP_FLAGS, "-I", str(ROOT / "include"), "-c", str(CSRC / src), "-o", str(obj)])
    return obj


def build_vgemm(jobs: int | None = None) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(len(HIP_SOURCES), max(1, os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_hip_object, HIP_SOURCES))
    out = PKG / "libvgemm.so"
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    return out


def build_c_lib(sources: list[Path], out: Path, extra: list[str] | None = None) -> Path:
    tmp = out.with_suffix(".so.tmp")
    _run(["gcc", *C_FLAGS, "-shared", "-o", str(tmp), *map(str, sources), "-lm", *(extra or [])])
    os.replace(tmp, out)
    return out


def build_dropin_test() -> Path:
    out = ROOT / "tests" / "cpp" / "dropin_test"
    src = ROOT / "tests" / "cpp" / "dropin_test.cpp"
    if not src.exists():
        return out
    tmp = out.with_name(out.name + ".tmp")
    _run([HIPCC, "-O2", "-std=c++17", "-I", str(ROOT / "include"), str(src), "-o", str(tmp),
          "-L", str(PKG), "-lvgemm", f"-Wl,-rpath,{PKG}", "-Wl,-rpath,$ORIGIN/../../vela_amd"])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_c_lib([CSRC / "datagen.c"], PKG / "libvela_datagen.so")
    build_c_lib([ORACLE / "oracle.c"], ORACLE / "liboracle.so")
    build_vgemm()
    build_dropin_test()


if __name__ == "__main__":
    build_all()
    print("built:", PKG / "libvgemm.so", PKG / "libvela_datagen.so", ORACLE / "liboracle.so")

"""The C++ drop-in headers (include/vela/gemm_hl.h, gemm.h, kernels.h) driven from C++ the way the
reference's engine and src/test_gemm_hl.cu drive src/gemm_hl.h: tests/cpp/dropin_test.cpp, built by
`python -m vela_amd.build`, run here as a child process (with the synthetic model file, so that
include/vela/poisd.h and include/vela/model.h are driven too)."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "cpp" / "dropin_test"


def test_cpp_dropin(gpu):
    assert EXE.exists(), f"{EXE} is not built: run `python -m vela_amd.build`"
    model = Path(__file__).resolve().parent / "golden" / "tiny_model.poisd"
    r = subprocess.run([str(EXE), str(model)], capture_output=True, text=True, timeout=180)
    print(r.stdout[-4000:], r.stderr[-2000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "ALL PASS" in r.stdout

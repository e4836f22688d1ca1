"""The C++ host layer (include/mako_h3.hpp) through its parity driver, tests/cpp/h3_kernels_test: built by
__graft_entry__.build(), it runs every op through the layer on the GPU and checks it against the CPU oracle, one
"ok"/"FAIL" line a check, in the manner of the reference's tests/h3_ref_test.cpp."""
import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parent / "cpp" / "h3_kernels_test"


def test_driver_is_built_and_links():
    assert EXE.exists(), "run __graft_entry__.build()"
    out = subprocess.run(["ldd", str(EXE)], capture_output=True, text=True, check=True).stdout
    assert "not found" not in out, out
    assert "libmako_h3.so" in out and "libmh3_oracle.so" in out


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["rows", "swiglu", "cubes", "attn", "int8", "proj", "cond", "errors"])
def test_host_layer_parity(mode):
    r = subprocess.run([str(EXE), mode], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout

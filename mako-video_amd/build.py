"""Builds libmako_h3.so, the gfx950 kernels and their C-ABI (include/mako_h3.h), in-tree with hipcc.

    python mako-video_amd/build.py            # -> mako-video_amd/lib/libmako_h3.so, libmh3_stream_probe.so

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction selection switched off (the compiler's
v_pk_*_f32 forms are not trusted on these boxes), then linked into one shared library that host code binds through
the C header.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "lib" / "libmako_h3.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Wall",
    "-Werror",
    "-Wno-unused-command-line-argument",
    "-Wno-unknown-warning-option",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]
SOURCES = ["rows.hip", "cond.hip", "heads.hip", "cubes.hip", "quant.hip", "gemm.hip", "attn.hip", "abi.cpp"]
# The streaming-bandwidth probe bench.py reports beside the kernels: its own library, not part of the C-ABI.
PROBE_SOURCE = "probe/stream_probe.hip"
PROBE_LIB = PKG / "lib" / "libmh3_stream_probe.so"


def _compile(src: str) -> Path:
    out = OBJ / (Path(src).stem + ".o")
    path = CSRC / src
    lang = ["-x", "hip"] if src.endswith(".hip") else ["-x", "hip"]
    cmd = [HIPCC, *COMMON, *lang, "-c", str(path), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 target feature and says so; that is the only expected noise.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return out


def _link(objs: list[Path], lib: Path, verbose: bool) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib.relative_to(REPO)}")


def build(verbose: bool = True) -> Path:
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found")
    OBJ.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES + [PROBE_SOURCE]))
    _link(objs[:-1], LIB, verbose)
    _link(objs[-1:], PROBE_LIB, verbose)
    return LIB


if __name__ == "__main__":
    build()

"""Build libsys1hip.so in-tree with hipcc for gfx950.

Every source under ``csrc/`` compiles to an object in ``_build/`` (in parallel), and the objects
link into ``sys1rust_amd/libsys1hip.so``. Run as ``python -m sys1rust_amd.build``.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libsys1hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-I", str(ROOT / "include"),
]

SOURCES = ["gemm.hip", "attention.hip", "elementwise.hip", "f32path.hip", "model.cpp", "api.cpp", "safetensors.cpp",
           "synth.cpp", "selfcheck.cpp"]
LIBS = ["-Wl,-rpath,/opt/rocm/lib"]


def _compile(src: str) -> Path:
    out = BUILD / (src.replace(".", "_") + ".o")
    cmd = [HIPCC, "-x", "hip", *COMMON, "-c", str(CSRC / src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip():
        # hipcc's host pass warns about the device-only target feature; keep the rest visible.
        lines = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
        if lines:
            print("\n".join(lines), file=sys.stderr)
    return out


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    jobs = min(len(SOURCES), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-o", str(tmp), *map(str, objs), *LIBS]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)

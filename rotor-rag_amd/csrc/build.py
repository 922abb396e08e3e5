"""Build librotor_hip.so (gfx950) in-tree with hipcc.

    python rotor-rag_amd/csrc/build.py          # or __graft_entry__.build()

Every HIP translation unit is compiled for gfx950 only, with packed-FP32 code
generation disabled (-Xclang -target-feature -Xclang -packed-fp32-ops), kernel-argument
preloading on, no fast-math (the quantiser relies on IEEE fp32 division), then linked into
rotor-rag_amd/rotor/lib/librotor_hip.so, next to the Python package that loads it.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
LIB_DIR = PKG / "rotor" / "lib"
LIB = LIB_DIR / "librotor_hip.so"
OBJ_DIR = PKG / "build" / "obj"
SOURCES = ["rt_layout.hip", "rt_quant.hip", "rt_gemv.hip", "rt_gemm.hip", "rt_model.hip", "rt_api.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Device code generation flags (also used by the code-generation tests):
#   packed-fp32-ops off; kernel arguments preloaded into SGPRs at wave launch (up to 16
#   dwords of leading scalar/pointer arguments; the code object keeps a fallback that
#   loads them where the firmware does not preload).
DEVICE_FLAGS = [
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-command-line-argument",
    *DEVICE_FLAGS,
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so: harmless.
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False) -> Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)

    def compile_one(src):
        obj = OBJ_DIR / (Path(src).stem + ".o")
        out = _run([HIPCC, *CFLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        if verbose and out.strip():
            print(out)
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

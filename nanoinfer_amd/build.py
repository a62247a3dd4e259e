"""Build recipe for the gfx950 library ``nanoinfer_amd/libnanoinfer_kv.so``.

Plain ``hipcc`` (no cmake, no torch extension): the library exposes a C ABI
with no torch types, so it is built as an ordinary shared object and loaded
with ctypes.  Run ``python -m nanoinfer_amd.build``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libnanoinfer_kv.so")
ARCH = "gfx950"

SOURCES = [os.path.join(CSRC, "kv_kernels.hip"), os.path.join(CSRC, "kv_host.cpp")]
HEADERS = [os.path.join(CSRC, "kv_plan.h"), os.path.join(INCLUDE, "nanoinfer_kv.h")]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def command(out: str = LIB) -> list[str]:
    return [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        # Packed-FP32 VALU forms stay off: ordinary f32 code only.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function",
        f"-I{INCLUDE}", f"-I{CSRC}",
        *SOURCES, "-o", out,
    ]


def build(verbose: bool = False) -> str:
    """Compile every source into the library (always recompiles)."""
    tmp = LIB + ".tmp"
    proc = subprocess.run(command(tmp), capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l and l.strip())
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err:
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


def stale() -> bool:
    if not os.path.exists(LIB):
        return True
    t = os.path.getmtime(LIB)
    return any(os.path.getmtime(p) > t for p in SOURCES + HEADERS)


if __name__ == "__main__":
    print(build(verbose=True))

"""Build recipe for the gfx950 library ``nanoinfer_amd/libnanoinfer_kv.so``,
the serving drivers over its C ABI (``libnanoinfer_drivers.so``) and their
command-line front end (``ni_drive``).

Plain ``hipcc`` (no cmake, no torch extension): the libraries expose C ABIs
with no torch types, so they are built as ordinary shared objects and loaded
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

DRIVERS_LIB = os.path.join(HERE, "libnanoinfer_drivers.so")
DRIVE_EXE = os.path.join(HERE, "ni_drive")

SOURCES = [os.path.join(CSRC, "kv_kernels.hip"), os.path.join(CSRC, "kv_host.cpp")]
HEADERS = [os.path.join(CSRC, "kv_plan.h"), os.path.join(INCLUDE, "nanoinfer_kv.h")]
DRIVER_SOURCES = [os.path.join(CSRC, "drivers.cpp")]
DRIVER_HEADERS = [os.path.join(INCLUDE, "nanoinfer_drivers.h")]


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
        # Q8 scales: amax / 127 and its inverse must be IEEE divisions.
        "-fhip-fp32-correctly-rounded-divide-sqrt",
        # Matrix-core accumulators in VGPRs: the online softmax rescales them
        # with VALU multiplies, which in AGPRs cost a read and a write each.
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        "-Wall", "-Wno-unused-function",
        f"-I{INCLUDE}", f"-I{CSRC}",
        *SOURCES, "-o", out,
    ]


def drivers_command(out: str = DRIVERS_LIB) -> list[str]:
    """Host code only, linked against the KV library next to it."""
    return [
        hipcc(), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
        f"-I{INCLUDE}", *DRIVER_SOURCES, f"-L{HERE}", "-lnanoinfer_kv", "-Wl,-rpath,$ORIGIN", "-o", out,
    ]


def drive_exe_command(out: str = DRIVE_EXE) -> list[str]:
    return [
        hipcc(), "-O2", "-std=c++17", "-Wall", f"-I{INCLUDE}", os.path.join(CSRC, "ni_drive.cpp"),
        f"-L{HERE}", "-lnanoinfer_drivers", "-lnanoinfer_kv", "-Wl,-rpath,$ORIGIN", "-o", out,
    ]


def _run(cmd: list[str], out: str, verbose: bool):
    """Build into out.tmp, then move it into place."""
    tmp = out + ".tmp"
    cmd = [tmp if c == out else c for c in cmd]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l and l.strip())
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err:
        print(err, file=sys.stderr)
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    """Compile the KV library, the drivers and ni_drive (always recompiles)."""
    _run(command(LIB), LIB, verbose)
    _run(drivers_command(DRIVERS_LIB), DRIVERS_LIB, verbose)
    _run(drive_exe_command(DRIVE_EXE), DRIVE_EXE, verbose)
    return LIB


def stale() -> bool:
    outs = [LIB, DRIVERS_LIB, DRIVE_EXE]
    if not all(os.path.exists(o) for o in outs):
        return True
    t = min(os.path.getmtime(o) for o in outs)
    return any(os.path.getmtime(p) > t for p in SOURCES + HEADERS + DRIVER_SOURCES + DRIVER_HEADERS)


if __name__ == "__main__":
    print(build(verbose=True))

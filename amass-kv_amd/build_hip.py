"""Build libamass_hip.so (every HIP source under csrc/) for gfx950, in tree.

    python amass-kv_amd/build_hip.py            # -> amass-kv_amd/amass/_lib/libamass_hip.so
                                                #    and libamass_calib.so (calib/)

Each .hip file compiles to an object in amass-kv_amd/_build/ (in parallel), then one
hipcc link produces the shared library.  Packed fp32 VALU ops are disabled for all device
code (-packed-fp32-ops).  The host toolchain is /opt/rocm's hipcc; the resulting library
binds to whichever libamdhip64 the process already has loaded (torch's, when torch is
imported first).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT_DIR = os.path.join(HERE, "amass", "_lib")
LIB = os.path.join(OUT_DIR, "libamass_hip.so")
ARCH = os.environ.get("AMASS_OFFLOAD_ARCH", "gfx950")

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-variable", "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(hipcc: str, src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc, *CFLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    """Compile every csrc/*.hip and link libamass_hip.so; returns the library path."""
    t0 = time.time()
    hipcc = _hipcc()
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s), srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[amass build] {len(srcs)} sources -> {LIB} ({time.time() - t0:.1f}s)")
    return LIB


CALIB_SRC = os.path.join(HERE, "calib", "gather_calib.hip")
CALIB_LIB = os.path.join(OUT_DIR, "libamass_calib.so")


def build_calib(verbose: bool = True) -> str:
    """Build libamass_calib.so: the HBM-counter calibration kernel bench.py profiles
    beside the hot path (measurement only; not part of libamass_hip.so's ABI)."""
    t0 = time.time()
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = CALIB_LIB + ".tmp"
    cmd = [_hipcc(), *CFLAGS, "-shared", CALIB_SRC, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {CALIB_SRC}:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, CALIB_LIB)
    if verbose:
        print(f"[amass build] calibration kernel -> {CALIB_LIB} ({time.time() - t0:.1f}s)")
    return CALIB_LIB


if __name__ == "__main__":
    build()
    build_calib()

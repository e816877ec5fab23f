"""Builds the gfx950 HIP library ``liblcpp_hip.so`` in-tree.

Every ``csrc/*.hip`` file is compiled by ``hipcc --offload-arch=gfx950`` into its own object (in
parallel), host-only ``csrc/*.cpp`` files by ``g++``, and the objects are linked into one shared
library next to this file.  The C-ABI is declared in ``include/lcpp_hip.h``.

``--phase-trace`` builds the diagnostic variant ``liblcpp_hip_trace.so`` instead: the same sources with
``LCPP_HIP_PHASE_TRACE`` defined, whose onesweep and scan kernels write per-tile phase stamps
(``phase_trace.py`` reads them).  The product library never contains that code.

Usage: ``python luisacompute-parallelprimitive_amd/build.py [--jobs N] [--phase-trace]``
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "liblcpp_hip.so"
TRACE_BUILD = PKG / "_build_trace"
TRACE_LIB = PKG / "liblcpp_hip_trace.so"
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3", "-std=c++20", f"--offload-arch={ARCH}", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
    # Keep the compiler from forming packed-FP32 VALU instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
]
HOST_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-fvisibility=hidden", "-Wall", f"-I{REPO / 'include'}"]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build liblcpp_hip.so")
    return path


def _compile(src: pathlib.Path, out_dir: pathlib.Path, defines: list[str]) -> pathlib.Path:
    obj = out_dir / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [_hipcc(), "-x", "hip", *HIP_FLAGS, *defines, "-c", str(src), "-o", str(obj)]
    else:
        cmd = ["g++", *HOST_FLAGS, *defines, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False, phase_trace: bool = False) -> pathlib.Path:
    out_dir, lib = (TRACE_BUILD, TRACE_LIB) if phase_trace else (BUILD, LIB)
    defines = ["-DLCPP_HIP_PHASE_TRACE"] if phase_trace else []
    out_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, out_dir, defines), sources))
    tmp = lib.with_suffix(".so.tmp")
    # Only the C-ABI (lcpp_hip_*) is exported: kernel stubs and C++ internals stay local, so two builds
    # loaded into one process never resolve each other's internals.
    exports = out_dir / "exports.map"
    exports.write_text("{\n  global: lcpp_hip_*;\n  local: *;\n};\n")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,--version-script={exports}", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--phase-trace", action="store_true", help="build the diagnostic liblcpp_hip_trace.so")
    args = ap.parse_args()
    build(args.jobs, verbose=True, phase_trace=args.phase_trace)
    sys.exit(0)

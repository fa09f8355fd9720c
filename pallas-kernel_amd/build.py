"""Build libtops_hip.so (gfx950) from csrc/ with hipcc, in-tree.

    python pallas-kernel_amd/build.py [-j N] [--phase-clocks]

Objects go to pallas-kernel_amd/_build/, the library to
pallas-kernel_amd/tops/_lib/libtops_hip.so (both git-ignored).  --phase-clocks also builds
tops/_lib/libtops_pipe_clocks.so: the pipelined sweep alone, compiled with
TOPS_PHASE_CLOCKS (per-wave phase clocks, read by pallas-kernel_amd/phase_clocks.py).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "tops", "_lib")
LIB = os.path.join(LIBDIR, "libtops_hip.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = ["-O3", "-std=c++17", "-fPIC", f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}"]
# Packed-FP32 VALU ops are disabled for all device code.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def sources():
    out = []
    for f in sorted(os.listdir(CSRC)):
        if f.endswith((".hip", ".cpp")):
            out.append(os.path.join(CSRC, f))
    return out


def compile_one(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC] + COMMON + DEVICE + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, len(srcs), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    shutil.move(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


CLOCKS_LIB = os.path.join(LIBDIR, "libtops_pipe_clocks.so")


def build_phase_clocks(verbose: bool = True) -> str:
    """The instrumented pipelined sweep (TOPS_PHASE_CLOCKS) as its own library."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    src = os.path.join(CSRC, "gla_sweep_pipe.hip")
    obj = os.path.join(BUILD, "gla_sweep_pipe.clocks.o")
    r = subprocess.run([HIPCC] + COMMON + DEVICE + ["-DTOPS_PHASE_CLOCKS", "-c", src, "-o", obj],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src} (TOPS_PHASE_CLOCKS):\n{r.stderr}")
    tmp = CLOCKS_LIB + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, obj],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    shutil.move(tmp, CLOCKS_LIB)
    if verbose:
        print(f"built {CLOCKS_LIB}")
    return CLOCKS_LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("--phase-clocks", action="store_true",
                    help="also build the instrumented sweep library (libtops_pipe_clocks.so)")
    a = ap.parse_args()
    try:
        build(a.j)
        if a.phase_clocks:
            build_phase_clocks()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)

"""Build ``libpack3d_hip.so`` for gfx950 from ``pack3d_amd/csrc`` with hipcc.

Usage: ``python -m pack3d_amd.build`` (or ``__graft_entry__.build()``).
Objects go to ``pack3d_amd/_build``; the shared library lands next to this
file so that it travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
PROBE_SRC = os.path.join(HERE, "probe")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libpack3d_hip.so")
PROBE_LIB = os.path.join(HERE, "libpack3d_probe.so")
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled for device code: the compiler forms them
# from ordinary float code, and this pool has seen wrong results from some
# forms.  The kernels never produce or consume NaN (masked scores are -inf),
# so fmax needs no NaN-quieting of its operands (-fno-honor-nans).  The
# kernels keep the default IEEE mode: a kernel compiled with
# -mno-amdgpu-ieee cannot inline the device library (threadIdx, blockIdx and
# __mul24 become out-of-line calls), which costs far more than it saves.
FLAGS = ["-x", "hip", "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-fno-honor-nans", "-Wno-nan-infinity-disabled"]


def _hipcc():
    """The ROCm clang driver."""
    for path in ("/opt/rocm/lib/llvm/bin/clang++", shutil.which("amdclang++")):
        if path and os.path.exists(path):
            return path
    raise RuntimeError("ROCm clang++ not found; the pack3d_amd HIP library cannot be built")


def _compile(src, hipcc, verbose):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc, *FLAGS, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msgs}")
    if verbose and msgs.strip():
        print(msgs, flush=True)
    return obj


def _link(hipcc, objs, out, verbose):
    tmp = out + ".tmp"
    cmd = [hipcc, "--hip-link", f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
           "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}", flush=True)


def build(verbose: bool = False) -> str:
    """Compile every HIP source and link the shared libraries: the product
    library from csrc/, and the measurement library (the issue-rate probe of
    probe/, with the status functions it reports through); returns the
    product library's path."""
    hipcc = _hipcc()
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    probes = sorted(os.path.join(PROBE_SRC, f) for f in os.listdir(PROBE_SRC) if f.endswith(".hip"))
    workers = min(len(sources) + len(probes), int(os.environ.get("MAX_JOBS", "8")), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda s: _compile(s, hipcc, verbose), sources + probes))
    _link(hipcc, objs[:len(sources)], LIB, verbose)
    status = os.path.join(BUILD, "status.hip.o")
    _link(hipcc, objs[len(sources):] + [status], PROBE_LIB, verbose)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)

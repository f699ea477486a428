"""Build libmtpx.so for gfx950 with hipcc (in-tree, no JIT cache).

    python imr-mlp_amd/build.py [-v] [--changed]

Each translation unit gets its own floating-point contraction policy: the
neighbour builder and the host geometry are compiled with
-ffp-contract=off (their results are compared bit for bit with the
reference), the E/F/S and training kernels with -ffp-contract=fast (FMA).
"""
from __future__ import annotations

import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libmtpx.so")
CALC_EFS = os.path.join(LIB_DIR, "mtpx_calc_efs")
CXX = os.environ.get("CXX", "g++")
OBJ_DIR = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=" + ARCH, "-munsafe-fp-atomics",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-Wall", "-Wno-unused-function"]

SOURCES = [
    ("efs_kernel.hip", ["-ffp-contract=fast"]),
    ("train_kernel.hip", ["-ffp-contract=fast"]),
    ("lin_kernel.hip", ["-ffp-contract=fast"]),
    ("lin_kernel.hip", ["-ffp-contract=fast", "-DMTPX_LIN_PART=2"], "lin_kernel_part2"),
    ("gram_kernel.hip", ["-ffp-contract=fast"]),
    ("neighbors.hip", ["-ffp-contract=off"]),
    ("geometry.cpp", ["-ffp-contract=off"]),
    ("model.cpp", ["-ffp-contract=off"]),
    ("capi.cpp", ["-ffp-contract=off"]),
    ("model_view.cpp", ["-ffp-contract=off"]),
    ("train_api.cpp", ["-ffp-contract=off"]),
    ("linear_api.cpp", ["-ffp-contract=off"]),
    ("sites.cpp", ["-ffp-contract=off"]),
    ("metadata.cpp", ["-ffp-contract=off"]),
    ("lbfgs.cpp", ["-ffp-contract=off"]),
    ("gpm.cpp", ["-ffp-contract=off"]),
]


def sources():
    """(source, flags, object name) of every translation unit; a source may
    be compiled more than once under different names."""
    out = []
    for e in SOURCES:
        src, flags = e[0], e[1]
        name = e[2] if len(e) > 2 else src
        if os.path.exists(os.path.join(CSRC, src)):
            out.append((src, flags, name))
    return out


def _newest_header() -> float:
    hs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hpp")]
    hs.append(os.path.join(ROOT, "include", "mtpx.h"))
    return max(os.path.getmtime(h) for h in hs)


def build(verbose: bool = False, changed_only: bool = False) -> str:
    """Compile every translation unit (changed_only: those older than their
    source or a header) and link the library."""
    os.makedirs(LIB_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    objs, cmds = [], []
    t0 = time.time()
    newest_h = _newest_header()
    for src, flags, name in sources():
        obj = os.path.join(OBJ_DIR, name + ".o")
        objs.append(obj)
        if changed_only and os.path.exists(obj):
            t_obj = os.path.getmtime(obj)
            if t_obj > os.path.getmtime(os.path.join(CSRC, src)) and t_obj > newest_h:
                continue
        cmds.append([HIPCC, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj] + COMMON + flags)
    # translation units compile in parallel (the kernel files dominate)
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd))
    failed = [c for c, p in zip(cmds, procs) if p.wait() != 0]
    if failed:
        raise subprocess.CalledProcessError(1, failed[0])
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    # the calc_efs front end over the C ABI (host code, links the library)
    tmp = CALC_EFS + ".tmp"
    cmd = [CXX, "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"),
           os.path.join(HERE, "calc_efs.cpp"), "-o", tmp, "-L", LIB_DIR, "-lmtpx",
           "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, CALC_EFS)
    if verbose:
        print("built %s in %.1fs" % (LIB, time.time() - t0), flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv, changed_only="--changed" in sys.argv)

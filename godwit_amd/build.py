"""Builds libgodwit_hip.so for gfx950 in-tree (godwit_amd/libgodwit_hip.so).

    python godwit_amd/build.py

Run it by path: importing the godwit_amd package loads the library this
script builds, so the script must not depend on the package.

Compiles every HIP source under godwit_amd/csrc with hipcc for gfx950 only.
Packed-FP32 instructions are disabled (-packed-fp32-ops): some of their
forms have returned wrong results on the target pool.
"""
from __future__ import annotations

import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libgodwit_hip.so")
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["gw_kernels.hip", "gw_decode.hip", "gw_prefill.hip", "gw_model.hip", "gw_api.hip"]
# Host-only C++ (no HIP), compiled by the host compiler.
HOST_SOURCES = ["gw_host.cpp"]
CXX = os.environ.get("CXX", "g++")
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-fvisibility=hidden"]
OBJDIR = os.path.join(HERE, "_build")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",
]


def build(verbose: bool = True) -> str:
    """Compiles the sources in parallel (hipcc per HIP file, the host compiler for
    the host-only C++), then links."""
    os.makedirs(OBJDIR, exist_ok=True)
    inc = ["-I", os.path.join(HERE, "..", "include")]
    t0 = time.time()
    procs = []
    for src in SOURCES + HOST_SOURCES:
        obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
        if src.endswith(".hip"):
            cmd = [HIPCC, *[f for f in FLAGS if f != "-shared"], *inc, "-c", "-o", obj,
                   os.path.join(CSRC, src)]
        else:
            cmd = [CXX, *HOST_FLAGS, *inc, "-c", "-o", obj, os.path.join(CSRC, src)]
        procs.append((src, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                 stderr=subprocess.STDOUT, text=True)))
    objs, failed, noise = [], False, []
    for src, obj, proc in procs:
        out, _ = proc.communicate()
        noise += [ln for ln in out.splitlines() if ln.strip() and "packed-fp32-ops" not in ln]
        if proc.returncode != 0:
            failed = True
            sys.stderr.write(f"{src}:\n{out}")
        objs.append(obj)
    if failed:
        raise RuntimeError("hipcc failed")
    tmp = LIB + ".tmp"
    link = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs],
                          capture_output=True, text=True)
    if link.returncode != 0:
        sys.stderr.write(link.stdout + link.stderr)
        raise RuntimeError(f"link failed ({link.returncode})")
    if noise and verbose:
        sys.stderr.write("\n".join(noise) + "\n")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} in {time.time() - t0:.1f}s")
    return LIB


if __name__ == "__main__":
    build()

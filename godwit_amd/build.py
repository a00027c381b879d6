"""Builds libgodwit_hip.so for gfx950 in-tree (godwit_amd/libgodwit_hip.so).

    python godwit_amd/build.py

Run it by path: importing the godwit_amd package loads the library this
script builds, so the script must not depend on the package.

Compiles every HIP source under godwit_amd/csrc with hipcc for gfx950 only.
Packed-FP32 instructions are disabled (-packed-fp32-ops): some of their
forms have returned wrong results on the target pool.

The grouped-GEMM and decode kernels order their loads with counted
s_waitcnt vmcnt(N) waits that assume every vector-memory operation in
flight is one the kernel issued itself; a register spill adds scratch
stores and loads to that count.  The build reads the compiler's per-kernel
resource report for those sources and fails if any kernel there spills a
vector register.
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libgodwit_hip.so")
# The same library with the one-token layer's phase stamps compiled in
# (-DGW_DECODE_TRACE; loaded when GODWIT_TRACE_LIB=1, see decode_timeline.py).
TRACE_LIB = os.path.join(HERE, "libgodwit_hip_trace.so")
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["gw_kernels.hip", "gw_decode.hip", "gw_prefill.hip", "gw_model.hip", "gw_api.hip"]
# Host-only C++ (no HIP), compiled by the host compiler.
HOST_SOURCES = ["gw_host.cpp"]
# Sources whose kernels must not spill vector registers (counted waits).
NO_SPILL = {"gw_decode.hip", "gw_prefill.hip"}
_REMARK = re.compile(r"remark: +(Function Name|VGPRs Spill|AGPRs Spill|ScratchSize \[bytes/lane\]): (\S+)")
# Stack bytes a NO_SPILL kernel may keep: a few bytes of an unused private
# segment appear in some kernels; an array placed on the stack or a call to an
# outlined function (whose frame holds its arguments) takes far more, and its
# scratch loads and stores would sit among the counted waits.
SCRATCH_LIMIT = 32


def _without_remarks(out: str) -> str:
    """Compiler output minus the resource-usage remarks and the source excerpt
    and caret lines printed under each."""
    keep, skipping = [], False
    for ln in out.splitlines():
        if "kernel-resource-usage" in ln:
            skipping = True
            continue
        if skipping and re.match(r"^\s*(\d+\s*)?\|", ln):
            continue
        skipping = False
        keep.append(ln)
    return "\n".join(keep)


def spilled_kernels(report: str) -> list[str]:
    """Kernels with a vector-register spill, or a stack frame above
    SCRATCH_LIMIT bytes a lane, in a -Rpass-analysis=kernel-resource-usage
    report (remarks in order: the kernel name, then its figures)."""
    bad, name = [], None
    for m in _REMARK.finditer(report):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            name = val
        elif key.startswith("ScratchSize"):
            if int(val) > SCRATCH_LIMIT and name:
                bad.append(f"{name} (stack {val} bytes a lane)")
        elif int(val) > 0 and name:
            bad.append(f"{name} ({key} {val})")
    return bad


def spill_check(report: str) -> list[str]:
    """The problems the report of a NO_SPILL source shows: its kernels with a
    vector-register spill, or, when it holds no kernel record at all (the
    compiler printed no report, so nothing was checked), that absence."""
    if not any(m.group(1) == "Function Name" for m in _REMARK.finditer(report)):
        return ["no kernel-resource-usage records in the compiler output: nothing was checked"]
    return spilled_kernels(report)


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


def build(verbose: bool = True, trace: bool = False) -> str:
    """Compiles the sources in parallel (hipcc per HIP file, the host compiler for
    the host-only C++), then links.  trace=True builds libgodwit_hip_trace.so
    (phase stamps in the one-token layer kernel) instead."""
    objdir = OBJDIR + ("_trace" if trace else "")
    lib_out = TRACE_LIB if trace else LIB
    extra = ["-DGW_DECODE_TRACE"] if trace else []
    os.makedirs(objdir, exist_ok=True)
    inc = ["-I", os.path.join(HERE, "..", "include")]
    t0 = time.time()
    procs = []
    for src in SOURCES + HOST_SOURCES:
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        if src.endswith(".hip"):
            cmd = [HIPCC, *[f for f in FLAGS if f != "-shared"], *extra, *inc, "-c", "-o", obj,
                   os.path.join(CSRC, src)]
            if src in NO_SPILL:
                cmd.append("-Rpass-analysis=kernel-resource-usage")
        else:
            cmd = [CXX, *HOST_FLAGS, *inc, "-c", "-o", obj, os.path.join(CSRC, src)]
        procs.append((src, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                 stderr=subprocess.STDOUT, text=True)))
    objs, failed, noise = [], False, []
    for src, obj, proc in procs:
        out, _ = proc.communicate()
        noise += [ln for ln in _without_remarks(out).splitlines()
                  if ln.strip() and "packed-fp32-ops" not in ln]
        if proc.returncode != 0:
            failed = True
            sys.stderr.write(f"{src}:\n{out}")
        elif src in NO_SPILL:
            problems = spill_check(out)
            if problems:
                failed = True
                sys.stderr.write(f"{src}: spill check failed:\n  " + "\n  ".join(problems) + "\n")
        objs.append(obj)
    if failed:
        raise RuntimeError("hipcc failed")
    tmp = lib_out + ".tmp"
    link = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs],
                          capture_output=True, text=True)
    if link.returncode != 0:
        sys.stderr.write(link.stdout + link.stderr)
        raise RuntimeError(f"link failed ({link.returncode})")
    if noise and verbose:
        sys.stderr.write("\n".join(noise) + "\n")
    os.replace(tmp, lib_out)
    if verbose:
        print(f"built {lib_out} in {time.time() - t0:.1f}s")
    return lib_out


if __name__ == "__main__":
    build(trace="--trace" in sys.argv[1:])

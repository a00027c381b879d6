"""The library's host-only C++ (godwit_amd/csrc/gw_host.cpp: the .gwt manifest
reader and the decode plan builder) built with g++ under the address and
undefined-behaviour sanitizers, driven by tests/host_fuzz.cpp: every
truncation of a valid manifest, 20,000 seeded byte-level mutations, nesting
and string extremes, out-of-range counts, strides, lengths and non-finite
floats, then 20,000 random assignment sequences through plan_add and
plan_regroup with the plan invariants checked.  CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "godwit_amd", "csrc")


def test_host_code_under_asan_ubsan(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path / "host_fuzz")
    cmd = [cxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           os.path.join(CSRC, "gw_host.cpp"), os.path.join(ROOT, "tests", "host_fuzz.cpp"),
           "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    run = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "host fuzz: ok" in run.stdout

"""The grouped GEMM's pipeline waits for a chunk's staged activations with a
counted `s_waitcnt vmcnt(N)`, N being the loads issued after that chunk's
LDS-DMA.  That count is only right if every chunk's DMAs are issued before
its weight loads; a scheduler that hoisted weight loads above the DMAs made
the wait return early (stale LDS read as activations).  This test compiles
gw_prefill.hip for gfx950 to assembly (the library's own flags) and checks,
for every instantiation of prefill_gemm_kernel, that the vector-memory loads
of each issue group come as DMAs first, then the four 16-byte weight loads.
CPU only: it needs hipcc, not a GPU."""
import os
import re
import subprocess

import pytest

from godwit_amd import build as gwbuild

SRC = os.path.join(gwbuild.CSRC, "gw_prefill.hip")


@pytest.fixture(scope="module")
def assembly(tmp_path_factory):
    if not os.path.exists(gwbuild.HIPCC):
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("asm") / "gw_prefill.s")
    flags = [f for f in gwbuild.FLAGS if f not in ("-shared", "-fvisibility=hidden")]
    cmd = [gwbuild.HIPCC, *flags, "-I", os.path.join(gwbuild.HERE, "..", "include"),
           "--cuda-device-only", "-S", SRC, "-o", out]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    with open(out) as f:
        return f.read()


def _issue_sequence(asm, name):
    body = asm[asm.index(name + ":"):]
    body = body[:body.index(".Lfunc_end")]
    seq = []
    for line in body.split("\n"):
        op = line.strip()
        if op.startswith("buffer_load") and " lds" in op:
            seq.append("X")                       # activation / scale / bias LDS-DMA
        elif op.startswith("global_load_dwordx4"):
            seq.append("W")                       # weight ring
    return "".join(seq)


def check_issue_order(asm, name):
    """First group: the scale and bias copies, then chunk 0's 2*planes DMAs,
    then its 4 weight loads; every later group: >= 2*planes DMAs, 4 loads."""
    planes = int(re.match(r"_ZN2gw19prefill_gemm_kernelILi(\d)E", name).group(1))
    seq = _issue_sequence(asm, name)
    groups = re.findall(r"X+W+", seq)
    assert groups and "".join(groups) == seq.rstrip("X"), (name, seq[:80])
    assert groups[0].count("X") >= 2 + 2 * planes, (name, seq[:40])
    for g in groups:
        assert g.count("W") == 4 and g.count("X") >= 2 * planes, (name, g)


def test_every_gemm_issues_dma_before_weights(assembly):
    names = re.findall(r"^(_ZN2gw19prefill_gemm_kernel\w+):", assembly, re.M)
    assert len(names) >= 11, names            # 8x4 / 12x4 / 8x2 shapes, planes, combine flag
    for name in names:
        check_issue_order(assembly, name)

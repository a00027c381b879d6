"""build() reads the compiler's per-kernel resource report for the sources whose
kernels order their loads with counted vmcnt waits (a register spill adds
scratch loads and stores to that count) and fails when one of them spills a
vector register.  These checks run the report parser and the remark filter on
text in the compiler's format.  CPU only."""
from godwit_amd import build as gwbuild

REPORT = """\
gw_prefill.hip:318:1: remark: Function Name: _ZN2gw19prefill_gemm_kernelILi1ELb1ELi8ELi2ELb0EEEvNS_8GemmArgsE [-Rpass-analysis=kernel-resource-usage]
  318 | {
      | ^
gw_prefill.hip:318:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:318:1: remark:     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:318:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:318:1: remark:     SGPRs Spill: 6 [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:318:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:318:1: remark: Function Name: _ZN2gw19prefill_gemm_kernelILi1ELb0ELi8ELi2ELb0EEEvNS_8GemmArgsE [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:318:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:318:1: remark:     SGPRs Spill: 22 [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:318:1: remark:     VGPRs Spill: 56 [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:318:1: remark: Function Name: _ZN2gw20prefill_route_kernelEPKfiiiPiPf [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:318:1: remark:     AGPRs Spill: 3 [-Rpass-analysis=kernel-resource-usage]
gw_prefill.hip:40:9: warning: unused variable 'x' [-Wunused-variable]
   40 |     int x;
      |         ^
"""


def test_spilled_kernels_names_vector_spills_only():
    bad = gwbuild.spilled_kernels(REPORT)
    # The first kernel spills only scalar registers (to vector lanes, no
    # memory): not flagged.  The second spills 56 VGPRs, the third 3 AGPRs.
    assert bad == ["_ZN2gw19prefill_gemm_kernelILi1ELb0ELi8ELi2ELb0EEEvNS_8GemmArgsE (VGPRs Spill 56)",
                   "_ZN2gw20prefill_route_kernelEPKfiiiPiPf (AGPRs Spill 3)"]


def test_spilled_kernels_empty_report():
    assert gwbuild.spilled_kernels("") == []
    assert gwbuild.spilled_kernels(REPORT.replace("VGPRs Spill: 56", "VGPRs Spill: 0")
                                   .replace("AGPRs Spill: 3", "AGPRs Spill: 0")) == []


def test_without_remarks_keeps_other_diagnostics():
    kept = gwbuild._without_remarks(REPORT).splitlines()
    assert not any("kernel-resource-usage" in ln for ln in kept)
    # the remarks' source excerpts go with them; a warning keeps its own
    assert "  318 | {" not in kept
    assert any("unused variable" in ln for ln in kept)
    assert "   40 |     int x;" in kept


def test_no_spill_sources_are_the_counted_wait_kernels():
    assert gwbuild.NO_SPILL == {"gw_decode.hip", "gw_prefill.hip"}
    assert gwbuild.NO_SPILL <= set(gwbuild.SOURCES)


def test_spill_check_fails_without_kernel_records():
    """A NO_SPILL source whose compiler output holds no kernel record (the
    report flag dropped, or every kernel compiled away) fails the build: an
    empty report must not pass as "no spills"."""
    clean = REPORT.replace("VGPRs Spill: 56", "VGPRs Spill: 0").replace("AGPRs Spill: 3",
                                                                      "AGPRs Spill: 0")
    assert gwbuild.spill_check(clean) == []
    assert len(gwbuild.spill_check(REPORT)) == 2
    for text in ("", "gw_prefill.hip:40:9: warning: unused variable 'x' [-Wunused-variable]\n"):
        problems = gwbuild.spill_check(text)
        assert len(problems) == 1 and "no kernel-resource-usage records" in problems[0]


def test_spilled_kernels_flags_stack_frames():
    """A kernel whose stack frame is larger than a few bytes (an array the
    compiler could not keep in registers, or a call to an outlined function)
    is flagged like a spill; a small unused private segment is not."""
    report = REPORT.replace("VGPRs Spill: 56", "VGPRs Spill: 0").replace("AGPRs Spill: 3", "AGPRs Spill: 0")
    big = report.replace("ScratchSize [bytes/lane]: 0", "ScratchSize [bytes/lane]: 1152")
    assert gwbuild.spilled_kernels(big) == [
        "_ZN2gw19prefill_gemm_kernelILi1ELb1ELi8ELi2ELb0EEEvNS_8GemmArgsE (stack 1152 bytes a lane)"]
    small = report.replace("ScratchSize [bytes/lane]: 0", "ScratchSize [bytes/lane]: 20")
    assert gwbuild.spilled_kernels(small) == []


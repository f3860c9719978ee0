"""The library build's scratch guard for the kernels that copy global memory straight into LDS
(their inline-assembly copies are waited for by hand and are only run without spills)."""

import pytest

from mdlarc_scale_amd import build


REPORT = """\
x.hip:69:1: remark: Function Name: _ZN3mdl19attn_prefill_kernelEv [-Rpass-analysis=kernel-resource-usage]
x.hip:69:1: remark:     VGPRs: 126 [-Rpass-analysis=kernel-resource-usage]
x.hip:69:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:331:1: remark: Function Name: _ZN3mdl16attn_lead_kernelEv [-Rpass-analysis=kernel-resource-usage]
x.hip:331:1: remark:     ScratchSize [bytes/lane]: {n} [-Rpass-analysis=kernel-resource-usage]
"""


def test_no_scratch_passes():
    build.check_no_scratch(REPORT.format(n=0), "x.hip")


def test_scratch_names_the_kernel():
    with pytest.raises(RuntimeError, match="attn_lead_kernel.*64 bytes"):
        build.check_no_scratch(REPORT.format(n=64), "x.hip")


def test_dma_sources_are_guarded():
    """Both LDS-ring kernel files include the copy header, so the build checks them."""
    guarded = {s for s in build.SOURCES if build._uses_dma(build.CSRC / s)}
    assert {"attn_prefill.hip", "prefill_gemm.hip"} <= guarded


ASM = """\
_ZN3mdl19attn_prefill_kernelEv:
\ts_load_dwordx4 s[0:3], s[4:5], 0x0
\t;;#ASMSTART
\ts_mov_b32 m0, s26
\ts_nop 0
\tglobal_load_lds_dwordx4 v[2:3], off
\t;;#ASMEND
\tv_mov_b32_e32 v1, 0 ; m0 in a comment is fine
{extra}
\ts_endpgm
"""


def test_m0_only_in_the_copies_passes():
    build.check_m0(ASM.format(extra=""), "x.hip")


@pytest.mark.parametrize("line", ["\ts_mov_b32 m0, -1", "\tv_movrels_b32_e32 v1, v2  ; uses m0",
                                  "\ts_sendmsg sendmsg(MSG_INTERRUPT)\n\ts_mov_b32 m0, s3",
                                  "\tds_read_addtid_b32 v0 offset:0 ; m0\n\tv_readlane_b32 s0, v1, m0"])
def test_compiler_m0_use_fails(line):
    """A compiler-generated instruction that names M0 outside the copies' asm blocks fails the
    build (the copies would overwrite what it keeps there)."""
    with pytest.raises(RuntimeError, match="M0"):
        build.check_m0(ASM.format(extra=line), "x.hip")


def test_m0_of_other_form_inside_a_block_fails():
    bad = ASM.replace("s_mov_b32 m0, s26", "s_mov_b32 m0, 0x1000")
    with pytest.raises(RuntimeError, match="M0"):
        build.check_m0(bad.format(extra=""), "x.hip")

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

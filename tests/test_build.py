"""Build checks (CPU only): the scratch guard on the decode kernels parses the
compiler's resource-usage remarks."""

from loraforge_amd import _build


def test_scratch_guard_reads_resource_remarks():
    remarks = [
        "nf4_gemv.hip:9:1: remark: Function Name: kernel_a [-Rpass-analysis=kernel-resource-usage]",
        "nf4_gemv.hip:9:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "nf4_gemv.hip:9:1: remark: Function Name: kernel_b [-Rpass-analysis=kernel-resource-usage]",
        "nf4_gemv.hip:9:1: remark:     ScratchSize [bytes/lane]: 44 [-Rpass-analysis=kernel-resource-usage]",
    ]
    assert _build._scratch_users(remarks) == ["kernel_b (44 bytes/lane)"]
    assert "nf4_gemv.hip" in _build.NO_SCRATCH

"""The build's no-scratch guard reads hipcc's kernel-resource-usage remarks."""
from affmae_amd.build_lib import _scratch_kernels

REMARKS = """x.hip:1:1: remark: Function Name: _Z21nbhd_attn_wave_kernelILi4EEvv [-Rpass-analysis=kernel-resource-usage]
x.hip:1:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]
x.hip:1:1: remark:     ScratchSize [bytes/lane]: 20 [-Rpass-analysis=kernel-resource-usage]
x.hip:9:1: remark: Function Name: _Z21nbhd_attn_wave_kernelILi2EEvv [-Rpass-analysis=kernel-resource-usage]
x.hip:9:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark: Function Name: _Z12other_kernelv [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     ScratchSize [bytes/lane]: 64 [-Rpass-analysis=kernel-resource-usage]
"""


def test_scratch_guard_flags_only_matching_kernels_with_scratch():
    bad = _scratch_kernels(REMARKS, "nbhd_attn_wave_kernel")
    assert bad == [("_Z21nbhd_attn_wave_kernelILi4EEvv", 20)]
    assert _scratch_kernels(REMARKS, "knn_win_kernel") == []

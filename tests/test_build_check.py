"""The build's scratch-memory check (CPU): kernels that spill must be listed
in build.SCRATCH_ALLOWED, and the instances the benchmark workloads run are
not."""
from fused_rope_attn_amd import build as B

REMARKS = """\
x.h:1:1: remark: Function Name: _ZN12_GLOBAL__N_113window_kernelILi80ENS_4BF16ELi2ELb0ELi2ELb0EEEvN12fra_internal7KParamsE [-Rpass-analysis=kernel-resource-usage]
x.h:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.h:1:1: remark: Function Name: _ZN12_GLOBAL__N_111long_kernelILi128ENS_4BF16ELi2ELb1ELb1EEEvN12fra_internal7KParamsE [-Rpass-analysis=kernel-resource-usage]
x.h:1:1: remark:     ScratchSize [bytes/lane]: 316 [-Rpass-analysis=kernel-resource-usage]
"""


def test_parse_and_allowlist():
    use = B.scratch_use(REMARKS)
    assert len(use) == 2 and sorted(use.values()) == [0, 316]
    assert B.check_scratch(use) == []


def test_spill_on_a_benchmark_instance_fails():
    # a spill in the headline window kernel (D=80, bf16, fp32 half-width tables) is not allowed
    use = {"_ZN12_GLOBAL__N_113window_kernelILi80ENS_4BF16ELi2ELb0ELi2ELb0EEEvN12fra_internal7KParamsE": 8,
           "_ZN12_GLOBAL__N_111long_kernelILi80ENS_4BF16ELi2ELb0ELb1EEEvN12fra_internal7KParamsE": 4}
    assert len(B.check_scratch(use)) == 2
    # an allowed family beyond its listed size fails too
    assert B.check_scratch({"_ZN12_GLOBAL__N_115bwd_long_kernelILi96ENS_4BF16ELb1ELi4EEEvN12fra_internal7BParamsE": 64})

"""The build's scratch guard: the compiler's kernel-resource remarks are
parsed per function, and a function with per-lane scratch is reported.
CPU only (parses text; the real check runs inside build())."""

from drama3_amd._build import scratch_users

REMARKS = """\
a.hip:24:1: remark: Function Name: _Z6kernelAv [-Rpass-analysis=kernel-resource-usage]
a.hip:24:1: remark:     VGPRs: 8 [-Rpass-analysis=kernel-resource-usage]
a.hip:24:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
a.hip:49:1: remark: Function Name: _Z6kernelBv [-Rpass-analysis=kernel-resource-usage]
a.hip:49:1: remark:     ScratchSize [bytes/lane]: 192 [-Rpass-analysis=kernel-resource-usage]
a.hip:60:1: remark: Function Name: _Z6kernelCv [-Rpass-analysis=kernel-resource-usage]
a.hip:60:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
"""


def test_scratch_users_names_only_functions_with_scratch():
    assert scratch_users(REMARKS) == [("_Z6kernelBv", 192)]
    assert scratch_users(REMARKS.replace("192", "0")) == []
    assert scratch_users("") == []

"""The library build refuses kernels that do not run from registers alone.

deltaattention_amd/build.py parses hipcc's per-kernel resource report and raises
ResourceError on scratch memory, VGPR spills or a dynamic stack (the attention kernels'
hand-issued LDS reads are only correct without spill copies).  CPU tests: the parser on a
recorded report, and a deliberately spilling kernel pushed through the real compile step.
"""
import os
import shutil

import pytest

from deltaattention_amd import build

REPORT = """\
k.hip:3:1: remark: Function Name: _Z4kernPf [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     TotalSGPRs: 20 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     ScratchSize [bytes/lane]: 44 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     Dynamic Stack: False [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     SGPRs Spill: 3 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     VGPRs Spill: 11 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     LDS Size [bytes/block]: 0 [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark: Function Name: _Z4goodPf [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark:     TotalSGPRs: 10 [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark:     VGPRs: 8 [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark:     Dynamic Stack: False [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark:     SGPRs Spill: 5 [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
"""


def test_parse_resource_report():
    ks = build.parse_resource_usage(REPORT)
    assert [k["name"] for k in ks] == ["_Z4kernPf", "_Z4goodPf"]
    assert ks[0]["vgpr"] == 256 and ks[0]["scratch"] == 44 and ks[0]["vgpr_spill"] == 11
    assert ks[0]["sgpr_spill"] == 3 and ks[0]["dynamic_stack"] == "False"
    assert ks[1]["scratch"] == 0 and ks[1]["sgpr_spill"] == 5


def test_gate_rejects_scratch_and_vgpr_spills_only():
    ks = build.parse_resource_usage(REPORT)
    with pytest.raises(build.ResourceError, match="_Z4kernPf"):
        build.check_resources(ks, "k.hip")
    build.check_resources(ks[1:], "k.hip")  # SGPR spills into VGPR lanes are allowed
    with pytest.raises(build.ResourceError):
        build.check_resources([dict(ks[1], dynamic_stack="True")], "k.hip")


SPILLING = r"""
#include <hip/hip_runtime.h>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void spills(const float* in, float* out) {
  float v[300];
#pragma unroll
  for (int i = 0; i < 300; ++i) v[i] = in[(threadIdx.x + i * 977) & 4095];
  for (int it = 0; it < 4; ++it) {
#pragma unroll
    for (int i = 0; i < 300; ++i) v[i] = v[i] * 0.5f + v[(i + 1) % 300];
    __syncthreads();
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 300; ++i) s += v[i] * (float)i;
  out[threadIdx.x] = s;
}
"""


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not available")
def test_real_compile_of_a_spilling_kernel_is_refused(tmp_path):
    src = tmp_path / "spills.hip"
    src.write_text(SPILLING)
    with pytest.raises(build.ResourceError, match="spills"):
        build.compile_checked(str(src), str(tmp_path / "spills.o"))

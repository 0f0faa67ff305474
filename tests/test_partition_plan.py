"""The host's choice of waves per world group (plan_partition in
phyz_amd/csrc/phz_host.cpp), checked without a GPU: the kernel is generated and
compiled with hiprtc for a 256-CU device and its block size read back.

The planner tries caps of 8, 4 and 2 waves and keeps the plan whose busiest
SIMD carries the fewest bodies per step, with the launch's workgroups per CU
dealing their waves to the 4 SIMDs in turn (ties keep more waves). The cases
are the measured ones: the MJCF humanoid runs 2 waves at 32768 worlds (two
workgroups per CU: 4 waves would stack both trunk waves on one SIMD) and 4 at
small sizes; the MJCF hand runs 4 (trunk + finger, finger, finger, two
fingers) instead of one wave per finger, which would put the trunk wave and a
finger wave on one SIMD; the builder humanoid, whose limbs balance, and the
welded-palm hand, whose waves never wait at a barrier, keep one wave per part.
"""
import pytest

from phyz_amd import workloads as W
from phyz_amd.sim import from_workload


@pytest.mark.parametrize("index,nworld,prec,block", [
    (8, 32768, "f32", 128),   # MJCF humanoid, 512 workgroups: 2 waves
    (8, 96, "f32", 256),      # MJCF humanoid, 2 workgroups: 4 waves
    (9, 16384, "f32", 256),   # MJCF hand: 4 waves
    (4, 32768, "f32", 256),   # builder humanoid: 4 waves (trunk+arm 6, arm 4, legs 6 and 6)
    (5, 16384, "f64", 320),   # builder hand (welded palm, no barrier): 5 waves
])
def test_waves_per_world_group(index, nworld, prec, block):
    s = from_workload(W.config(index), prec, nworld=nworld, device=-1)
    s.compile()
    assert s.kernel_info()["block"] == block

"""The host's choice of waves per world group (plan_partition in
phyz_amd/csrc/phz_host.cpp), checked without a GPU: the kernel is generated and
compiled with hiprtc for a 256-CU device and its block size (and, from the
generated source, its groups) read back.

The planner prices a step in body weights: each wave's own bodies, the
floating trunk's pass 1 on every wave, and the trunk's passes 2 and 3, which
wave 0 runs while the other waves wait at the barrier. One wave fits a SIMD, so
workgroups beyond floor(4 / waves) per CU run in further rounds. The cases are
the measured ones: at 32768 worlds (two workgroups per CU) the MJCF humanoid
and the builder humanoid run 2 waves (4 waves would
run the two workgroups one after the other, paying the serial trunk section
twice); at small sizes 4; the MJCF hand runs 4 (a 4-body finger beside the
trunk's contacts, a finger, a finger, two fingers) rather than one wave per
finger, which would put two waves on one SIMD; the welded-palm hand, whose waves never wait at a barrier, keeps
one wave per finger.
"""
import pytest

from phyz_amd import workloads as W
from phyz_amd.sim import from_workload


@pytest.mark.parametrize("index,nworld,prec,block", [
    (8, 32768, "f32", 128),   # MJCF humanoid, 512 workgroups: 2 waves
    (8, 96, "f32", 256),      # MJCF humanoid, 2 workgroups: 4 waves
    (9, 16384, "f32", 256),   # MJCF hand: 4 waves
    (4, 32768, "f32", 128),   # builder humanoid: 2 waves (a leg and an arm each)
    (4, 96, "f32", 256),      # builder humanoid, 2 workgroups: 4 waves
    (5, 16384, "f64", 320),   # builder hand (welded palm, no barrier): 5 waves
    (8, 32768, "f64", 256),   # MJCF humanoid f64: one wave per subtree, never merged
    (9, 16384, "f64", 320),   # MJCF hand f64: one wave per finger, never merged
])
def test_waves_per_world_group(index, nworld, prec, block):
    s = from_workload(W.config(index), prec, nworld=nworld, device=-1)
    s.compile()
    assert s.kernel_info()["block"] == block


@pytest.mark.parametrize("index,prec,groups", [
    (8, "f32", [6, 8]),    # MJCF humanoid: both arms with the trunk's contacts, both legs
    (4, "f32", [10, 10]),  # builder humanoid: leg (6) + arm (4) on each wave
])
def test_two_wave_plans_balance_limbs(index, prec, groups, tmp_path, monkeypatch):
    """Wave 0 runs the trunk's passes 2 and 3 while the other wave waits at the
    barrier, so that section is on both waves' clocks and is not charged to
    wave 0 alone. The trunk's ground contacts, which only wave 0 computes, are
    (MJCF humanoid: 10.43 ms per 1000 steps with this plan, 10.55 ms with a
    leg and an arm on each wave, 13.01 ms with the trunk and one leg on wave
    0)."""
    import re
    src = tmp_path / "step.hip"
    monkeypatch.setenv("PHZ_DUMP_SOURCE", str(src))
    s = from_workload(W.config(index), prec, nworld=32768, device=-1)
    s.compile()
    glen = re.search(r"static constexpr int glen\[2\] = \{(\d+), (\d+)\}", src.read_text())
    assert glen is not None
    assert sorted(int(x) for x in glen.groups()) == groups


def _three_limb_model(base_joint: str, links: int):
    """A root with three limbs of `links` revolute links each: the planner sees
    exactly three parts below the trunk."""
    import numpy as np
    from phyz_amd.model import FIXED, FREE, Joint, ModelBuilder, SpatialInertia, SpatialTransform

    b = ModelBuilder().gravity([0.0, 0.0, -9.81]).dt(0.001)
    jt = FREE if base_joint == "free" else FIXED
    b.add_body("root", -1, Joint(jt, SpatialTransform.identity(), np.zeros(3)),
               SpatialInertia.new(1.0, [0.0, 0.0, 0.0], np.eye(3) * 0.01))
    for limb in range(3):
        parent = 0
        for k in range(links):
            ptj = SpatialTransform.from_translation([0.1, 0.05 * (limb - 1), 0.0] if k == 0 else [0.2, 0.0, 0.0])
            idx = len(b._bodies)
            b.add_revolute_body(f"l{limb}_{k}", parent, ptj,
                                SpatialInertia.new(0.5, [0.1, 0.0, 0.0], np.diag([1e-3, 2e-3, 2e-3])),
                                axis=(0.0, 1.0, 0.0) if k % 2 else (0.0, 0.0, 1.0))
            parent = idx
    return b.build()


@pytest.mark.parametrize("base,links", [("fixed", 2), ("fixed", 6), ("free", 5)])
@pytest.mark.parametrize("nworld", [64, 65536])
@pytest.mark.parametrize("max_groups", [None, "4", "8"])
def test_no_three_wave_plan(base, links, nworld, max_groups, monkeypatch):
    """A tree with exactly three subtrees below its trunk (a welded base, any
    size; a floating base with 14 or more bodies) is never given a 3-wave
    (192-thread) kernel, whatever the planner's cap or PHZ_MAX_GROUPS."""
    from phyz_amd.sim import BatchSim

    if max_groups is None:
        monkeypatch.delenv("PHZ_MAX_GROUPS", raising=False)
    else:
        monkeypatch.setenv("PHZ_MAX_GROUPS", max_groups)
    m = _three_limb_model(base, links)
    s = BatchSim(m, nworld, "f64", device=-1)
    s.compile()
    assert s.kernel_info()["block"] in (64, 128), s.kernel_info()


@pytest.mark.parametrize("index,block", [(8, 256), (9, 320)])
def test_f64_never_merges_subtrees(index, block, monkeypatch):
    """A cap below the subtree count merges subtrees into one wave in f32 only:
    in f64 the planner keeps one subtree per wave (the MJCF humanoid's merged
    f64 kernels gave NaN or launch-varying values from launches of many
    steps)."""
    monkeypatch.setenv("PHZ_MAX_GROUPS", "2")
    s32 = from_workload(W.config(index), "f32", nworld=96, device=-1)
    s32.compile()
    assert s32.kernel_info()["block"] == 128
    s64 = from_workload(W.config(index), "f64", nworld=96, device=-1)
    s64.compile()
    assert s64.kernel_info()["block"] == block


@pytest.mark.parametrize("index,nworld,prec,lanes", [
    (1, 4096, "f64", 2),     # double pendulum, 64 workgroups: two lanes per world
    (1, 4096, "f32", 2),     # in f32 too
    (1, 32768, "f64", 2),    # 1024 split waves: one per SIMD
    (1, 65536, "f64", 1),    # beyond one per SIMD
    (2, 1024, "f64", 4),     # chain7 at 1024 worlds: four lanes
    (2, 4096, "f64", 4),     # 256 split waves: one per CU
    (2, 8192, "f64", 1),     # 512 split waves: one lane
    (2, 1024, "f32", 1),     # f32 chain7 never splits (hardware sincos)
    (2, 65536, "f64", 1),    # chain7 at 65536 worlds fills the SIMDs already
    (3, 1024, "f64", 1),     # contact keeps one lane
])
def test_lanes_per_world(index, nworld, prec, lanes, monkeypatch):
    """Small launches split each world's revolute-joint sincos over 2 lanes
    (two revolute joints) while the split waves fit one per SIMD, and over 4
    lanes only in f64 while they fit one per CU (the measured rule in
    lanes_per_world); PHZ_LANES=1 turns the split off, and PHZ_LANES=4 forces
    it wherever the model allows it."""
    monkeypatch.delenv("PHZ_LANES", raising=False)
    s = from_workload(W.config(index), prec, nworld=nworld, device=-1)
    s.compile()
    assert s.kernel_info()["lanes_per_world"] == lanes
    monkeypatch.setenv("PHZ_LANES", "1")
    s = from_workload(W.config(index), prec, nworld=nworld, device=-1)
    s.compile()
    assert s.kernel_info()["lanes_per_world"] == 1
    monkeypatch.setenv("PHZ_LANES", "4")
    s = from_workload(W.config(index), prec, nworld=nworld, device=-1)
    s.compile()
    assert s.kernel_info()["lanes_per_world"] == {1: 2, 2: 4, 3: 1}[index]


@pytest.mark.parametrize("index,nworld,prec,two", [
    (3, 131072, "f32", True),    # ant: 2048 waves over 1024 SIMDs, 356 registers
    (3, 262144, "f32", True),
    (3, 65536, "f32", False),    # one wave per SIMD either way
    (7, 131072, "f32", True),    # MJCF ant: both kernels in order (reassociated: 960 bytes of spills)
    (7, 65536, "f32", False),
    (2, 131072, "f64", False),   # chain7 f64: 284 bytes of 8-byte spills
    (2, 65536, "f64", False),
    (2, 262144, "f32", False),   # chain7 f32 already fits two waves per SIMD
    (6, 131072, "f32", False),   # terrain + impulse: its two-wave build spills too much
])
def test_two_waves_per_simd(index, nworld, prec, two, monkeypatch):
    """A one-wave-per-world-group kernel above 256 registers gets a second
    build of the same arithmetic for two resident waves per SIMD (run by
    launches of 16 steps or more) when the launch has more waves than SIMDs
    and the rebuild spills at most 512 bytes per lane (f32 reassociated; 768
    in order, which then builds both kernels in order; 128 for f64);
    kernel_info reports the kernel of a full launch. PHZ_TWO_WAVES=0 keeps
    one wave per SIMD."""
    monkeypatch.delenv("PHZ_TWO_WAVES", raising=False)
    s = from_workload(W.config(index), prec, nworld=nworld, device=-1)
    s.compile()
    info = s.kernel_info()
    assert (info["vgpr"] + max(info["agpr"], 0) <= 256 and info["scratch_bytes"] > 0) == two
    if two:
        assert info["scratch_bytes"] <= 768
        monkeypatch.setenv("PHZ_TWO_WAVES", "0")
        s = from_workload(W.config(index), prec, nworld=nworld, device=-1)
        s.compile()
        one = s.kernel_info()
        assert one["vgpr"] + one["agpr"] > 256 and one["scratch_bytes"] == 0


@pytest.mark.parametrize("nworld,two", [(131072, True), (32768, False)])
def test_two_wave_policy_kernel(nworld, two, monkeypatch):
    """The control loop's policy kernel (about 370 registers at hidden 256) is
    built for two resident waves per SIMD when the launch has more waves than
    SIMDs (131072 worlds: 4096 waves of 32 worlds), spilling at most 512 bytes
    per lane; PHZ_TWO_WAVES=0 keeps one."""
    from phyz_amd.sim import from_control_loop
    monkeypatch.delenv("PHZ_TWO_WAVES", raising=False)
    info = from_control_loop(W.control_loop(), "f32", nworld=nworld, device=-1).control_kernel_info("policy")
    assert (info["scratch_bytes"] > 0) == two
    assert info["scratch_bytes"] <= 512
    monkeypatch.setenv("PHZ_TWO_WAVES", "0")
    info = from_control_loop(W.control_loop(), "f32", nworld=nworld, device=-1).control_kernel_info("policy")
    assert info["scratch_bytes"] == 0 and info["vgpr"] + info["agpr"] > 256

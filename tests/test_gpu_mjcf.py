"""The reference's MJCF benchmark models on the device, with the CPU model's
actuators, soft joint limits and dry friction (whose oracle restatement is
pinned in tests/test_mjcf.py), against the oracle.

One device step from the same states (qdd, with limits violated, controls
past their ranges, contact on), then rollouts under the replayed actuator
noise stream. f64 kernels are held to 1e-10 (one step) and 1e-8 (rollouts);
f32 kernels to 1e-4.
"""
import os

import numpy as np
import pytest

from oracle.oracle import Oracle
from phyz_amd import workloads as W
from phyz_amd.mjcf import MjcfLoader
from phyz_amd.model import pack_geometries, uniform_frequency_gains
from phyz_amd.sim import BatchSim, from_workload
from tests.helpers import as_precision, rel_err_rows

pytestmark = pytest.mark.gpu

MODELS = ["ant", "humanoid", "shadow_hand", "half_cheetah"]
NOISE = (0xA55, 1, -0.03, 0.03)  # uniform controls, about twice the converted ctrlrange


def states(m, n, seed):
    rng = np.random.default_rng(seed)
    q = np.zeros((n, m.nq))
    v = rng.normal(size=(n, m.nv)) * 0.5
    for i, b in enumerate(m.bodies):
        j, o = b.joint, m.q_offsets[i]
        if j.ndof() == 1:
            lo, hi = j.limits if j.limits is not None else (-1.0, 1.0)
            q[:, o] = rng.uniform(lo - 0.1, hi + 0.1, size=n)  # some worlds past each limit
        elif j.ndof() == 6:
            q[:, o:o + 3] = rng.normal(size=(n, 3)) * 0.2
            q[:, o + 3:o + 6] = rng.normal(size=(n, 3)) * 0.05
    c = rng.uniform(-0.05, 0.05, size=(n, m.nctrl()))
    return q, v, c


def build(m, n, prec, noise=False):
    gains = uniform_frequency_gains(m, 50.0, 1.0)
    geom, _ = pack_geometries(m, gains=gains)
    orc = Oracle(m, contact=(geom, 0.0, 1.0),
                 noise=None if not noise else (*NOISE, list(range(m.nctrl()))))
    s = BatchSim(m, n, prec)
    s.enable_ground_contact_per_body(0.0, 1.0, gains)
    if noise:
        s.enable_control_noise(*NOISE, list(range(m.nctrl())))
    return s, orc


@pytest.mark.parametrize("prec", ["f64", "f32"])
@pytest.mark.parametrize("name", MODELS)
def test_mjcf_model_step_matches_oracle(name, prec):
    """Also the regression case for the kernels' finite-math rule: the
    half-cheetah's f64 contact kernel gave wrong accelerations at -O3 while a
    select discarded a division by a vanishing value; every such denominator
    is now guarded."""
    m = W.mjcf_model(name)
    n = 200
    s, orc = build(m, n, prec)
    assert s.nctrl == m.nu()
    q, v, c = (as_precision(a, prec) for a in states(m, n, seed=len(name)))
    s.load_states(q, v, c)
    s.step()
    qdd = s.readback_qdd()
    assert np.array_equal(s.readback_controls(), c)  # actuator controls are inputs, not overwritten
    want, _ = orc.step_batch(q.copy(), v.copy(), c.copy(), 1, threads=8)
    err = rel_err_rows(qdd, want)
    print(f"{name} {prec}: qdd max {err.max():.2e} median {np.median(err):.2e}", flush=True)
    assert err.max() <= (1e-10 if prec == "f64" else 1e-4)


def inside_limits(m, q, margin=0.05):
    q = q.copy()
    for i, b in enumerate(m.bodies):
        if b.joint.ndof() == 1 and b.joint.limits is not None:
            lo, hi = b.joint.limits
            o = m.q_offsets[i]
            q[:, o] = np.clip(q[:, o], lo + margin, hi - margin)
    return q


@pytest.mark.parametrize("name", MODELS)
def test_mjcf_model_rollout_f64(name):
    """100 steps under the replayed actuator noise from states inside the
    limits. The reference's explicit limit law (stiffness 1000, damping 60)
    is unstable on the lightest links once they reach a limit (on the hand,
    damping / inertia x dt is about 100), so some worlds diverge in the
    oracle as well: the device must diverge on exactly those, and match the
    oracle on the rest, which must be most of the batch."""
    m = W.mjcf_model(name)
    n = 128
    s, orc = build(m, n, "f64", noise=True)
    q, v, c = states(m, n, seed=7)
    q = inside_limits(m, q)
    v *= 0.2
    s.load_states(q, v, c)
    s.step_many(60)
    s.step_many(40)
    qd, vd = s.readback_states()
    orc.step_batch(q, v, c, 100, rng=orc.rng_states(n), threads=8)
    fin = np.isfinite(q).all(axis=1) & np.isfinite(v).all(axis=1) & (np.abs(v).max(axis=1) < 1e4)
    dfin = np.isfinite(qd).all(axis=1) & np.isfinite(vd).all(axis=1) & (np.abs(vd).max(axis=1) < 1e4)
    dq = np.abs(qd[fin] - q[fin]).max()
    dv = np.abs(vd[fin] - v[fin]).max() / max(1.0, np.abs(v[fin]).max())
    print(f"{name}: {fin.sum()}/{n} worlds stay finite; 100-step f64 divergence q {dq:.2e} v {dv:.2e}", flush=True)
    assert fin.mean() >= 0.75
    assert np.array_equal(fin, dfin)
    assert dq <= 1e-8 and dv <= 1e-8


FRICTION_ARM = """<mujoco><option gravity="0 0 -9.81" timestep="0.001"/>
  <default><joint damping="0.05" armature="0.002"/><geom type="capsule" size="0.03"/></default>
  <worldbody><body name="a" pos="0 0 1"><joint name="j0" axis="0 1 0" range="-0.5 0.5" frictionloss="0.3"/>
      <geom fromto="0 0 0 0.3 0 0"/>
      <body name="b" pos="0.3 0 0"><joint name="j1" axis="0 1 0" range="-1 0.2" frictionloss="0.1" stiffness="2"/>
        <geom fromto="0 0 0 0.25 0 0"/>
        <body name="c" pos="0.25 0 0"><joint name="j2" type="slide" axis="1 0 0" range="-0.05 0.05" frictionloss="0.5"/>
          <geom type="sphere" size="0.05"/></body></body></body></worldbody>
  <actuator><velocity joint="j0" kv="4" forcerange="-1.5 1.5"/><general joint="j1" gainprm="3" biasprm="0 -2 -0.5"/>
    <position joint="j2" kp="50" kv="1" ctrlrange="-0.1 0.1"/></actuator></mujoco>"""


@pytest.mark.parametrize("prec", ["f64", "f32"])
def test_friction_loss_force_range_and_servos(prec):
    """Dry friction across stick and slip speeds, a velocity servo clipped by
    its force range, a general actuator with bias terms, a slide joint past
    both limits."""
    m = MjcfLoader.from_xml_str(FRICTION_ARM).build_model()
    n = 256
    rng = np.random.default_rng(5)
    q = np.column_stack([rng.uniform(-0.7, 0.7, n), rng.uniform(-1.2, 0.4, n), rng.uniform(-0.08, 0.08, n)])
    v = rng.normal(size=(n, 3)) * np.array([1.0, 1.0, 0.05])
    v[:64] *= 1e-3  # inside tanh's linear range
    c = rng.uniform(-2, 2, size=(n, 3))
    q, v, c = (as_precision(a, prec) for a in (q, v, c))
    s = BatchSim(m, n, prec)
    o = Oracle(m)
    s.load_states(q, v, c)
    s.step()
    want, _ = o.step_batch(q.copy(), v.copy(), c.copy(), 1)
    err = rel_err_rows(s.readback_qdd(), want)
    print(f"friction arm {prec}: qdd {err.max():.2e}", flush=True)
    assert err.max() <= (1e-10 if prec == "f64" else 1e-4)
    s.step_many(200)
    qd, _ = s.readback_states()
    o.step_batch(q, v, c, 201)  # the step above and these 200
    assert np.abs(qd - q).max() <= (1e-8 if prec == "f64" else 2e-3)


def test_mjcf_hand_partitioned_equals_lane_per_world():
    """The hand's trunk runs through its two wrist hinges (floating-trunk
    partition); its rollouts equal the one-lane-per-world kernel's."""
    m = W.mjcf_model("shadow_hand")
    n = 96
    q, v, c = states(m, n, seed=11)
    q = inside_limits(m, q)
    v *= 0.2
    out = []
    for mode in ("auto", "0"):
        os.environ["PHZ_PARTITION"] = mode
        try:
            s, _ = build(m, n, "f64", noise=True)
            s.compile()
            blk = s.kernel_info()["block"]
            s.load_states(q, v, c)
            s.step_many(50)
            out.append((blk, s.readback_states()))
        finally:
            os.environ.pop("PHZ_PARTITION", None)
    assert out[0][0] == 320 and out[1][0] == 64  # f64 keeps one finger per wave: 5 waves
    (qa, va), (qb, vb) = out[0][1], out[1][1]
    fa = np.isfinite(qa).all(axis=1) & (np.abs(va).max(axis=1) < 1e4)
    fb = np.isfinite(qb).all(axis=1) & (np.abs(vb).max(axis=1) < 1e4)
    assert np.array_equal(fa, fb) and fa.mean() >= 0.75
    assert np.abs(qa[fa] - qb[fa]).max() <= 1e-9
    assert np.abs(va[fa] - vb[fa]).max() <= 1e-8 * max(1.0, np.abs(vb[fa]).max())


THREE_WAVE_F64 = ("the humanoid's 3-wave f64 kernel with control noise (512 VGPR+AGPR, 364 B scratch) "
                  "returned launch-varying values of order 1e67 from the first step, while the same plan "
                  "without noise equals the one-lane-per-world kernel over 50 steps; no cause found in the "
                  "source, so launches never get this plan (the planner picks among caps 8, 4 and 2, and "
                  "PHZ_MAX_GROUPS rounds down to 1, 2, 4 or 8)")


UNMERGED_WAVES = {"humanoid": 4, "shadow_hand": 5}  # subtrees below the floating trunk


@pytest.mark.parametrize("name,groups", [("shadow_hand", 4), ("shadow_hand", 2), ("humanoid", 2),
                                         pytest.param("humanoid", 3, marks=pytest.mark.skip(reason=THREE_WAVE_F64))])
def test_mjcf_merged_groups_match(name, groups):
    """The planner may give a world group fewer waves than the tree has parts
    (the hand runs 4 waves, the humanoid's 32768 worlds run 2), so several
    subtrees share one wave's code. PHZ_MAX_GROUPS forces that plan at
    a small size: one f32 step matches the oracle. f64 plans never merge
    subtrees (the merged f64 humanoid kernel's 50-step launches went NaN while
    one-step launches of the same binary did not), so under the same cap the
    f64 kernel keeps one subtree per wave; its rollout equals the
    one-lane-per-world kernel's and a repeated rollout is bit-identical."""
    m = W.mjcf_model(name)
    n = 96
    q, v, c = states(m, n, seed=13)
    os.environ["PHZ_MAX_GROUPS"] = str(groups)
    try:
        s, o = build(m, n, "f32")
        s.compile()
        assert s.kernel_info()["block"] == 64 * groups
        qf, vf, cf = (as_precision(a, "f32") for a in (q, v, c))
        s.load_states(qf, vf, cf)
        s.step()
        want, _ = o.step_batch(qf.copy(), vf.copy(), cf.copy(), 1)
        err = rel_err_rows(s.readback_qdd(), want)
        print(f"{name} {groups} waves f32: qdd {err.max():.2e}", flush=True)
        assert err.max() <= 1e-4
    finally:
        os.environ.pop("PHZ_MAX_GROUPS", None)
    q = inside_limits(m, q)
    v *= 0.2
    out = []
    for key, val in (("PHZ_MAX_GROUPS", str(groups)), ("PHZ_MAX_GROUPS", str(groups)), ("PHZ_PARTITION", "0")):
        os.environ[key] = val
        try:
            s, _ = build(m, n, "f64", noise=True)
            s.compile()
            blk = s.kernel_info()["block"]
            s.load_states(q, v, c)
            s.step_many(50)
            out.append((blk, s.readback_states()))
        finally:
            os.environ.pop(key, None)
    unmerged = 64 * UNMERGED_WAVES[name]
    assert out[0][0] == out[1][0] == unmerged and out[2][0] == 64
    (qa, va), (qr, vr), (qb, vb) = out[0][1], out[1][1], out[2][1]
    assert np.array_equal(qa.view(np.uint64), qr.view(np.uint64)) and np.array_equal(va.view(np.uint64), vr.view(np.uint64))
    fa = np.isfinite(qa).all(axis=1) & (np.abs(va).max(axis=1) < 1e4)
    fb = np.isfinite(qb).all(axis=1) & (np.abs(vb).max(axis=1) < 1e4)
    assert np.array_equal(fa, fb) and fa.mean() >= 0.5
    assert np.abs(qa[fa] - qb[fa]).max() <= 1e-9
    assert np.abs(va[fa] - vb[fa]).max() <= 1e-8 * max(1.0, np.abs(vb[fa]).max())


def _span_bits(sim, q, v, c, tg, steps, reps):
    out = []
    for _ in range(reps):
        sim.load_states(q, v, c)
        if tg is not None:
            sim.set_position_targets(tg)
        sim.step_many(steps)
        qg, vg = sim.readback_states()
        out.append((qg.copy(), vg.copy()))
    return out


@pytest.mark.parametrize("cfg,nworld,groups", [(8, 32768, None), (9, 16384, None), (8, 2048, 2), (9, 2048, 2)])
def test_merged_f32_plans_multistep_repeat(cfg, nworld, groups):
    """The merged f32 plans the benchmarks run (the MJCF humanoid's 2 waves at
    32768 worlds, the hand's 4 waves at 16384, five fingers on four waves) and
    the 2-wave cap at a small size, over 200-step launches: repeated from the
    same state they give the same bits, every world stays finite, and the
    states stay within the f32 rollout bound of the one-lane-per-world
    kernel's (the two differ only in the order the trunk sums its subtrees'
    contributions)."""
    w = W.config(cfg)
    q, v, c, tg = w.initial_state(nworld)
    if groups is not None:
        os.environ["PHZ_MAX_GROUPS"] = str(groups)
    try:
        sim = from_workload(w, "f32", nworld=nworld)
        info = sim.kernel_info()
    finally:
        os.environ.pop("PHZ_MAX_GROUPS", None)
    parts = UNMERGED_WAVES[{8: "humanoid", 9: "shadow_hand"}[cfg]]
    waves = info["block"] // 64
    print(f"cfg {cfg} f32, {nworld} worlds: {waves} waves for {parts} subtrees, kernel {info}", flush=True)
    assert 1 < waves < parts  # subtrees share waves
    outs = _span_bits(sim, q, v, c, tg, 200, 3)
    for k, (qg, vg) in enumerate(outs[1:], start=1):
        same = np.all(qg.view(np.uint32) == outs[0][0].view(np.uint32), axis=1) & \
            np.all(vg.view(np.uint32) == outs[0][1].view(np.uint32), axis=1)
        assert same.all(), f"repeat {k} differs in {(~same).sum()} worlds"
    qa, va = outs[0]
    assert np.isfinite(qa).all() and np.isfinite(va).all()
    os.environ["PHZ_PARTITION"] = "0"
    try:
        one = from_workload(w, "f32", nworld=nworld)
        assert one.kernel_info()["block"] == 64
        (qb, vb), = _span_bits(one, q, v, c, tg, 200, 1)
    finally:
        os.environ.pop("PHZ_PARTITION", None)
    dq = np.abs(qa - qb).max(axis=1)
    dv = np.abs(va - vb).max(axis=1) / np.maximum(1.0, np.abs(vb).max(axis=1))
    print(f"  merged vs one lane after 200 steps: q max {dq.max():.2e} p99 {np.percentile(dq, 99):.2e} "
          f"median {np.median(dq):.2e}; v max {dv.max():.2e} p99 {np.percentile(dv, 99):.2e}", flush=True)
    # Measured: q max 1.0e-6, v max 2.5e-6 (relative) over these cases.
    assert dq.max() <= 1e-5 and dv.max() <= 1e-5

"""Device-resident control loop against the CPU oracle (oracle/policy_ref.py).

Ports of the reference suites crates/phyz-gpu/tests/cuda_vs_cpu.rs:
suite_policy (874-1115), suite_policy_base_targets (1124-1170),
suite_policy_clamp_slots (1180-1282) and suite_policy_support (1455-1651), with
the reference's tolerances (f32 device: observations 1e-4, actions and targets
2e-4, log-prob 1e-3, FK 1e-5), plus the MFMA tiling at full widths (hidden 256,
ragged widths, partial world tiles), the captured rollout, and NaN isolation.
The random streams are replayed exactly on the CPU (world_seed + xorshift64 +
Box–Muller), so the comparison is per value, not statistical.
"""
import math

import numpy as np
import pytest

from oracle import policy_ref as PR
from oracle.oracle import Oracle
from phyz_amd import policy as P
from phyz_amd import workloads as W
from phyz_amd.model import PdDof
from phyz_amd.sim import BatchSim, PhzError
from tests import models as TM

pytestmark = pytest.mark.gpu


def cpu_policy_step(model, orc, spec, weights, std, rngs, zs, base, q, v):
    """One control step of every world on the CPU from the device's q, v."""
    obs, act, logp, tg = [], [], [], []
    for w in range(q.shape[0]):
        o = np.array(PR.observe_reference(model, orc, q[w], v[w], spec.obs))
        t = np.zeros(len(base[w]))
        a, lp = PR.policy_reference(spec, weights, std, rngs[w], o, zs[w], np.asarray(base[w], dtype=float), t)
        obs.append(o)
        act.append(a)
        logp.append(lp)
        tg.append(t)
    return np.array(obs), np.array(act), np.array(logp), np.array(tg)


def free_base_states(model, nworld, limb_q, limb_v):
    q = np.zeros((nworld, model.nq))
    v = np.zeros((nworld, model.nv))
    for w in range(nworld):
        f = float(w)
        q[w, 0], q[w, 1], q[w, 2], q[w, 5] = 0.2 * f, -0.1 * f, 0.3 * f, 1.0 + 0.1 * f
        q[w, limb_q] = 0.4 - 0.2 * f
        v[w, 0], v[w, 1], v[w, 3], v[w, limb_v] = 0.5 * f, -0.2, 0.1 * f, 0.7
    return q, v


@pytest.mark.parametrize("prec", ["f32", "f64"])
def test_policy_loop_matches_cpu(prec):
    """suite_policy: three control steps with physics between them."""
    model = TM.free_base_with_limb()
    nworld = 4
    lq, lv = model.q_offsets[1], model.v_offsets[1]
    sim = BatchSim(model, nworld, prec)
    sim.enable_pd_control([PdDof(lq, lv, 20.0, 1.0, 10.0)])
    spec = P.PolicySpec(
        obs=[P.BodyPitch(0), P.BodyRoll(0), P.V(0), P.V(1), P.V(2), P.QMinus(lq, 0.1), P.V(lv), P.Const(0.5),
             P.BodyYawError(0, 0.3), P.BodyPosZ(1)],
        hidden=16, act_slots=[0], act_clamp=0.4, noise_rho=0.3,
        input_noise=[0.01, 0.01, 0.0, 0.0, 0.0, 0.02, 0.0, 0.0, 0.0, 0.0], history_steps=3)
    sim.enable_policy(spec)
    wr = PR.KernelRng(0xC0FFEE)
    weights = np.array([0.3 * wr.normal() for _ in range(spec.n_weights())])
    std = np.array([0.2])
    base = [[0.05 * w] for w in range(nworld)]
    sim.set_policy_weights(weights)
    sim.set_policy_std(std)
    sim.set_policy_base_targets(base)
    seed = 99
    sim.seed_policy(seed)
    q0, v0 = free_base_states(model, nworld, lq, lv)
    sim.load_states(q0, v0)
    sim.enable_state_history(2)

    orc = Oracle(model)
    rngs = [PR.KernelRng.for_world(seed, w) for w in range(nworld)]
    zs = [np.zeros(1) for _ in range(nworld)]
    want_obs, want_act, want_logp = [], [], []
    after_first = None
    for step in range(3):
        if step == 0:
            sim.record_state(0)
        sim.run_policy(step)
        q, v = sim.readback_states()
        o, a, lp, tg = cpu_policy_step(model, orc, spec, weights, std, rngs, zs, base, q, v)
        want_obs.append(o)
        want_act.append(a)
        want_logp.append(lp)
        got_t = sim.readback_targets()
        d = np.abs(got_t - tg).max()
        print(f"{prec} step {step}: target diff {d:.2e}", flush=True)
        assert d < 2e-4
        for _ in range(5):
            sim.step()
        if step == 0:
            sim.record_state(1)
            after_first = sim.readback_states()

    obs_h, out_h = sim.readback_policy_history(0, 3)
    do = np.abs(obs_h - np.array(want_obs)).max()
    da = np.abs(out_h[:, :, :1] - np.array(want_act)).max()
    dl = np.abs(out_h[:, :, 1] - np.array(want_logp)).max()
    print(f"{prec}: obs {do:.2e} act {da:.2e} logp {dl:.2e}", flush=True)
    assert do < 1e-4 and da < 2e-4 and dl < 1e-3
    # The physics ran between steps and the noise was recorded.
    assert obs_h[0, 0, 0] != obs_h[1, 0, 0] or obs_h[0, 0, 5] != obs_h[1, 0, 5]

    # FK readout against the oracle's FK on the same state.
    sim.compute_kinematics()
    kin = sim.readback_kinematics()
    q, v = sim.readback_states()
    for w in range(nworld):
        want = PR.kinematics_rows(orc, q[w], v[w])
        tol = 1e-5 if prec == "f32" else 1e-12
        assert np.abs(kin[w] - want).max() < tol

    # State history: slot 0 the loaded state, slot 1 after the first five steps.
    qh, vh = sim.readback_state_history(0, 2)
    tol = 1e-6 if prec == "f32" else 0.0
    assert np.abs(qh[0] - q0).max() <= tol and np.abs(vh[0] - v0).max() <= tol
    assert np.array_equal(qh[1], after_first[0]) and np.array_equal(vh[1], after_first[1])

    # Shape guards.
    with pytest.raises(PhzError, match="exceeds history_steps"):
        sim.run_policy(3)
    with pytest.raises(PhzError, match="exceeds 2 slots"):
        sim.record_state(2)
    bad = P.PolicySpec(**{**spec.__dict__, "act_slots": [7]})
    with pytest.raises(PhzError, match="action slot 7 exceeds the 1 registered PD servos"):
        sim.enable_policy(bad)


def arm_pd():
    return [PdDof(k, k, 20.0, 1.0, 10.0) for k in range(4)]


def test_policy_writes_every_base_target():
    """suite_policy_base_targets: zero weights, near-zero std: every servo reads its base."""
    model = TM.arm_6dof()
    nworld = 3
    spec = P.PolicySpec(obs=[P.Const(1.0), P.QMinus(0, 0.0), P.V(0)], hidden=8, act_slots=[0, 2], act_clamp=0.5,
                        input_noise=[0.0] * 3, history_steps=1)
    base = [[0.1 + 0.01 * (4 * w + j) for j in range(4)] for w in range(nworld)]
    sim = BatchSim(model, nworld, "f32")
    sim.enable_pd_control(arm_pd())
    sim.enable_policy(spec)
    sim.set_policy_weights(np.zeros(spec.n_weights()))
    sim.set_policy_std([1e-9] * 2)
    sim.set_policy_base_targets(base)
    sim.seed_policy(11)
    sim.load_states(np.zeros((nworld, model.nq)), np.zeros((nworld, model.nv)))
    sim.run_policy(0)
    assert np.abs(sim.readback_targets() - np.array(base)).max() < 1e-6


def test_policy_clamps_per_action_slot():
    """suite_policy_clamp_slots: each slot saturates at its own clamp; a broadcast
    per-slot clamp is the scalar path bit for bit."""
    model = TM.arm_6dof()
    nworld = 3
    base = [[0.1 + 0.01 * (4 * w + j) for j in range(4)] for w in range(nworld)]
    wr = PR.KernelRng(0x5EED)
    spec0 = P.PolicySpec(obs=[P.Const(1.0), P.QMinus(0, 0.0), P.V(0)], hidden=8, act_slots=[0, 2], act_clamp=0.5,
                         act_clamp_slots=[0.02, 0.7], input_noise=[0.0] * 3, history_steps=1)
    weights = np.array([4.0 * wr.normal() for _ in range(spec0.n_weights())])

    def run(spec):
        sim = BatchSim(model, nworld, "f32")
        sim.enable_pd_control(arm_pd())
        sim.enable_policy(spec)
        sim.set_policy_weights(weights)
        sim.set_policy_std([0.1, 0.1])
        sim.set_policy_base_targets(base)
        sim.seed_policy(4242)
        sim.load_states(np.zeros((nworld, model.nq)), np.zeros((nworld, model.nv)))
        sim.run_policy(0)
        _, out = sim.readback_policy_history(0, 1)
        return sim.readback_targets(), out[0, :, :2]

    got, acts = run(spec0)
    lim = [0.02, 0.7]
    for w in range(nworld):
        for k, slot in enumerate([0, 2]):
            a = acts[w, k]
            want = base[w][slot] + np.clip(a, -lim[k], lim[k])
            assert abs(got[w, slot] - want) < 2e-6
            assert abs(a) > lim[k], "the action must reach its clamp for the test to mean anything"
    assert abs(got[0, 0] - base[0][0]) < 0.5 * abs(got[0, 2] - base[0][2])
    a, _ = run(P.PolicySpec(**{**spec0.__dict__, "act_clamp": 0.37, "act_clamp_slots": None}))
    b, _ = run(P.PolicySpec(**{**spec0.__dict__, "act_clamp": 0.37, "act_clamp_slots": [0.37, 0.37]}))
    assert np.array_equal(a, b)
    sim = BatchSim(model, nworld, "f32")
    sim.enable_pd_control(arm_pd())
    with pytest.raises(ValueError, match="act_clamp_slots has 1 entries for 2 actions"):
        sim.enable_policy(P.PolicySpec(**{**spec0.__dict__, "act_clamp_slots": [0.1]}))


def test_com_over_support_matches_cpu():
    """suite_policy_support: BodyPos and ComOverSupport (heading frame and world
    frame) over yawed, tilted rigs, two control steps, 1e-5."""
    model = TM.trunk_and_two_feet()
    nworld = 4
    lq, lv, rq, rv = model.q_offsets[1], model.v_offsets[1], model.q_offsets[2], model.v_offsets[2]
    sole = lambda k: (k, [0.01, 0.0, -0.04])
    sup = [sole(1), sole(2)]
    obs = [P.BodyPos(0, 0), P.BodyPos(0, 1), P.BodyPos(2, 0), P.ComOverSupport(sup, 0, 0), P.ComOverSupport(sup, 0, 1),
           P.ComOverSupport(sup, 0, 2), P.ComOverSupport(sup, None, 0), P.ComOverSupport([sole(1)], None, 1), P.V(0),
           P.QMinus(lq, 0.0)]
    sim = BatchSim(model, nworld, "f32")
    sim.enable_pd_control([PdDof(lq, lv, 20.0, 1.0, 10.0), PdDof(rq, rv, 20.0, 1.0, 10.0)])
    spec = P.PolicySpec(obs=obs, hidden=8, act_slots=[0, 1], act_clamp=0.3, input_noise=[0.0] * len(obs),
                        history_steps=2)
    sim.enable_policy(spec)
    wr = PR.KernelRng(0xB0A7)
    sim.set_policy_weights([0.2 * wr.normal() for _ in range(spec.n_weights())])
    sim.set_policy_std([0.1, 0.1])
    sim.set_policy_base_targets(np.zeros((nworld, 2)))
    sim.seed_policy(7)
    q = np.zeros((nworld, model.nq))
    v = np.zeros((nworld, model.nv))
    for w in range(nworld):
        q[w, 2] = {1: math.pi / 2, 2: 0.4, 3: -1.2}.get(w, 0.0)
        q[w, 0], q[w, 1], q[w, 3], q[w, 5] = 0.15 * w, -0.05 * w, 0.3 * w, 1.0
        q[w, lq], q[w, rq] = 0.2 - 0.1 * w, -0.15 + 0.05 * w
        v[w, lv] = 0.4
    sim.load_states(q, v)
    orc = Oracle(model)
    for step in range(2):
        sim.run_policy(step)
        dq, dv = sim.readback_states()
        obs_h, _ = sim.readback_policy_history(step, step + 1)
        for w in range(nworld):
            want = PR.observe_reference(model, orc, dq[w], dv[w], obs)
            d = np.abs(obs_h[0, w] - want).max()
            assert d < 1e-5, f"step {step} world {w}: {obs_h[0, w]} vs {want}"
            assert np.abs(obs_h[0, w, 3:6]).sum() > 1e-4
        sim.step_many(5)


def ant_policy_setup(hidden, nworld, prec="f32", n_in_extra=0, n_out=8, history=2):
    w = W.config(3)
    m = w.model
    pd = [PdDof(6 + k, 6 + k, 20.0, 1.0, 10.0) for k in range(8)]
    obs = ([P.BodyPitch(0), P.BodyRoll(0), P.BodyYawError(0, 0.1), P.BodyPosZ(0), P.BodyPos(0, 0)]
           + [P.QMinus(i, 0.05 * i) for i in range(6, 14)] + [P.V(i) for i in range(14)]
           + [P.ComOverSupport([(2, [0.0, 0.0, -0.1]), (4, [0.0, 0.0, -0.1])], 0, a % 3) for a in range(n_in_extra)])
    slots = [k % 8 for k in range(n_out)]
    spec = P.PolicySpec(obs=obs, hidden=hidden, act_slots=slots, act_clamp=0.5, noise_rho=0.4,
                        input_noise=[0.02 if i % 3 == 0 else 0.0 for i in range(len(obs))], history_steps=history)
    sim = BatchSim(m, nworld, prec)
    sim.enable_ground_contact(0.0, 1e4, 100.0, 1.0)
    sim.enable_pd_control(pd)
    sim.enable_policy(spec)
    rng = np.random.default_rng(hidden + nworld)
    n_in = spec.n_in()
    parts = [rng.normal(size=hidden * n_in) / math.sqrt(n_in), 0.1 * rng.normal(size=hidden),
             rng.normal(size=hidden * hidden) / math.sqrt(hidden), 0.1 * rng.normal(size=hidden),
             rng.normal(size=n_out * hidden) / math.sqrt(hidden), 0.1 * rng.normal(size=n_out)]
    weights = np.concatenate(parts)
    std = 0.1 + 0.05 * np.arange(n_out)
    base = rng.uniform(-0.2, 0.2, size=(nworld, 8))
    sim.set_policy_weights(weights)
    sim.set_policy_std(std)
    sim.set_policy_base_targets(base)
    sim.seed_policy(123)
    q, v, _, _ = w.initial_state(nworld)
    sim.load_states(q, v)
    return m, sim, spec, weights, std, base


@pytest.mark.parametrize("hidden,nworld,extra,n_out", [(256, 300, 0, 8), (100, 130, 3, 20), (64, 64, 0, 32), (16, 37, 1, 1)])
def test_policy_tiles_match_cpu(hidden, nworld, extra, n_out):
    """Full and ragged widths (hidden not a multiple of 16, n_in not a multiple of
    4, two output blocks) and partial world tiles."""
    m, sim, spec, weights, std, base = ant_policy_setup(hidden, nworld, n_in_extra=extra, n_out=n_out)
    orc = Oracle(m)
    rngs = [PR.KernelRng.for_world(123, w) for w in range(nworld)]
    zs = [np.zeros(n_out) for _ in range(nworld)]
    info = sim.control_kernel_info("policy")
    for step in range(2):
        sim.run_policy(step)
        q, v = sim.readback_states()
        o, a, lp, tg = cpu_policy_step(m, orc, spec, weights, std, rngs, zs, base, q, v)
        obs_h, out_h = sim.readback_policy_history(step, step + 1)
        do = np.abs(obs_h[0] - o).max()
        da = np.abs(out_h[0, :, :n_out] - a).max()
        dl = np.abs(out_h[0, :, n_out] - lp).max()
        dt = np.abs(sim.readback_targets() - tg).max()
        print(f"H {hidden} worlds {nworld} step {step} ({info['worlds_per_block']} worlds/wave): "
              f"obs {do:.2e} act {da:.2e} logp {dl:.2e} targets {dt:.2e}", flush=True)
        assert do < 1e-4 and da < 2e-4 and dl < 1e-3 and dt < 2e-4
        sim.step_many(3)


def test_rollout_is_the_manual_sequence():
    """phz_rollout (captured) == run_policy; step_many; record_state by hand, bit for bit."""
    outs = []
    for mode in ("manual", "rollout", "rollout_nograph"):
        m, sim, spec, *_ = ant_policy_setup(32, 200, history=4)
        sim.enable_state_history(4)
        if mode == "manual":
            for c in range(4):
                sim.run_policy(c)
                sim.step_many(5)
                sim.record_state(c)
        else:
            sim.set_graphs_enabled(mode == "rollout")
            sim.rollout(0, 2, 5, True)
            sim.rollout(2, 2, 5, True)
        outs.append(sim.readback_policy_history(0, 4) + sim.readback_state_history(0, 4) + (sim.readback_targets(),))
    for o in outs[1:]:
        for x, y in zip(outs[0], o):
            assert np.array_equal(x, y)


def test_nan_world_stays_in_its_world():
    """Worlds are MFMA tile columns: a NaN state in one world leaves every other
    world's observations and actions unchanged."""
    res = []
    for poison in (False, True):
        m, sim, spec, *_ = ant_policy_setup(64, 100)
        if poison:
            q, v = sim.readback_states()
            q[17, 6] = np.nan
            sim.load_states(q, v)
        sim.run_policy(0)
        res.append(sim.readback_policy_history(0, 1))
    keep = np.ones(100, bool)
    keep[17] = False
    assert np.array_equal(res[0][0][:, keep], res[1][0][:, keep])
    assert np.array_equal(res[0][1][:, keep], res[1][1][:, keep])
    assert np.isnan(res[1][1][0, 17]).any()


def test_two_wave_policy_kernel_same_bits():
    """At 131072 worlds (4096 policy waves over 1024 SIMDs) the policy kernel
    is built for two resident waves per SIMD; the same build of the same
    source, so a rollout's observations, actions, log-probs, targets and
    states equal the one-wave kernel's (PHZ_TWO_WAVES=0) bit for bit."""
    import os
    from phyz_amd import workloads as W
    from phyz_amd.sim import from_control_loop
    cl = W.control_loop()
    n = 131072
    outs, infos = [], []
    for one_wave in (False, True):
        if one_wave:
            os.environ["PHZ_TWO_WAVES"] = "0"
        try:
            sim = from_control_loop(cl, "f32", nworld=n)
            q, v, _, _ = cl.base.initial_state(n)
            sim.load_states(q, v)
            sim.seed_policy(cl.seed)
            infos.append(sim.control_kernel_info("policy"))
            sim.rollout(0, 3, cl.control_every, True)
        finally:
            os.environ.pop("PHZ_TWO_WAVES", None)
        outs.append(sim.readback_policy_history(0, 3) + sim.readback_state_history(0, 3) + (sim.readback_targets(),))
        sim.close()
    print(f"policy kernels: {infos}", flush=True)
    assert infos[0]["scratch_bytes"] > 0 and infos[0]["vgpr"] + max(infos[0]["agpr"], 0) <= 256
    assert infos[1]["scratch_bytes"] == 0 and infos[1]["vgpr"] + infos[1]["agpr"] > 256
    for x, y in zip(outs[0], outs[1]):
        assert np.array_equal(x, y, equal_nan=True)

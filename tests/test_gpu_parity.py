"""HIP step kernel against the f64 oracle, through the C ABI (BatchSim).

Per-step parity follows the reference's GPU-vs-CPU suites
(crates/phyz-gpu/tests/cuda_vs_cpu.rs:183-397), held to qdd normwise
relative error <= 1e-10 per step on the f64 kernels and <= 1e-4 on the f32
kernels. Inputs are the workloads' seeded states, plus
states taken from an oracle rollout so that contact, PD saturation and fast
joints are exercised.
"""
import numpy as np
import pytest

from phyz_amd import workloads as W
from phyz_amd.sim import BatchSim, from_workload
from tests.helpers import abs_err_rows, as_precision, oracle_for, rel_err_rows

pytestmark = pytest.mark.gpu

TOL_QDD = {"f64": 1e-10, "f32": 1e-4}
CASES = [(1, "f64"), (2, "f64"), (2, "f32"), (3, "f32"), (4, "f32"), (4, "f64"), (5, "f64")]


def _states(w, orc, nworld, warm_steps):
    q, v, c, tg = w.initial_state(nworld)
    if warm_steps:
        rng = orc.rng_states(nworld)
        orc.step_batch(q, v, c, warm_steps, targets=tg, rng=rng, threads=8)
    return q, v, c, tg


def _cpu_step(orc, w, q0, v0, ctrl):
    """One oracle step from (q0, v0) with the controls the device applied."""
    n = q0.shape[0]
    qdd = np.zeros((n, w.model.nv))
    q1, v1 = np.zeros_like(q0), np.zeros_like(v0)
    rows = np.zeros((n, w.model.nbodies, 8))
    for k in range(n):
        ext = None
        if w.contact is not None:
            ext, rows[k] = orc.contact(q0[k], v0[k])
        qdd[k] = orc.aba(q0[k], v0[k], ctrl[k], ext)
        q1[k], v1[k] = orc.integrate(q0[k], v0[k], qdd[k])
    return qdd, q1, v1, rows


@pytest.mark.parametrize("cfg,prec", CASES)
@pytest.mark.parametrize("warm", [0, 300])
def test_step_parity(cfg, prec, warm):
    w = W.config(cfg)
    orc = oracle_for(w)
    nworld = 200  # not a multiple of the 64-lane wave: exercises the tail guard
    q, v, c, tg = _states(w, orc, nworld, warm)
    q, v, c = (as_precision(a, prec) for a in (q, v, c))
    sim = from_workload(w, prec, nworld=nworld)
    sim.load_states(q, v, c)
    if tg is not None:
        tg = as_precision(tg, prec)
        sim.set_position_targets(tg)
    sim.step()
    qg, vg = sim.readback_states()
    ctrl = sim.readback_controls()
    qdd = sim.readback_qdd()
    print(f"cfg {cfg} {prec} warm {warm}: kernel {sim.kernel_info()}", flush=True)

    # Controls the device applied: PD law and the control stream.
    if w.pd is not None:
        for d in w.pd:
            tau = np.clip(d.kp * (tg[:, d.q_index] - q[:, d.q_index]) - d.kd * v[:, d.v_index], -d.max_force, d.max_force)
            tol = 1e-12 if prec == "f64" else 1e-5
            assert np.allclose(ctrl[:, d.v_index], tau, rtol=tol, atol=tol * d.max_force)
    if w.noise is not None and prec == "f64" and warm == 0:
        # Replay of the per-world stream (oracle draws in f64 with 53-bit uniforms).
        rng = orc.rng_states(nworld)
        qc, vc, cc = q.copy(), v.copy(), c.copy()
        orc.step_batch(qc, vc, cc, 1, targets=tg, rng=rng, threads=8)
        np.testing.assert_allclose(ctrl[:, w.noise.dofs], cc[:, w.noise.dofs], rtol=1e-13, atol=1e-13)

    ctrl_in = as_precision(ctrl, prec)
    qdd_c, q1_c, v1_c, rows_c = _cpu_step(orc, w, q, v, ctrl_in)
    e = rel_err_rows(qdd, qdd_c)
    print(f"  qdd rel err max {e.max():.3e} median {np.median(e):.3e}", flush=True)
    assert np.all(np.isfinite(qdd))
    if prec == "f32" and w.contact is not None:
        # For scale: the same law evaluated wholly in f32 arithmetic (the
        # reference device's precision) on the same states.
        floor = np.array([rel_err_rows(orc.qdd_f32(q[k], v[k], ctrl_in[k]), qdd_c[k]) for k in range(nworld)])
        print(f"  all-f32 evaluation of the same states: max {floor.max():.3e}", flush=True)
    assert np.all(e <= TOL_QDD[prec]), f"qdd rel err {e.max():.3e} (world {e.argmax()})"
    scale_v = np.maximum(np.abs(v1_c).max(axis=1), 1.0)
    assert (abs_err_rows(vg, v1_c) / scale_v).max() <= 10 * TOL_QDD[prec]
    assert abs_err_rows(qg, q1_c).max() <= 10 * TOL_QDD[prec] * max(1.0, np.abs(q1_c).max())
    if w.contact is not None:
        rows = sim.readback_contacts()
        touching = rows_c[:, :, 0] > 0
        if warm:
            assert touching.any(), "warm state should be in contact"
        agree = (rows[:, :, 0] > 0) == touching
        assert agree.mean() > 0.99
        both = agree & touching
        if both.any():
            f_err = np.abs(rows[:, :, 5:8] - rows_c[:, :, 5:8]).max(axis=-1)[both]
            f_scale = np.maximum(np.abs(rows_c[:, :, 5:8]).max(axis=-1)[both], 1.0)
            print(f"  contact rows: {both.sum()} touching, force rel err {(f_err / f_scale).max():.3e}", flush=True)
            assert (f_err / f_scale).max() <= (1e-9 if prec == "f64" else 1e-3)


@pytest.mark.parametrize("prec", ["f64", "f32"])
def test_graph_replay_bit_identical(prec):
    """Graph replay equals direct launches bit for bit (cuda_vs_cpu.rs:1295-1378),
    and one 10-step span equals ten 1-step spans."""
    w = W.config(2)
    q, v, c, _ = w.initial_state(128)
    outs = []
    for graphs, chunks in ((True, [10]), (False, [10]), (False, [1] * 10), (True, [3, 7])):
        sim = from_workload(w, prec, nworld=128)
        sim.set_graphs_enabled(graphs)
        sim.load_states(q, v, c)
        for n in chunks:
            sim.step_many(n)
        outs.append(sim.readback_states())
    for o in outs[1:]:
        assert np.array_equal(o[0], outs[0][0]) and np.array_equal(o[1], outs[0][1])


def test_time_step_many_is_kernel_time():
    """phz_time_step_many reports each span's kernel time from events its
    launches stamp: positive, no longer than the same span's wall clock, and
    for a span of two launches (1500 steps, 1000 per launch) about the sum of
    its launches; a span of no steps is refused."""
    import time
    from phyz_amd.sim import PhzError
    w = W.config(2)
    q, v, c, _ = w.initial_state(4096)
    sim = from_workload(w, "f32", nworld=4096)
    sim.load_states(q, v, c)
    one = sim.time_step_many(500, 3)
    two = sim.time_step_many(1500, 2)
    sim.synchronize()
    t0 = time.perf_counter()
    sim.step_many(500)
    sim.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    print(f"500 steps: events {one} ms, wall {wall_ms:.3f} ms; 1500 steps: {two} ms", flush=True)
    assert np.all(one > 0) and np.all(two > 0)
    assert np.median(one) <= wall_ms * 1.05
    assert 2.0 * np.median(one) < np.median(two) < 4.0 * np.median(one)
    with pytest.raises(PhzError):
        sim.time_step_many(0, 1)


@pytest.mark.parametrize("cfg,prec", CASES + [(6, "f32"), (6, "f64")])
def test_repeat_launch_bit_identical(cfg, prec):
    """The same inputs stepped again give the same bits, every world: a kernel
    that picks up values left behind by an earlier launch fails this."""
    w = W.config(cfg)
    n = 4096
    q, v, c, tg = w.initial_state(n)
    sim = from_workload(w, prec, nworld=n)
    outs = []
    for _ in range(8):
        sim.load_states(q, v, c)
        if tg is not None:
            sim.set_position_targets(tg)
        sim.step()
        qdd, ctrl = sim.readback_qdd(), sim.readback_controls()
        bits = np.uint64 if qdd.dtype == np.float64 else np.uint32
        outs.append((qdd.view(bits), ctrl.view(bits)))
    for k, (qdd, ctrl) in enumerate(outs[1:], start=1):
        bad = ~(np.all(qdd == outs[0][0], axis=1) & np.all(ctrl == outs[0][1], axis=1))
        assert not bad.any(), f"cfg {cfg} {prec}: repeat {k} differs in {bad.sum()} worlds"


def test_worlds_independent_and_nan_isolated():
    """A NaN injected into one world stays in that world (no cross-world state)."""
    w = W.config(3)
    q, v, c, _ = w.initial_state(130)
    q[7, 6] = np.nan
    sim = from_workload(w, "f32", nworld=130)
    sim.load_states(q, v, c)
    sim.step_many(20)
    qg, vg = sim.readback_states()
    bad = ~np.isfinite(qg).all(axis=1) | ~np.isfinite(vg).all(axis=1)
    assert bad[7]
    assert not bad[np.arange(130) != 7].any()


@pytest.mark.parametrize("cfg,prec", [(4, "f64"), (5, "f64"), (7, "f64"), (8, "f64"), (9, "f64"), (8, "f32"), (9, "f32")])
def test_repeat_span_bit_identical(cfg, prec):
    """Spans of many steps per launch, repeated from the same state, give the
    same bits in every world: the partitioned kernels (and the MJCF f64 ones,
    which spill registers to scratch) hold no state across steps or launches
    beyond what the span carries."""
    w = W.config(cfg)
    n = 2048
    q, v, c, tg = w.initial_state(n)
    sim = from_workload(w, prec, nworld=n)
    print(f"cfg {cfg} {prec}: kernel {sim.kernel_info()}", flush=True)
    outs = []
    for _ in range(4):
        sim.load_states(q, v, c)
        if tg is not None:
            sim.set_position_targets(tg)
        sim.step_many(200)
        qg, vg = sim.readback_states()
        bits = np.uint64 if qg.dtype == np.float64 else np.uint32
        outs.append((qg.view(bits).copy(), vg.view(bits).copy()))
    for k, (qg, vg) in enumerate(outs[1:], start=1):
        bad = ~(np.all(qg == outs[0][0], axis=1) & np.all(vg == outs[0][1], axis=1))
        assert not bad.any(), f"cfg {cfg} {prec}: repeat {k} differs in {bad.sum()} worlds"

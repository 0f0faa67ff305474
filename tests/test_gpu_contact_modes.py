"""Heightfield terrain, body-attached plane and impulse-mode contact on the
device against the oracle (whose agreement with the reference's own contact
pass is pinned in tests/test_oracle_contact_modes.py).

Per step: qdd, the carried contact forces and the warm-start impulses, from
the same states. Over several steps (several launches, graph replay on and
off): the state and the contact state. f64 kernels are held to 1e-10 (one
step) and 1e-8 (rollouts). f32 kernels to 1e-4 per step in every mode (qdd,
and the carried impulses and forces relative to their largest): they decide
every contact's activation (the ground's and terrain's depth and cell, the
body-attached plane's depth range and footprint) from an f64 chain of the
contact path's world frames, as the f64 oracle decides it, and apply the law
in f32 where it is continuous.
"""
import dataclasses

import numpy as np
import pytest

from oracle.oracle import ContactCfg, Oracle
from phyz_amd import workloads as W
from phyz_amd.model import BodyPlane, Heightfield, pack_geometries, uniform_frequency_gains
from phyz_amd.sim import BatchSim, PhzError
from tests import models as TM
from tests.helpers import as_precision, rel_err_rows

pytestmark = pytest.mark.gpu

HF = TM.bumpy_heightfield()


def hf_obj(t=HF):
    nx, ny, ox, oy, oz, cell, h = t
    return Heightfield(origin=(ox, oy, oz), cell=cell, nx=nx, ny=ny, heights=np.asarray(h).reshape(ny, nx))


def setup(model, mode, plane=None, hf=None, mu=0.8, omega=50.0, sweeps=16):
    gains = uniform_frequency_gains(model, omega, 1.0)
    geom, _ = pack_geometries(model, gains=gains)
    if plane is not None:
        geom[plane.body, 7] = 1.0
        for b in plane.exclude:
            geom[b, 7] = 1.0
    erp = model.dt / (0.04 + model.dt) if mode == 1 else 0.001 / 0.041
    cfg = ContactCfg(solve_mode=mode, sweeps=sweeps, erp=erp,
                     plane=None if plane is None else (plane.body, plane.offset, plane.max_depth, plane.half_x, plane.half_y),
                     heightfield=hf)
    orc = Oracle(model, contact=(geom, 0.0, mu), contact_cfg=cfg)
    return gains, orc


def make_sim(model, prec, n, mode, gains, plane=None, hf=None, mu=0.8, sweeps=16):
    s = BatchSim(model, n, prec)
    if mode == 1:
        s.enable_contact_impulse(0.0, mu, gains, plane, None if hf is None else hf_obj(hf))
        s.contact_sweeps = sweeps
    else:
        s.enable_contact_terrain(0.0, mu, gains, plane, None if hf is None else hf_obj(hf))
    return s


def settled(model, orc, n, steps, seed, xy=0.0, z=(0.15, 0.3)):
    rng = np.random.default_rng(seed)
    q = np.zeros((n, model.nq))
    v = rng.normal(size=(n, model.nv)) * 0.3
    for i, b in enumerate(model.bodies):
        if b.joint.jtype == 4:
            o = model.q_offsets[i]
            q[:, o:o + 3] = rng.normal(size=(n, 3)) * 0.5
            q[:, o + 3:o + 5] = rng.uniform(-xy, xy, size=(n, 2))
            q[:, o + 5] = rng.uniform(*z, size=n)
    c = np.zeros((n, model.nv))
    ext = np.zeros((n, model.nbodies, 6))
    cs = np.zeros((n, model.nbodies, 56))
    orc.step_batch(q, v, c, steps, threads=8, ext_state=ext, cs_state=cs)
    return q, v, c, ext, cs


def deck_states(model, orc, n, seed):
    rng = np.random.default_rng(seed)
    q = np.zeros((n, model.nq))
    q[:, 5] = 0.02
    for o, z in ((6, 0.09), (12, 0.06)):
        q[:, o:o + 3] = rng.normal(size=(n, 3)) * 0.2
        q[:, o + 3] = rng.uniform(-0.3, 0.3, size=n)
        q[:, o + 4] = rng.uniform(-0.05, 0.05, size=n)
        q[:, o + 5] = z
    v = rng.normal(size=(n, model.nv)) * 0.1
    c = np.zeros((n, model.nv))
    ext = np.zeros((n, 3, 6))
    cs = np.zeros((n, 3, 56))
    orc.step_batch(q, v, c, 150, threads=8, ext_state=ext, cs_state=cs)
    return q, v, c, ext, cs


def cases():
    out = []
    for name in ("sphere", "box", "capsule"):
        for mode in (0, 1):
            for terr in ("flat", "hf"):
                if mode == 0 and terr == "flat":
                    continue
                out.append((f"{'impulse' if mode else 'penalty'}_{terr}_{name}", name, mode, terr))
    out += [("penalty_plane_deck", "deck", 0, "flat"), ("impulse_plane_deck", "deck", 1, "flat"),
            ("impulse_flat_ant", "ant", 1, "flat")]
    return out


def build_case(kind, mode, terr, n):
    hf = HF if terr == "hf" else None
    plane = None
    if kind == "deck":
        m = TM.deck_and_feet()
        plane = BodyPlane(*TM.DECK_PLANE)
    elif kind == "ant":
        m = W.config(3).model
    else:
        m = TM.shapes()[kind]
    gains, orc = setup(m, mode, plane, hf, mu=1.0 if kind == "ant" else 0.8, omega=60.0 if kind == "ant" else 50.0)
    if kind == "deck":
        st = deck_states(m, orc, n, seed=3 + mode)
    elif kind == "ant":
        w = W.config(3)
        q, v, c, _ = w.initial_state(n)
        ext = np.zeros((n, 9, 6))
        cs = np.zeros((n, 9, 56))
        orc.step_batch(q, v, c, 300, threads=8, ext_state=ext, cs_state=cs)
        st = (q, v, c, ext, cs)
    else:
        st = settled(m, orc, n, 300, seed=len(kind) + 10 * mode, xy=0.8 if hf is not None else 0.0)
    return m, gains, orc, plane, hf, st


@pytest.mark.parametrize("prec", ["f64", "f32"])
@pytest.mark.parametrize("name,kind,mode,terr", cases())
def test_contact_mode_matches_oracle(name, kind, mode, terr, prec):
    n = 70
    m, gains, orc, plane, hf, (q, v, c, ext, cs) = build_case(kind, mode, terr, n)
    q, v = as_precision(q, prec), as_precision(v, prec)
    ext, cs = as_precision(ext, prec), as_precision(cs, prec)
    s = make_sim(m, prec, n, mode, gains, plane, hf, mu=1.0 if kind == "ant" else 0.8)
    s.load_states(q, v, c)
    if mode == 1:
        s.load_contact_state(cs, ext)
    # One device step against one oracle step from the same state.
    s.step()
    qdd = s.readback_qdd()
    dcs, dext = s.readback_contact_state()
    q1, v1, c1 = q.copy(), v.copy(), c.copy()
    e1, s1 = ext.copy(), cs.copy()
    want_qdd, rows = orc.step_batch(q1, v1, c1, 1, threads=8, want_contacts=True, ext_state=e1, cs_state=s1)
    err = rel_err_rows(qdd, want_qdd).max()
    tol = 1e-10 if prec == "f64" else 1e-4
    print(f"{name} {prec}: qdd {err:.2e}", flush=True)
    assert err <= tol
    touch = dcs[:, :, 0] > 0
    assert np.mean(touch == (rows[:, :, 0] > 0)) >= (1.0 if prec == "f64" else 0.98)
    if mode == 1:
        iscale = max(np.abs(s1[:, :, 8:]).max(), 1e-6)
        ierr = np.abs(dcs[:, :, 8:] - s1[:, :, 8:]).max() / iscale
        escale = max(np.abs(e1).max(), 1.0)
        eerr = np.abs(dext - e1).max() / escale
        print(f"   impulses {ierr:.2e} forces {eerr:.2e}", flush=True)
        assert ierr <= (1e-9 if prec == "f64" else 1e-4) and eerr <= (1e-9 if prec == "f64" else 1e-4)
    # Several launches (graph replay) against the oracle's rollout.
    s.step_many(5)
    s.step_many(5)
    qd, vd = s.readback_states()
    orc.step_batch(q1, v1, c1, 10, threads=8, ext_state=e1, cs_state=s1)
    dq = np.abs(qd - q1).max()
    dv = np.abs(vd - v1).max() / max(1.0, np.abs(v1).max())
    print(f"   11-step state: q {dq:.2e} v {dv:.2e}", flush=True)
    if prec == "f64":
        assert dq <= 1e-8 and dv <= 1e-8
    else:
        assert dq <= 1e-4 and dv <= 1e-3


def test_graph_replay_and_launch_splits_are_bit_identical_in_impulse_mode():
    """The solver state crosses launch boundaries exactly: one 12-step span,
    12 single steps, and spans of 5 + 7 with graphs off agree bit for bit."""
    m, gains, orc, plane, hf, (q, v, c, ext, cs) = build_case("box", 1, "hf", 64)
    outs = []
    for how in ("span", "single", "split_nograph"):
        s = make_sim(m, "f32", 64, 1, gains, plane, hf)
        s.load_states(q, v, c)
        s.load_contact_state(cs, ext)
        if how == "span":
            s.step_many(12)
        elif how == "single":
            for _ in range(12):
                s.step()
        else:
            s.set_graphs_enabled(False)
            s.step_many(5)
            s.step_many(7)
        outs.append(s.readback_states() + s.readback_contact_state())
    for o in outs[1:]:
        for a, b in zip(outs[0], o):
            assert np.array_equal(a, b)


def test_set_heightfield_and_sweeps():
    """New terrain in place (same node count, shifted heights), and a sweep count of 4."""
    m = TM.shapes()["sphere"]
    hf2 = list(HF)
    hf2[6] = np.asarray(HF[6] * 0.5 + 0.02, dtype=np.float32).astype(np.float64)
    hf2 = tuple(hf2)
    gains, orc = setup(m, 1, None, hf2, sweeps=4)
    q, v, c, ext, cs = settled(m, orc, 40, 200, seed=9, xy=0.8)
    s = make_sim(m, "f64", 40, 1, gains, None, HF, sweeps=4)
    assert s.contact_sweeps == 4
    s.set_heightfield(hf_obj(hf2))
    s.load_states(q, v, c)
    s.load_contact_state(cs, ext)
    s.step_many(3)
    qd, vd = s.readback_states()
    orc.step_batch(q, v, c, 3, threads=8, ext_state=ext, cs_state=cs)
    assert np.abs(qd - q).max() <= 1e-9 and np.abs(vd - v).max() <= 1e-8
    bigger = Heightfield(origin=(0, 0, 0), cell=0.1, nx=20, ny=20, heights=np.zeros((20, 20)))
    with pytest.raises(PhzError, match="buffer was sized for 81"):
        s.set_heightfield(bigger)
    s.contact_sweeps = 0
    with pytest.raises(PhzError, match="at least one contact sweep"):
        s.step()


@pytest.mark.parametrize("prec", ["f64", "f32"])
@pytest.mark.parametrize("kind", ["box", "ant"])
def test_impulse_sweep_counts(kind, prec):
    """Every sweep count from 1 to 16 matches the oracle's sweeps one step ahead
    (f64 to 1e-10; a wrong count or a stale sweep shows as a percent-level gap)."""
    n = 70
    m, gains, orc, plane, hf, (q, v, c, ext, cs) = build_case(kind, 1, "flat", n)
    q, v = as_precision(q, prec), as_precision(v, prec)
    ext, cs = as_precision(ext, prec), as_precision(cs, prec)
    from oracle import oracle as O
    for sweeps in (1, 2, 3, 4, 5, 8, 16):
        orc.cfg.sweeps = sweeps
        orc.cfg.apply(O.lib(), orc._h)
        s = make_sim(m, prec, n, 1, gains, mu=1.0 if kind == "ant" else 0.8, sweeps=sweeps)
        s.load_states(q, v, c)
        s.load_contact_state(cs, ext)
        s.step()
        qdd = s.readback_qdd()
        dcs, _ = s.readback_contact_state()
        e1, s1 = ext.copy(), cs.copy()
        want, _ = orc.step_batch(q.copy(), v.copy(), c.copy(), 1, threads=8, ext_state=e1, cs_state=s1)
        err = rel_err_rows(qdd, want).max()
        ierr = np.abs(dcs[:, :, 8:] - s1[:, :, 8:]).max() / max(np.abs(s1[:, :, 8:]).max(), 1e-6)
        print(f"{kind} {prec} sweeps {sweeps}: qdd {err:.2e} impulses {ierr:.2e}", flush=True)
        assert err <= (1e-10 if prec == "f64" else 1e-4)
        assert ierr <= (1e-9 if prec == "f64" else 1e-4)


@pytest.mark.parametrize("prec", ["f64", "f32"])
def test_terrain_impulse_workload(prec):
    """The benchmark's terrain + impulse workload (ant, rolling heightfield, 16
    sweeps, control noise) configured through from_workload, at 256 worlds:
    250 device steps (noise stream replayed exactly by the oracle; the ants
    drop from 0.5-1 m and land) from the seeded initial states, then one more step against the oracle from the
    device's own state, carried contact forces and warm-start impulses."""
    from phyz_amd.sim import from_workload
    from tests.helpers import oracle_for
    w = W.config(6)
    n = 256
    orc = oracle_for(w)
    q, v, c, _ = w.initial_state(n)
    q, v = as_precision(q, prec), as_precision(v, prec)
    sim = from_workload(w, prec, nworld=n)
    assert sim.contact_sweeps == 16
    sim.load_states(q, v, c)
    sim.step_many(250)
    qd, vd = sim.readback_states()
    dcs, dext = sim.readback_contact_state()
    ext, cs = np.zeros((n, 9, 6)), np.zeros((n, 9, 56))
    rng = orc.rng_states(n)
    orc.step_batch(q, v, c, 250, rng=rng, threads=8, ext_state=ext, cs_state=cs)
    touching = (dcs[:, :, 0] > 0).sum()
    dq = np.abs(qd - q).max()
    print(f"{prec}: 250 steps, {touching} feet touching, state q {dq:.2e}", flush=True)
    assert touching > n  # most worlds have feet on the terrain
    if prec == "f64":
        assert dq <= 1e-8 and np.abs(vd - v).max() <= 1e-7 * max(1.0, np.abs(v).max())
    # One step from the device's state with the device's noisy torques.
    orc0 = oracle_for(dataclasses.replace(w, noise=None))
    sim.step()
    ctrl = as_precision(sim.readback_controls(), prec)
    qdd = sim.readback_qdd()
    cs1, ext1 = sim.readback_contact_state()
    e0, s0 = np.ascontiguousarray(dext), np.ascontiguousarray(dcs)
    want, _ = orc0.step_batch(qd.copy(), vd.copy(), ctrl, 1, threads=8, ext_state=e0, cs_state=s0)
    err = rel_err_rows(qdd, want).max()
    ierr = np.abs(cs1[:, :, 8:] - s0[:, :, 8:]).max() / max(np.abs(s0[:, :, 8:]).max(), 1e-6)
    eerr = np.abs(ext1 - e0).max() / max(np.abs(e0).max(), 1.0)
    print(f"   one step: qdd {err:.2e} impulses {ierr:.2e} forces {eerr:.2e}", flush=True)
    assert err <= (1e-10 if prec == "f64" else 1e-4)
    assert ierr <= (1e-9 if prec == "f64" else 1e-4) and eerr <= (1e-9 if prec == "f64" else 1e-4)

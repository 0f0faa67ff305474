"""The oracle's heightfield terrain, body-attached plane and impulse-mode contact.

1. Against the reference's own contact pass and impulse sweeps
   (crates/phyz-gpu/cuda/phyz_kernels.cu:804-1132 and the sequencing of
   crates/phyz-gpu/src/cuda/mod.rs:899-928, compiled as host C++ and run in f32;
   tests/golden/make_ref_contact_modes.py): qdd, state, external forces and the
   warm-start impulses agree to f32 rounding.
2. Properties the golden vectors do not fix: a constant heightfield is the flat
   ground; a planar heightfield gives the plane's normal and depth; plane
   contacts act equally and oppositely on both bodies; an impulse-mode box
   rests without sinking and carries its weight; Coulomb sliding decelerates at
   mu g.
"""
import os

import numpy as np
import pytest

from oracle.oracle import ContactCfg, Oracle
from phyz_amd.model import pack_geometries, uniform_frequency_gains
from tests import models as TM
from tests.helpers import rel_err_rows

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_contact_modes.npz")
Z = np.load(GOLDEN)
NAMES = sorted({k.split("/")[0] for k in Z.files})


def cfg_from(g):
    mode, sweeps = (int(x) for x in g["mode"])
    plane = None if g["plane"][0] < 0 else (int(g["plane"][0]), *g["plane"][1:])
    hf = None
    if g["hf"][0] > 0:
        nx, ny, ox, oy, oz, cell = g["hf"]
        hf = (int(nx), int(ny), ox, oy, oz, cell, g["hf_heights"])
    p = g["prm"]
    return ContactCfg(solve_mode=mode, sweeps=sweeps, restitution=p[0], restitution_threshold=p[1], erp=p[2],
                      margin=p[3], solimp=tuple(p[4:9]), plane=plane, heightfield=hf)


def load_case(name):
    g = {k.split("/")[1]: Z[k] for k in Z.files if k.startswith(name + "/")}
    nb, nq, nv, steps = (int(x) for x in g["dims"])
    orc = Oracle(tables=(g["table"], nq, nv, g["gravity"], float(g["dt"][0])), contact=(g["geom"], 0.0, float(g["mu"][0])),
                 contact_cfg=cfg_from(g))
    return g, orc, nb, steps


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_reference_contact_modes(name):
    g, orc, nb, steps = load_case(name)
    q, v, c = g["q0"].copy(), g["v0"].copy(), g["ctrl0"].copy()
    n = q.shape[0]
    ext = np.zeros((n, nb, 6))
    cs = np.zeros((n, nb, 56))
    qdd, rows = orc.step_batch(q, v, c, steps, threads=1, want_contacts=True, ext_state=ext, cs_state=cs)
    err = rel_err_rows(g["qdd"], qdd).max()
    assert err <= 2e-4, f"{name}: qdd {err:.2e}"
    assert np.abs(v - g["v"]).max() <= 2e-5 * max(1.0, np.abs(g["v"]).max())
    assert np.abs(q - g["q"]).max() <= 5e-6
    escale = max(np.abs(g["ext"]).max(), 1.0)
    assert np.abs(ext - g["ext"]).max() <= 2e-4 * escale
    if int(g["mode"][0]) == 1:
        iscale = max(np.abs(g["cs"][:, :, 8:]).max(), 1e-6)
        assert np.abs(cs[:, :, 8:] - g["cs"][:, :, 8:]).max() <= 2e-4 * iscale
    touch_ref = g["cs"][:, :, 0] > 0
    touch = rows[:, :, 0] > 0
    assert np.mean(touch == touch_ref) >= 0.98 and touch_ref.any()
    if "plane" in name:
        # The feet are on the deck: plane forces act on them.
        assert np.abs(g["ext"][:, 1:, :]).max() > 0.1


def sphere_model():
    return TM.shapes()["sphere"]


def contact_oracle(m, cfg, ground_h=0.0, mu=0.8):
    geom, _ = pack_geometries(m, gains=uniform_frequency_gains(m, 50.0, 1.0))
    if cfg.plane is not None:
        geom[cfg.plane[0], 7] = 1.0
    return Oracle(m, contact=(geom, ground_h, mu), contact_cfg=cfg)


def test_constant_heightfield_is_flat_ground():
    """A heightfield of constant height h is the flat ground at h, bit for bit."""
    m = sphere_model()
    h0 = 0.037
    hf = (5, 4, -1.0, -1.0, 0.01, 0.5, np.full(20, h0 - 0.01))
    rng = np.random.default_rng(1)
    for mode in (0, 1):
        flat = contact_oracle(m, ContactCfg(solve_mode=mode), ground_h=h0)
        terr = contact_oracle(m, ContactCfg(solve_mode=mode, heightfield=hf), ground_h=5.0)
        for _ in range(5):
            q = np.zeros(m.nq)
            q[0:3] = rng.normal(size=3)
            q[3:5] = rng.uniform(-0.5, 0.5, size=2)
            q[5] = h0 + 0.09
            v = rng.normal(size=m.nv)
            cs_a, cs_b = np.zeros(56 * m.nbodies), np.zeros(56 * m.nbodies)
            a = flat.contact_pass(q, v, cs_a)
            b = terr.contact_pass(q, v, cs_b)
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]) and np.array_equal(cs_a, cs_b)
            assert a[1][0, 0] == 1.0


@pytest.mark.parametrize("slope", [0.0, 0.2, -0.35])
def test_planar_heightfield_normal_and_depth(slope):
    """h = slope x + 0.02 y: a sphere over it touches at its lowest point with
    depth n_z (h - z_low), n = normalize(-slope, -0.02, 1)."""
    m = sphere_model()
    xs = np.arange(6) * 0.4 - 1.0
    ys = np.arange(6) * 0.4 - 1.0
    h = slope * xs[None, :] + 0.02 * ys[:, None]
    hf = (6, 6, -1.0, -1.0, 0.0, 0.4, h)
    orc = contact_oracle(m, ContactCfg(heightfield=hf))
    q = np.zeros(m.nq)
    q[3], q[4] = 0.13, -0.21
    h_c = slope * 0.13 + 0.02 * -0.21
    geom, _ = pack_geometries(m)
    radius = geom[0, 1]
    q[5] = h_c + radius - 0.004
    ext, rows = orc.contact_pass(q, np.zeros(m.nv))
    n = np.array([-slope, -0.02, 1.0])
    n /= np.linalg.norm(n)
    assert rows[0, 0] == 1.0
    assert rows[0, 1] == pytest.approx(n[2] * 0.004, abs=1e-12)
    # Force along the terrain normal (no tangential velocity).
    f = rows[0, 5:8]
    np.testing.assert_allclose(f / np.linalg.norm(f), n, atol=1e-12)


def test_plane_contact_is_action_and_reaction():
    """Deck far above the ground: plane contacts only; equal and opposite forces
    on foot and deck at one point (world force and moment sums vanish)."""
    m = TM.deck_and_feet()
    for mode in (0, 1):
        orc = contact_oracle(m, ContactCfg(solve_mode=mode, plane=TM.DECK_PLANE), ground_h=-10.0)
        q = np.zeros(m.nq)
        q[0:3] = [0.02, -0.01, 0.2]
        q[5] = 1.0  # deck centre; its top face is at z = 1.02 (tilted slightly)
        q[6:12] = [0.1, 0.2, 0.0, 0.1, 0.0, 1.02 + 0.05 - 0.006]
        q[12:18] = [0.0, 0.0, 0.3, -0.15, 0.02, 1.02 + 0.02 - 0.006]
        v = np.random.default_rng(2).normal(size=m.nv) * 0.1
        fk = orc.fk(q, v)
        ext, rows = orc.contact_pass(q, v, np.zeros(56 * 3))
        F = np.zeros(3)
        Mo = np.zeros(3)
        for i in range(3):
            R = fk[i, 0:9].reshape(3, 3)  # body -> world
            p = fk[i, 9:12]
            fw = R @ ext[i, 3:6]
            tw = R @ ext[i, 0:3] + np.cross(p, fw)
            F += fw
            Mo += tw
        assert np.abs(ext[1:]).max() > 1.0, "feet must be pressed into the deck"
        assert np.abs(F).max() <= 1e-9 * np.abs(ext).max()
        assert np.abs(Mo).max() <= 1e-9 * np.abs(ext).max()
        assert rows[:, 0].sum() == 0.0  # plane contacts are not in the readback rows


def test_impulse_box_rests_without_sinking_and_carries_its_weight():
    m = TM.shapes()["box"]
    geom, _ = pack_geometries(m, gains=uniform_frequency_gains(m, 50.0, 1.0))
    orc = Oracle(m, contact=(geom, 0.0, 0.8), contact_cfg=ContactCfg(solve_mode=1, erp=m.dt / (0.04 + m.dt)))
    hz = geom[0, 3]
    q = np.zeros((1, m.nq))
    q[0, 5] = hz + 0.01
    v = np.zeros((1, m.nv))
    c = np.zeros((1, m.nv))
    ext, cs = np.zeros((1, 1, 6)), np.zeros((1, 1, 56))
    _, rows = orc.step_batch(q, v, c, 3000, want_contacts=True, ext_state=ext, cs_state=cs)
    mass = m.bodies[0].inertia.mass
    assert abs(q[0, 5] - hz) < 2e-3            # no m g / k sink
    assert np.abs(v).max() < 1e-3
    assert rows[0, 0, 7] == pytest.approx(mass * 9.81, rel=1e-3)


def test_impulse_sliding_box_decelerates_at_mu_g():
    m = TM.shapes()["box"]
    geom, _ = pack_geometries(m, gains=uniform_frequency_gains(m, 50.0, 1.0))
    mu = 0.5
    orc = Oracle(m, contact=(geom, 0.0, mu), contact_cfg=ContactCfg(solve_mode=1, erp=m.dt / (0.04 + m.dt)))
    hz = geom[0, 3]
    q = np.zeros((1, m.nq))
    q[0, 5] = hz
    v = np.zeros((1, m.nv))
    c = np.zeros((1, m.nv))
    ext, cs = np.zeros((1, 1, 6)), np.zeros((1, 1, 56))
    orc.step_batch(q, v, c, 300, ext_state=ext, cs_state=cs)  # settle
    v[0, 3] = 1.5
    v0 = v[0, 3]
    orc.step_batch(q, v, c, 100, ext_state=ext, cs_state=cs)
    decel = (v0 - v[0, 3]) / (100 * m.dt)
    assert decel == pytest.approx(mu * 9.81, rel=0.02)


@pytest.mark.parametrize("case", ["box_hf", "trunk_plane"])
def test_split_impulse_step_equals_full_solves(case):
    """The kernels' impulse step (one factorization, per sweep only the
    velocities at v + dt qdd and the force-dependent half of the ABA) against
    full solves every sweep by CRBA + Cholesky: the ABA is linear in the
    external forces, so the two agree to f64 rounding over many steps."""
    if case == "box_hf":
        m = TM.shapes()["box"]
        cfg = ContactCfg(solve_mode=1, sweeps=6, erp=m.dt / (0.04 + m.dt), heightfield=TM.bumpy_heightfield())
        geom, _ = pack_geometries(m, gains=uniform_frequency_gains(m, 50.0, 1.0))
        hz = geom[0, 3]
        q0 = np.zeros((3, m.nq))
        q0[:, 0:3] = [[0.0, 0.0, 0.0], [0.1, -0.2, 0.3], [0.4, 0.1, -0.1]]
        q0[:, 3:5] = [[0.0, 0.0], [0.3, -0.2], [-0.4, 0.35]]
        q0[:, 5] = hz + 0.02
    else:
        m = TM.deck_and_feet()
        cfg = ContactCfg(solve_mode=1, sweeps=4, erp=m.dt / (0.04 + m.dt), plane=TM.DECK_PLANE)
        geom, _ = pack_geometries(m, gains=uniform_frequency_gains(m, 50.0, 1.0))
        geom[TM.DECK_PLANE[0], 7] = 1.0
        q0 = np.zeros((2, m.nq))
        q0[:, 5] = 0.05
        q0[:, 6:12] = [0.1, 0.2, 0.0, 0.1, 0.0, 0.07 + 0.05 - 0.004]
        q0[:, 12:18] = [0.0, 0.0, 0.3, -0.15, 0.02, 0.07 + 0.02 - 0.004]
        q0[1, 3] = 0.01
    orc = Oracle(m, contact=(geom, 0.0, 0.8), contact_cfg=cfg)
    rng = np.random.default_rng(4)
    n = q0.shape[0]
    v0 = rng.normal(size=(n, m.nv)) * 0.2
    c0 = rng.normal(size=(n, m.nv)) * 0.5
    out = []
    for dense in (False, True):
        q, v, c = q0.copy(), v0.copy(), c0.copy()
        ext, cs = np.zeros((n, m.nbodies, 6)), np.zeros((n, m.nbodies, 56))
        qdd, _ = orc.step_batch(q, v, c, 60, dense=dense, ext_state=ext, cs_state=cs)
        out.append((q, v, qdd, ext, cs))
    (qa, va, da, ea, ca), (qb, vb, db, eb, cb) = out
    assert np.abs(ea).max() > 1.0, "the bodies must be in contact"
    assert np.abs(qa - qb).max() <= 1e-10
    assert np.abs(va - vb).max() <= 1e-8 * max(1.0, np.abs(vb).max())
    assert rel_err_rows(db, da).max() <= 1e-8
    assert np.abs(ea - eb).max() <= 1e-8 * np.abs(eb).max()
    assert np.abs(ca - cb).max() <= 1e-8 * max(1.0, np.abs(cb).max())

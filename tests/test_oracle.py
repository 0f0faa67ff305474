"""Pins of the f64 oracle by closed forms, invariants and independent algorithms.

Mirrors the reference's known-answer tests:
  crates/phyz-rigid/src/aba.rs:456-550        equilibrium, ABA <-> RNEA, pendulum, free fall
  crates/phyz-gpu/tests/joint_offset_vs_cpu.rs:47-84   closed-form offset double pendulum
  crates/phyz-rigid/src/integrate.rs:100-117  hinge integration
  crates/phyz-rigid/tests/free_joint.rs       fall at g, torque-free spin, body-frame velocity
  crates/phyz-rigid/tests/frame_conventions.rs FK frame convention
  crates/phyz-math/src/lib.rs:74-101          quat exp/log round trip
  crates/phyz-gpu/tests/contact_drop.rs, ground_contact.rs, cuda_vs_cpu.rs:272-367  contact, PD
and adds an independent CRBA + RNEA solve (Featherstone RBDA ch. 5-6) for both
ABA formulations on random trees with every joint type.
"""
import math

import numpy as np
import pytest

from oracle.oracle import Oracle, quat_exp_log, world_seed
from phyz_amd.model import (FREE, Geometry, Joint, ModelBuilder, SpatialInertia, SpatialTransform, pack_geometries,
                            uniform_frequency_gains)
from tests import models as TM

G = 9.81


@pytest.mark.parametrize("dense", [False, True])
def test_offset_double_pendulum_closed_form(dense):
    """M = [[4/3, 1/2], [1/2, 1/3]], tau = -g sin(theta) [3/2, 1/2] (joint_offset_vs_cpu.rs:43-53)."""
    o = Oracle(TM.double_pendulum_offset())
    for theta in (0.4, -1.1, 2.5):
        m11, m12, m22 = 4 / 3, 0.5, 1 / 3
        t1, t2 = -1.5 * G * math.sin(theta), -0.5 * G * math.sin(theta)
        det = m11 * m22 - m12 * m12
        a1 = (m22 * t1 - m12 * t2) / det
        a2 = (m11 * t2 - m12 * t1) / det
        qdd = o.aba([theta, 0.0], [0.0, 0.0], [0.0, 0.0], dense=dense)
        assert abs(qdd[0] - a1) < 1e-12 and abs(qdd[1] - (a2 - a1)) < 1e-12


def test_equilibrium_and_single_pendulum():
    o = Oracle(TM.double_pendulum_offset())
    assert np.abs(o.aba([0, 0], [0, 0], [0, 0])).max() < 1e-12
    m = (ModelBuilder().gravity([0, -G, 0])
         .add_revolute_body("l", -1, SpatialTransform.identity(),
                            SpatialInertia.new(1.0, [0, -0.5, 0], np.diag([1 / 12, 0, 1 / 12]))).build())
    o1 = Oracle(m)
    qdd = o1.aba([math.pi / 2], [0.0], [0.0])
    assert abs(qdd[0] - (-(G * 0.5) / (1.0 / 3.0))) < 1e-12


def test_aba_rnea_consistency():
    """RNEA(ABA(q, v, 0)) = 0 (aba.rs:470-485)."""
    o = Oracle(TM.double_pendulum_offset())
    q, v = [0.3, 0.2], [0.1, -0.1]
    qdd = o.aba(q, v, [0, 0])
    assert np.abs(o.rnea(q, v, qdd)).max() < 1e-12


@pytest.mark.parametrize("seed,nj,free", [(1, 8, True), (2, 12, True), (3, 6, False), (4, 20, True)])
@pytest.mark.parametrize("dense", [False, True])
def test_aba_equals_crba_rnea_solve(seed, nj, free, dense):
    """ABA against M(q) qdd = tau - h(q, v) with an independent CRBA/RNEA, on
    random trees over revolute, prismatic, ball, fixed and free joints, with
    springs, damping, armature and external forces."""
    m = TM.random_tree(seed, nj, free)
    o = Oracle(m)
    rng = np.random.default_rng(seed)
    for _ in range(3):
        q = rng.normal(size=m.nq) * 0.7
        v = rng.normal(size=m.nv)
        tau = rng.normal(size=m.nv)
        ext = rng.normal(size=(m.nbodies, 6))
        qdd = o.aba(q, v, tau, ext, dense=dense)
        M = o.crba(q)
        np.testing.assert_allclose(M, M.T, atol=1e-12)
        assert np.linalg.eigvalsh(M).min() > 0
        h = o.rnea(q, v, np.zeros(m.nv), ext)
        want = np.linalg.solve(M, o.generalized_forces(q, v, tau) - h)
        assert np.abs(qdd - want).max() <= 1e-11 * max(1.0, np.abs(want).max())


def test_dense_and_struct_formulations_agree():
    m = TM.random_tree(9, 15, True)
    o = Oracle(m)
    rng = np.random.default_rng(9)
    for _ in range(5):
        q, v, t = rng.normal(size=m.nq), rng.normal(size=m.nv), rng.normal(size=m.nv)
        a, b = o.aba(q, v, t), o.aba(q, v, t, dense=True)
        assert np.abs(a - b).max() <= 1e-12 * max(1.0, np.abs(b).max())


def test_hinge_integrates_scalar():
    """integrate.rs:100-117: v = 0 + 0.1*2, q = 0 + 0.1*0.2 (dt 0.1)."""
    m = (ModelBuilder().dt(0.1)
         .add_revolute_body("l", -1, SpatialTransform.identity(), SpatialInertia.point_mass(1.0, [0, 0, -0.5])).build())
    q, v = Oracle(m).integrate([0.0], [0.0], [2.0])
    assert abs(v[0] - 0.2) < 1e-15 and abs(q[0] - 0.02) < 1e-15


def _free_body(gravity=(0, 0, -G), inertia=np.eye(3), dt=0.001):
    return (ModelBuilder().gravity(gravity).dt(dt)
            .add_body("b", -1, Joint(FREE, SpatialTransform.identity(), np.zeros(3)),
                      SpatialInertia.new(1.0, np.zeros(3), inertia)).build())


def test_free_fall_at_g_without_yaw():
    """free_joint.rs:46-84: qdd = (0,0,0,0,0,-g); z(t) = 1 - g/2 (t^2 + t dt)."""
    m = _free_body()
    o = Oracle(m)
    q = np.zeros((1, 6)); q[0, 5] = 1.0
    v = np.zeros((1, 6)); c = np.zeros((1, 6))
    qdd = o.aba(q[0], v[0], c[0])
    assert np.abs(qdd[:5]).max() < 1e-12 and abs(qdd[5] + G) < 1e-12
    o.step_batch(q, v, c, 200)
    t = 0.2
    assert abs(q[0, 5] - (1.0 - 0.5 * G * (t * t + t * m.dt))) < 1e-9
    assert np.abs(q[0, :5]).max() < 1e-14
    assert abs(v[0, 5] + G * t) < 1e-9


def test_torque_free_spin_is_exact():
    """free_joint.rs:91-140: spin about a principal axis keeps omega; rotation = omega t."""
    m = _free_body(gravity=(0, 0, 0), inertia=np.diag([1.0, 1.0, 2.0]))
    o = Oracle(m)
    q = np.zeros((1, 6)); v = np.zeros((1, 6)); v[0, 2] = 3.0
    o.step_batch(q, v, np.zeros((1, 6)), 1000)
    assert np.abs(v[0, :2]).max() < 1e-9 and abs(v[0, 2] - 3.0) < 1e-9
    wrapped = (3.0 + math.pi) % (2 * math.pi) - math.pi
    _, lg = quat_exp_log(q[0, :3])
    assert np.abs(q[0, :2]).max() < 1e-9 and abs(lg[2] - wrapped) < 1e-9
    assert np.abs(q[0, 3:]).max() < 1e-12


def test_free_joint_linear_velocity_is_body_frame():
    """free_joint.rs:146-169: yaw 90 deg, body +x velocity translates along world +y."""
    m = _free_body(gravity=(0, 0, 0), dt=1.0)
    q, v = Oracle(m).integrate([0, 0, math.pi / 2, 0, 0, 0], [0, 0, 0, 1.0, 0, 0], np.zeros(6))
    assert abs(q[3]) < 1e-12 and abs(q[4] - 1.0) < 1e-12 and abs(q[5]) < 1e-12


def test_fk_frame_convention():
    """frame_conventions.rs:17-79: pos is the world position; rot^T maps body to world."""
    m = (ModelBuilder()
         .add_body("root", -1, Joint(FREE, SpatialTransform.identity(), np.zeros(3)),
                   SpatialInertia.new(1.0, np.zeros(3), np.eye(3) * 0.1))
         .add_revolute_body("child", 0, SpatialTransform.from_translation([0, 0, -1.0]),
                            SpatialInertia.point_mass(1.0, np.zeros(3))).build())
    o = Oracle(m)
    q = np.zeros(7); q[5] = 2.5
    fk = o.fk(q, np.zeros(7))
    assert abs(fk[0, 11] - 2.5) < 1e-12 and abs(fk[1, 11] - 1.5) < 1e-12
    m2 = (ModelBuilder().add_revolute_body("l", -1, SpatialTransform.identity(),
                                           SpatialInertia.point_mass(1.0, [0, 0, -0.5])).build())
    fk2 = Oracle(m2).fk([math.pi / 2], [0.0])
    body_to_world = fk2[0, :9].reshape(3, 3)  # stored body -> world
    mapped = body_to_world @ np.array([1.0, 0, 0])
    assert abs(mapped[0]) < 1e-12 and abs(mapped[1] - 1.0) < 1e-12


@pytest.mark.parametrize("w", [[0, 0, 0], [1e-18, 0, 0], [0.3, -0.7, 1.1], [0, 0, 3.0], [-2.0, 0.5, 0.25]])
def test_quat_exp_log_round_trip(w):
    """lib.rs:74-101: exp matches the closed form and log(exp(w)) = w."""
    q, lg = quat_exp_log(w)
    a = np.linalg.norm(w)
    if a > 0:
        want = np.concatenate([[math.cos(a / 2)], np.asarray(w) / a * math.sin(a / 2)])
        assert np.abs(q - want).max() <= 8 * np.finfo(float).eps
    assert np.linalg.norm(lg - np.asarray(w)) <= 1e-12


def test_rng_seed_mixing_matches_splitmix64():
    """world_seed: SplitMix64 of seed + golden * (world + 1) (policy_pipeline.rs:417-424),
    checked against a from-scratch 64-bit implementation."""
    M = (1 << 64) - 1

    def sm(seed, w):
        z = (seed + 0x9E3779B97F4A7C15 * (w + 1)) & M
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return (z ^ (z >> 31)) or 1

    for seed in (0, 1, 0xC4A17, M):
        for w in (0, 1, 7, 65535):
            assert world_seed(seed, w) == sm(seed, w)


def test_box_drop_rests_at_mg_over_k():
    """contact_drop.rs:19-70: mass-proportional gains (omega 50, zeta 1) rest the box
    at -0.9 - g tc^2 (within 1e-3) and at rest."""
    m = (ModelBuilder().gravity([0, 0, -G]).dt(0.001)
         .add_body("box", -1, Joint(FREE, SpatialTransform.from_translation([0, 0, 1.0]), np.zeros(3)),
                   SpatialInertia.new(1.0, np.zeros(3), np.eye(3) * 0.01), Geometry.box([0.1, 0.1, 0.1])).build())
    geom, n = pack_geometries(m, gains=uniform_frequency_gains(m, 50.0, 1.0))
    assert n == 1
    o = Oracle(m, contact=(geom, 0.0, 0.8))
    q, v, c = np.zeros((1, 6)), np.zeros((1, 6)), np.zeros((1, 6))
    o.step_batch(q, v, c, 2000)
    assert abs(q[0, 5] - (-0.9 - G * 0.02 * 0.02)) < 1e-3
    assert abs(v[0, 5]) < 1e-2


def test_sphere_rests_one_radius_up_with_weight_on_ground():
    """cuda_vs_cpu.rs:319-367 / ground_contact.rs: rests at z = r (+-0.02), normal
    force ~ mg (+-15%), contact point on the plane; airborne reports no contact."""
    mass, r, om = 1.0, 0.1, 200.0
    m = (ModelBuilder().gravity([0, 0, -G]).dt(0.001)
         .add_free_body("body", -1, SpatialTransform.identity(), SpatialInertia.new(mass, np.zeros(3), np.eye(3) * 0.4 * mass * r * r),
                        Geometry.sphere(r)).build())
    geom, _ = pack_geometries(m, mass * om * om, 2.0 * mass * om)
    for ground in (0.0, 0.35):
        o = Oracle(m, contact=(geom, ground, 0.5))
        q = np.zeros((1, 6)); q[0, 5] = ground + 0.5
        v, c = np.zeros((1, 6)), np.zeros((1, 6))
        _, rows = o.step_batch(q, v, c, 1, want_contacts=True)
        assert rows[0, 0, 0] == 0.0
        _, rows = o.step_batch(q, v, c, 2000, want_contacts=True)
        assert abs(q[0, 5] - (ground + r)) < 0.02
        assert rows[0, 0, 0] == 1.0
        assert abs(rows[0, 0, 7] - mass * G) < 0.15 * mass * G
        assert abs(rows[0, 0, 4] - ground) < 1e-6


def test_coulomb_friction_stops_a_sliding_sphere():
    """Sliding decelerates at mu g (kinetic regime of the regularised Coulomb law)
    until it sticks."""
    mass, r = 1.0, 0.1
    m = (ModelBuilder().gravity([0, 0, -G]).dt(0.001)
         .add_free_body("body", -1, SpatialTransform.identity(), SpatialInertia.new(mass, np.zeros(3), np.eye(3) * 1e6),
                        Geometry.sphere(r)).build())
    geom, _ = pack_geometries(m, mass * 200.0 ** 2, 2.0 * mass * 200.0)
    mu = 0.5
    o = Oracle(m, contact=(geom, 0.0, mu))
    q = np.zeros((1, 6)); q[0, 5] = r - G / 200.0 ** 2
    v = np.zeros((1, 6)); v[0, 3] = 1.0
    c = np.zeros((1, 6))
    o.step_batch(q, v, c, 50)  # let the normal contact settle; still sliding (v ~ 0.75)
    v0 = v[0, 3]
    assert v0 > 0.5
    o.step_batch(q, v, c, 100)
    decel = (v0 - v[0, 3]) / 0.1
    assert abs(decel - mu * G) < 0.02 * mu * G


def test_pd_servo_matches_damped_oscillator():
    """PD law (pd_pipeline.rs:8-13) on a gravity-free slider: x'' = (kp (t - x) - kd x') / m,
    whose solution the semi-implicit step follows to O(dt); and the clamp: a saturated
    servo accelerates at max_force / m."""
    from phyz_amd.model import PdDof, pack_pd_dofs
    m = (ModelBuilder().gravity([0, 0, 0]).dt(1e-4)
         .add_prismatic_body("s", -1, SpatialTransform.identity(), [1.0, 0, 0], SpatialInertia.point_mass(2.0, np.zeros(3)))
         .build())
    kp, kd, mass, target = 50.0, 4.0, 2.0, 0.8
    o = Oracle(m, pd=pack_pd_dofs([PdDof(0, 0, kp, kd, 1e9)]))
    q, v, c = np.array([[0.3]]), np.zeros((1, 1)), np.zeros((1, 1))
    o.step_batch(q, v, c, 5000, targets=np.array([[target]]))
    w0, zeta = math.sqrt(kp / mass), kd / (2 * math.sqrt(kp * mass))
    wd, t = w0 * math.sqrt(1 - zeta * zeta), 0.5
    x = target + (0.3 - target) * math.exp(-zeta * w0 * t) * (math.cos(wd * t) + zeta * w0 / wd * math.sin(wd * t))
    assert abs(q[0, 0] - x) < 2e-3
    o2 = Oracle(m, pd=pack_pd_dofs([PdDof(0, 0, kp, kd, 1.0)]))
    q, v, c = np.array([[0.0]]), np.zeros((1, 1)), np.zeros((1, 1))
    o2.step_batch(q, v, c, 1000, targets=np.array([[100.0]]))
    assert abs(c[0, 0] - 1.0) < 1e-15
    assert abs(v[0, 0] - 1.0 / mass * 0.1) < 1e-12


def test_normal_noise_moments():
    """The control stream's normal draws: mean a, std b (Box-Muller)."""
    m = TM.arm_6dof()
    o = Oracle(m, noise=(123, 0, 0.5, 2.0, list(range(6))))
    n = 4000
    q, v, c = np.zeros((n, 6)), np.zeros((n, 6)), np.zeros((n, 6))
    o.step_batch(q, v, c, 1, rng=o.rng_states(n), threads=8)
    assert abs(c.mean() - 0.5) < 0.05 and abs(c.std() - 2.0) < 0.05
    u = Oracle(m, noise=(5, 1, -1.0, 1.0, [0, 1]))
    q, v, c = np.zeros((n, 6)), np.zeros((n, 6)), np.zeros((n, 6))
    u.step_batch(q, v, c, 1, rng=u.rng_states(n), threads=8)
    assert c[:, :2].min() >= -1.0 and c[:, :2].max() < 1.0 and abs(c[:, :2].mean()) < 0.05

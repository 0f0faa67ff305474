"""The five benchmark workloads: models, seeded initial states, per-step inputs.

Each workload is a fixed model shared by every world plus seeded per-world
initial states. Per-step torques, where a workload has them, come from the
device control-noise stream (SplitMix64 world seed + xorshift64, the recipe of
crates/phyz-gpu/src/policy_pipeline.rs:417-456), which the oracle replays.

  1 double_pendulum  README model (README.md:46-60): two revolute Z joints at one
                     pivot, rods m=1.0 h=0.5 and m=0.8 h=0.4, gravity -Y, dt 2e-3.
                     4096 worlds x 500 steps, f64, no contact, zero torque.
  2 chain7           7 revolute joints, axes Z,Y,Z,Y,..., rods along +X with the
                     next joint at the tip; m~U[0.5,2], L~U[0.2,0.5]; dt 1e-3.
                     65536 worlds x 1000 steps, f32 and f64, tau~N(0,1) per step.
  3 ant              free torso (sphere r 0.25, 1 kg) + 4 x (hip Z, knee Y); leg
                     segments 0.2-0.4 m, 0.1-0.3 kg; 4 foot spheres r 0.08;
                     ground k 1e4, d 100, mu 1; dt 2e-3. 131072 worlds x 1000
                     steps, f32, tau~U[-1,1] per step on the hinges.
  4 humanoid         free torso + 21 hinges over 22 links (3-DOF hips/shoulders
                     and 2-DOF ankles expanded into chains with 1e-9 kg links,
                     crates/phyz-mjcf/src/parser.rs:737-790); masses 0.5-8 kg;
                     hinge armature 0.01, damping 0.5; 10 contact spheres; dt 1e-3. 32768 worlds x 1000 steps,
                     f32 and f64, tau~N(0,2) per step on the hinges.
  5 hand             fixed palm + 24 revolute DOF in 5 fingers (5,5,5,5,4);
                     m 0.01-0.05 kg, L 0.02-0.05 m; PD servos on every DOF with
                     per-world targets; dt 5e-4. 16384 worlds x 2000 steps, f64.
  6 ant_terrain_impulse  workload 3 on a 41 x 41 node rolling heightfield (8 m
                     square, +-0.06 m) with impulse-mode contact: a leading ABA,
                     then 16 sweeps of [contact at the free velocity, ABA re-solve]
                     per step (mod.rs:899-928). 131072 worlds x 1000 steps, f32.
"""
from __future__ import annotations

import dataclasses
import math
import os
from typing import List, Optional, Tuple

import numpy as np

from .model import (BALL, FIXED, FREE, PRISMATIC, REVOLUTE, Geometry, Heightfield, Joint, Model, ModelBuilder,
                    PdDof, SpatialInertia, SpatialTransform, model_from_tables, pack_geometries, pack_pd_dofs,
                    rotation_axis_angle, uniform_frequency_gains)

NOISE_NORMAL = 0
NOISE_UNIFORM = 1


@dataclasses.dataclass
class Contact:
    ground_height: float
    stiffness: float
    damping: float
    friction: float


@dataclasses.dataclass
class Noise:
    seed: int
    dist: int
    a: float
    b: float
    dofs: List[int]


@dataclasses.dataclass
class Workload:
    index: int
    name: str
    model: Model
    nworld: int
    nsteps: int
    precisions: Tuple[str, ...]
    contact: Optional[Contact] = None
    pd: Optional[List[PdDof]] = None
    noise: Optional[Noise] = None
    init_seed: int = 0
    _init: Optional[object] = None
    heightfield: Optional[Heightfield] = None  # terrain in place of the flat ground
    impulse_sweeps: int = 0                    # > 0: impulse-mode contact with this many sweeps
    gains_omega: float = 0.0                   # > 0: per-body contact gains k = m w^2, d = 2 m w

    def initial_state(self, nworld: Optional[int] = None):
        """World-major f64 (q, v, ctrl, targets|None) for the first `nworld` worlds."""
        n = self.nworld if nworld is None else nworld
        q, v, ctrl, tg = self._init(self, max(n, 1))
        return q[:n].copy(), v[:n].copy(), ctrl[:n].copy(), None if tg is None else tg[:n].copy()

    def geometry_table(self):
        if self.contact is None:
            return None, 0
        if self.gains_omega > 0.0:
            return pack_geometries(self.model, gains=self.contact_gains())
        return pack_geometries(self.model, self.contact.stiffness, self.contact.damping)

    def contact_gains(self):
        """Per-body (stiffness, damping): uniform-frequency gains when the workload
        names a frequency, else the workload's ground gains on every body."""
        if self.gains_omega > 0.0:
            return uniform_frequency_gains(self.model, self.gains_omega, 1.0)
        return [(self.contact.stiffness, self.contact.damping)] * self.model.nbodies

    def impulse_erp(self) -> float:
        """Baumgarte factor of impulse mode: dt / (2 * 0.02 * 1 + dt), time constant
        0.02 s, damping ratio 1 (the impulse-mode default of mod.rs:680-701)."""
        return self.model.dt / (0.04 + self.model.dt)

    def pd_table(self):
        return None if self.pd is None else pack_pd_dofs(self.pd)

    def summary(self) -> dict:
        return {"workload": self.name, "config": self.index, "nworld": self.nworld, "steps": self.nsteps,
                "bodies": self.model.nbodies, "nv": self.model.nv}


def _rod_x(mass: float, length: float, radius: float = 0.02) -> SpatialInertia:
    """Uniform rod along +X from the joint: COM at L/2, axial inertia of a solid cylinder."""
    it = mass * length * length / 12.0
    ia = 0.5 * mass * radius * radius
    return SpatialInertia.new(mass, [0.5 * length, 0.0, 0.0], np.diag([ia, it, it]))


def _rod_dir(mass: float, length: float, d, radius: float = 0.02) -> SpatialInertia:
    """Uniform rod from the joint along unit direction d."""
    d = np.asarray(d, dtype=np.float64)
    d = d / np.linalg.norm(d)
    it = mass * length * length / 12.0
    ia = 0.5 * mass * radius * radius
    I = it * (np.eye(3) - np.outer(d, d)) + ia * np.outer(d, d)
    return SpatialInertia.new(mass, 0.5 * length * d, I)


def _dummy() -> SpatialInertia:
    """Placeholder link of a multi-joint body (parser.rs:737-790): 1e-9 kg, 1e-9 I."""
    return SpatialInertia.new(1e-9, np.zeros(3), np.eye(3) * 1e-9)


# ── 1: double pendulum ──────────────────────────────────────────────────────
def double_pendulum_model() -> Model:
    return (ModelBuilder().gravity([0.0, -9.81, 0.0]).dt(0.002)
            .add_revolute_body("upper", -1, SpatialTransform.identity(), SpatialInertia.rod(1.0, 0.5))
            .add_revolute_body("lower", 0, SpatialTransform.identity(), SpatialInertia.rod(0.8, 0.4))
            .build())


def _init_dp(w: Workload, n: int):
    rng = np.random.default_rng(w.init_seed)
    q = rng.uniform(-math.pi, math.pi, size=(n, 2))
    v = rng.uniform(-1.0, 1.0, size=(n, 2))
    return q, v, np.zeros((n, 2)), None


# ── 2: 7-link chain ─────────────────────────────────────────────────────────
def chain7_model(seed: int = 7) -> Model:
    rng = np.random.default_rng(seed)
    masses = rng.uniform(0.5, 2.0, size=7)
    lengths = rng.uniform(0.2, 0.5, size=7)
    b = ModelBuilder().gravity([0.0, 0.0, -9.81]).dt(0.001)
    for i in range(7):
        axis = (0.0, 0.0, 1.0) if i % 2 == 0 else (0.0, 1.0, 0.0)
        ptj = SpatialTransform.identity() if i == 0 else SpatialTransform.from_translation([lengths[i - 1], 0.0, 0.0])
        b.add_revolute_body(f"link{i}", i - 1, ptj, _rod_x(masses[i], lengths[i]), axis=axis)
    return b.build()


def _init_chain(w: Workload, n: int):
    rng = np.random.default_rng(w.init_seed)
    q = rng.uniform(-math.pi, math.pi, size=(n, 7))
    v = rng.normal(0.0, 0.5, size=(n, 7))
    return q, v, np.zeros((n, 7)), None


# ── 3: ant ──────────────────────────────────────────────────────────────────
def ant_model(seed: int = 3) -> Model:
    rng = np.random.default_rng(seed)
    b = ModelBuilder().gravity([0.0, 0.0, -9.81]).dt(0.002)
    b.add_free_body("torso", -1, SpatialTransform.identity(), SpatialInertia.sphere(1.0, 0.25))
    alpha = math.radians(60.0)
    shin_dir = np.array([math.cos(alpha), 0.0, -math.sin(alpha)])
    for k in range(4):
        phi = math.radians(45.0 + 90.0 * k)
        d = np.array([math.cos(phi), math.sin(phi), 0.0])
        l_thigh, l_shin = rng.uniform(0.2, 0.4, size=2)
        m_thigh, m_shin = rng.uniform(0.1, 0.3, size=2)
        # Joint frame x-axis along the leg: the parent->joint map is R_z(-phi).
        hip = SpatialTransform.new(rotation_axis_angle([0, 0, 1], -phi), 0.25 * d)
        hip_idx = len(b._bodies)
        b.add_revolute_body(f"thigh{k}", 0, hip, _rod_x(m_thigh, l_thigh, 0.04), axis=(0.0, 0.0, 1.0))
        knee = SpatialTransform.from_translation([l_thigh, 0.0, 0.0])
        foot = Geometry.sphere(0.08, SpatialTransform.from_translation(l_shin * shin_dir))
        b.add_body(f"shin{k}", hip_idx, Joint(REVOLUTE, knee, np.array([0.0, 1.0, 0.0])),
                   _rod_dir(m_shin, l_shin, shin_dir, 0.04), foot)
    return b.build()


def _init_ant(w: Workload, n: int):
    rng = np.random.default_rng(w.init_seed)
    q = np.zeros((n, 14))
    q[:, 5] = rng.uniform(0.5, 1.0, size=n)
    q[:, 6:] = rng.uniform(-0.5, 0.5, size=(n, 8))
    return q, np.zeros((n, 14)), np.zeros((n, 14)), None


# ── 4: humanoid ─────────────────────────────────────────────────────────────
def humanoid_model(seed: int = 4) -> Model:
    rng = np.random.default_rng(seed)
    mass = lambda: float(rng.uniform(0.5, 8.0))
    b = ModelBuilder().gravity([0.0, 0.0, -9.81]).dt(0.001)
    X, Y, Z = (1.0, 0.0, 0.0), (0.0, 1.0, 0.0), (0.0, 0.0, 1.0)
    down = np.array([0.0, 0.0, -1.0])
    T = SpatialTransform.from_translation
    I = SpatialTransform.identity

    def hinge(name, parent, ptj, axis, inertia, geom=None):
        # MuJoCo-humanoid-like joint regularisation: rotor armature and viscous damping.
        idx = len(b._bodies)
        b.add_body(name, parent, Joint(REVOLUTE, ptj, np.array(axis), damping=0.5, armature=0.01), inertia, geom)
        return idx

    b.add_free_body("torso", -1, I(), _rod_dir(mass(), 0.35, [0, 0, 1], 0.1),
                    Geometry.sphere(0.09, T([0.0, 0.0, 0.45])))
    pelvis = hinge("pelvis", 0, T([0.0, 0.0, -0.25]), Y, _rod_dir(mass(), 0.15, down, 0.1), Geometry.sphere(0.09))
    for side, s in (("l", 1.0), ("r", -1.0)):
        h1 = hinge(f"hip_x_{side}", pelvis, T([0.0, 0.1 * s, -0.1]), X, _dummy())
        h2 = hinge(f"hip_y_{side}", h1, I(), Y, _dummy())
        thigh = hinge(f"thigh_{side}", h2, I(), Z, _rod_dir(mass(), 0.4, down, 0.06))
        shin = hinge(f"shin_{side}", thigh, T([0.0, 0.0, -0.4]), Y, _rod_dir(mass(), 0.4, down, 0.05),
                     Geometry.sphere(0.05))
        a1 = hinge(f"ankle_y_{side}", shin, T([0.0, 0.0, -0.4]), Y, _dummy())
        hinge(f"foot_{side}", a1, I(), X, SpatialInertia.new(mass(), [0.05, 0.0, -0.04], np.diag([2e-3, 4e-3, 4e-3])),
              Geometry.sphere(0.05, T([0.05, 0.0, -0.05])))
    for side, s in (("l", 1.0), ("r", -1.0)):
        s1 = hinge(f"shoulder_x_{side}", 0, T([0.0, 0.2 * s, 0.15]), X, _dummy())
        s2 = hinge(f"shoulder_y_{side}", s1, I(), Y, _dummy())
        upper = hinge(f"upper_arm_{side}", s2, I(), Z, _rod_dir(mass(), 0.28, down, 0.04),
                      Geometry.sphere(0.04, T([0.0, 0.0, -0.28])))
        hinge(f"forearm_{side}", upper, T([0.0, 0.0, -0.28]), Y, _rod_dir(mass(), 0.25, down, 0.035),
              Geometry.sphere(0.04, T([0.0, 0.0, -0.25])))
    return b.build()


def _init_humanoid(w: Workload, n: int):
    rng = np.random.default_rng(w.init_seed)
    nq = w.model.nq
    q = np.zeros((n, nq))
    q[:, 5] = rng.uniform(1.2, 1.4, size=n)
    q[:, 6:] = rng.uniform(-0.3, 0.3, size=(n, nq - 6))
    return q, np.zeros((n, nq)), np.zeros((n, nq)), None


# ── 5: hand ─────────────────────────────────────────────────────────────────
HAND_FINGERS = (5, 5, 5, 5, 4)


def hand_model(seed: int = 5) -> Tuple[Model, float, float]:
    """Returns (model, kp, kd). PD gains keep sqrt(kp/I_min)*dt = 0.1 for the
    lightest link's inertia about its own joint, damping ratio 0.5. (At 0.2,
    the f64 oracle itself ran 276 of the 16384 worlds into a clamped
    oscillation above 100 rad/s and 2 to NaN within 2000 steps: the coupled
    fingers' mass matrix has modes lighter than any single link. At 0.1 every
    world stays finite, |v| <= 63 rad/s.)"""
    rng = np.random.default_rng(seed)
    dt = 0.0005
    b = ModelBuilder().gravity([0.0, 0.0, -9.81]).dt(dt)
    b.add_fixed_body("palm", -1, SpatialTransform.identity(),
                     SpatialInertia.new(0.3, [0.0, 0.0, 0.0], np.diag([3e-4, 3e-4, 5e-4])))
    i_min = math.inf
    bases = [([0.02, -0.04, 0.0], -0.6), ([0.09, -0.025, 0.0], -0.1), ([0.095, 0.0, 0.0], 0.0),
             ([0.09, 0.025, 0.0], 0.1), ([0.08, 0.045, 0.0], 0.2)]
    for f, nlink in enumerate(HAND_FINGERS):
        base_pos, yaw = bases[f]
        parent = 0
        prev_len = 0.0
        for j in range(nlink):
            m = float(rng.uniform(0.01, 0.05))
            L = float(rng.uniform(0.02, 0.05))
            if j == 0:
                ptj = SpatialTransform.new(rotation_axis_angle([0, 0, 1], -yaw), base_pos)
                axis = (0.0, 0.0, 1.0)            # abduction
            else:
                ptj = SpatialTransform.from_translation([prev_len, 0.0, 0.0])
                axis = (0.0, 1.0, 0.0)            # flexion
            inertia = _rod_x(m, L, 0.006)
            i_min = min(i_min, m * L * L / 3.0)
            idx = len(b._bodies)
            b.add_revolute_body(f"f{f}_l{j}", parent, ptj, inertia, axis=axis)
            parent = idx
            prev_len = L
    omega = 0.1 / dt
    kp = i_min * omega * omega
    kd = 2.0 * 0.5 * i_min * omega
    return b.build(), kp, kd


def _init_hand(w: Workload, n: int):
    rng = np.random.default_rng(w.init_seed)
    nv = w.model.nv
    q = rng.uniform(-0.3, 1.2, size=(n, nv))
    targets = rng.uniform(-0.3, 1.2, size=(n, nv))
    return q, np.zeros((n, nv)), np.zeros((n, nv)), targets


def config(index: int) -> Workload:
    """Workload `index` (1..5) at its full size."""
    if index == 1:
        return Workload(1, "double_pendulum", double_pendulum_model(), 4096, 500, ("f64",), init_seed=101,
                        _init=_init_dp)
    if index == 2:
        m = chain7_model()
        return Workload(2, "chain7", m, 65536, 1000, ("f32", "f64"),
                        noise=Noise(seed=0xC4A17, dist=NOISE_NORMAL, a=0.0, b=1.0, dofs=list(range(7))),
                        init_seed=102, _init=_init_chain)
    if index == 3:
        m = ant_model()
        return Workload(3, "ant", m, 131072, 1000, ("f32",),
                        contact=Contact(0.0, 1e4, 100.0, 1.0),
                        noise=Noise(seed=0xA17, dist=NOISE_UNIFORM, a=-1.0, b=1.0, dofs=list(range(6, 14))),
                        init_seed=103, _init=_init_ant)
    if index == 4:
        m = humanoid_model()
        return Workload(4, "humanoid", m, 32768, 1000, ("f32", "f64"),
                        contact=Contact(0.0, 1e4, 100.0, 1.0),
                        noise=Noise(seed=0x4D, dist=NOISE_NORMAL, a=0.0, b=2.0, dofs=list(range(6, m.nv))),
                        init_seed=104, _init=_init_humanoid)
    if index == 5:
        m, kp, kd = hand_model()
        pd = [PdDof(j, j, kp, kd, kp * math.pi) for j in range(m.nv)]
        return Workload(5, "hand", m, 16384, 2000, ("f64",), pd=pd, init_seed=105, _init=_init_hand)
    if index == 6:
        w = config(3)
        return dataclasses.replace(w, index=6, name="ant_terrain_impulse", heightfield=rolling_terrain(),
                                   impulse_sweeps=16)
    if index in MJCF_WORKLOADS:
        name, nworld, precisions = MJCF_WORKLOADS[index]
        m = dataclasses.replace(mjcf_model(name), dt=MJCF_DT)
        lo = min(a.ctrl_range[0] for a in m.actuators)
        hi = max(a.ctrl_range[1] for a in m.actuators)
        return Workload(index, f"mjcf_{name}", m, nworld, 1000, precisions, contact=Contact(0.0, 0.0, 0.0, 1.0),
                        noise=Noise(seed=0x3C0 + index, dist=NOISE_UNIFORM, a=lo, b=hi, dofs=list(range(m.nu()))),
                        init_seed=100 + index, _init=_init_mjcf, gains_omega=50.0)
    raise ValueError(f"no workload {index}")


# The reference's five benchmark configurations; EXTRA are workloads beyond
# them: contact modes (heightfield terrain, impulse solve) and the reference's
# own MJCF benchmark models.
ALL = (1, 2, 3, 4, 5)
EXTRA = (6, 7, 8, 9)


# ── 7-9: the reference's MJCF benchmark models, driven by their actuators ───
# name, worlds, precisions. Controls: uniform over the actuators' control range
# every step (the files' ctrlrange, which the loader converts to radians under
# angle="degree" as the reference does).
# Step: 1 ms, not the files' timestep (5 ms humanoid, 2 ms hand). The soft
# joint-limit law (joint.rs:196-247, k = 1000, d = 60) is explicit, and its
# damping term is unstable once d dt / I > 2 for a link's inertia I about its
# joint: at the files' steps 13% of humanoid and 27% of hand worlds (oracle,
# 128 worlds, 1000 steps) ran away as soon as a light link reached a limit,
# and none without limits. At 1 ms every world of the three models stays
# finite over 2000 steps (oracle, 512 worlds each).
MJCF_DT = 0.001
MJCF_WORKLOADS = {7: ("ant", 131072, ("f32",)), 8: ("humanoid", 32768, ("f32", "f64")),
                  9: ("shadow_hand", 16384, ("f32", "f64"))}


def _init_mjcf(w: Workload, n: int):
    """Hinges uniform over the middle 80% of their range, free roots slightly
    tilted at their file placement, at rest."""
    rng = np.random.default_rng(w.init_seed)
    m = w.model
    q = np.zeros((n, m.nq))
    for i, b in enumerate(m.bodies):
        j, o = b.joint, m.q_offsets[i]
        if j.ndof() == 1 and j.limits is not None:
            lo, hi = j.limits
            r = hi - lo
            q[:, o] = rng.uniform(lo + 0.1 * r, hi - 0.1 * r, size=n)
        elif j.ndof() == 6:
            q[:, o:o + 3] = rng.normal(size=(n, 3)) * 0.05
    return q, np.zeros((n, m.nv)), np.zeros((n, m.nu())), None


# ── 6: ant on rolling terrain, impulse-mode contact ─────────────────────────
def rolling_terrain(n: int = 41, cell: float = 0.2, amp: float = 0.06, seed: int = 6) -> Heightfield:
    """An n x n node heightfield, 8 m square centred on the origin: a seeded sum
    of six plane waves of 1.5-4 m wavelength, peak-to-peak about 2 amp."""
    rng = np.random.default_rng(seed)
    xs = (np.arange(n) - (n - 1) / 2) * cell
    X, Y = np.meshgrid(xs, xs)  # [iy][ix]
    h = np.zeros((n, n))
    for _ in range(6):
        lam = rng.uniform(1.5, 4.0)
        th = rng.uniform(0.0, 2 * math.pi)
        ph = rng.uniform(0.0, 2 * math.pi)
        k = 2 * math.pi / lam
        h += np.sin(k * (math.cos(th) * X + math.sin(th) * Y) + ph)
    h *= amp / np.abs(h).max()
    return Heightfield(origin=(float(xs[0]), float(xs[0]), 0.0), cell=cell, nx=n, ny=n, heights=h)


# ── the reference's MJCF benchmark models ───────────────────────────────────
MJCF_TABLES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data", "mjcf_models.npz")


def mjcf_model(name: str) -> Model:
    """One of the reference's benchmark MJCF models (ant, humanoid, shadow_hand,
    half_cheetah, simple_arm) as phyz_amd.mjcf loads it, from the packed tables
    phyz_amd/data/make_mjcf_models.py wrote (the model files stay in the reference)."""
    z = np.load(MJCF_TABLES)
    g = lambda k: z[f"{name}/{k}"]  # noqa: E731
    nq, nv, dt = g("dims")
    acts = g("actuators")
    return model_from_tables(g("body"), g("geom"), g("gravity"), dt, int(nq), int(nv), g("joint_terms"),
                             acts if acts.size else None, g("body_names"), g("joint_names"), g("actuator_names"))


# ── control loop: the ant driven by an on-device policy ─────────────────────
@dataclasses.dataclass
class ControlLoop:
    """An RL collector's rollout on the ant (workload 3's model and contact, no
    control-noise torques): every `control_every` physics steps, FK, a 29-feature
    observation row, a 29-256-256-8 tanh MLP with an AR(1) Gaussian sample, and
    the clamped actions onto hip/knee PD targets; the state is recorded after
    each control step (docs/design/cuda-backend.md section 7 of the reference)."""
    name: str
    base: Workload
    pd: List[PdDof]
    spec: object
    weights: np.ndarray
    std: np.ndarray
    seed: int
    n_control: int
    control_every: int

    @property
    def nworld(self) -> int:
        return self.base.nworld

    def base_targets(self, n: Optional[int] = None) -> np.ndarray:
        """Standing pose: hips 0, knees 0.5 rad, every world."""
        n = self.nworld if n is None else n
        row = np.array([0.0, 0.5] * 4)
        return np.tile(row, (n, 1))

    def flops_per_world(self) -> int:
        """MLP multiply-adds x 2 per world and control step (biases, tanh and the
        sample not counted)."""
        i, h, o = self.spec.n_in(), self.spec.hidden, self.spec.n_out()
        return 2 * (i * h + h * h + h * o)


def control_loop(hidden: int = 256) -> ControlLoop:
    from .policy import BodyPitch, BodyPos, BodyPosZ, BodyRoll, BodyYawError, ComOverSupport, PolicySpec, QMinus, V
    base = config(3)
    m = base.model
    base = dataclasses.replace(base, name="ant_control", noise=None)
    pd = [PdDof(6 + k, 6 + k, 20.0, 1.0, 10.0) for k in range(8)]
    feet = [(2 + 2 * k, [0.0, 0.0, 0.0]) for k in range(4)]
    obs = ([BodyPitch(0), BodyRoll(0), BodyYawError(0, 0.0), BodyPosZ(0), BodyPos(0, 0)]
           + [QMinus(6 + k, 0.5 if k % 2 else 0.0) for k in range(8)] + [V(j) for j in range(14)]
           + [ComOverSupport(feet, 0, 0), ComOverSupport(feet, 0, 1)])
    spec = PolicySpec(obs=obs, hidden=hidden, act_slots=list(range(8)), act_clamp=0.5, noise_rho=0.5,
                      input_noise=[0.01] * len(obs), history_steps=50)
    rng = np.random.default_rng(0xC0)
    n_in, h, n_out = spec.n_in(), hidden, spec.n_out()
    weights = np.concatenate([rng.normal(size=h * n_in) / math.sqrt(n_in), np.zeros(h),
                              rng.normal(size=h * h) / math.sqrt(h), np.zeros(h),
                              0.1 * rng.normal(size=n_out * h) / math.sqrt(h), np.zeros(n_out)])
    return ControlLoop("ant_control", base, pd, spec, weights, np.full(n_out, 0.2), seed=0xC0DE,
                       n_control=50, control_every=5)

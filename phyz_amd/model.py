"""Model description and the f64 wire tables the C ABI takes.

Host-side mirror of the reference's model types and packers:

* ``SpatialInertia`` / ``SpatialTransform``  — phyz-math (tang) semantics:
  inertia about the COM; transform ``rot`` = parent->joint coordinate map,
  ``pos`` = joint origin in parent coordinates (crates/phyz-model/src/joint.rs:31-36).
* ``Joint`` / ``ModelBuilder``               — crates/phyz-model/src/joint.rs:27-160,
  crates/phyz-model/src/model.rs:379-551 (q/v offsets assigned in body order,
  default gravity (0, 0, -9.81), dt 1e-3).
* ``pack_bodies`` / ``pack_geometries`` / ``pack_pd_dofs`` — the slot layouts of
  crates/phyz-gpu/src/layout.rs:19-93, in f64 instead of f32, with integer slots
  stored as exact integer-valued doubles instead of bit casts.
"""
from __future__ import annotations

import dataclasses
import math
from typing import List, Optional, Sequence

import numpy as np

GRAVITY = 9.81

# Joint type codes (layout.rs:23) and geometry codes (layout.rs:43).
REVOLUTE, PRISMATIC, FIXED, BALL, FREE = 0, 1, 2, 3, 4
G_NONE, G_SPHERE, G_BOX, G_CAPSULE, G_CYLINDER, G_MESH = 0, 1, 2, 3, 4, 5

BODY_STRIDE = 36
GEOM_STRIDE = 24
JOINT_TERMS_STRIDE = 8
ACTUATOR_STRIDE = 16
DEFAULT_LIMIT_STIFFNESS = 1000.0  # joint.rs:96-104
DEFAULT_LIMIT_DAMPING = 60.0
PD_DOF_STRIDE = 8
CONTACT_ROW = 8
MAX_BODIES = 32

_NDOF = {REVOLUTE: 1, PRISMATIC: 1, FIXED: 0, BALL: 3, FREE: 6}


def joint_ndof(jtype: int) -> int:
    return _NDOF[jtype]


def _mat3(m) -> np.ndarray:
    a = np.asarray(m, dtype=np.float64).reshape(3, 3)
    return a.copy()


def _vec3(v) -> np.ndarray:
    return np.asarray(v, dtype=np.float64).reshape(3).copy()


def rotation_axis_angle(axis, angle: float) -> np.ndarray:
    """Rotation matrix of `angle` about unit `axis` (Rodrigues, active sense)."""
    a = _vec3(axis)
    a = a / np.linalg.norm(a)
    k = np.array([[0, -a[2], a[1]], [a[2], 0, -a[0]], [-a[1], a[0], 0]])
    return np.eye(3) + math.sin(angle) * k + (1 - math.cos(angle)) * (k @ k)


@dataclasses.dataclass
class SpatialTransform:
    rot: np.ndarray = dataclasses.field(default_factory=lambda: np.eye(3))
    pos: np.ndarray = dataclasses.field(default_factory=lambda: np.zeros(3))

    @staticmethod
    def identity() -> "SpatialTransform":
        return SpatialTransform()

    @staticmethod
    def from_translation(p) -> "SpatialTransform":
        return SpatialTransform(np.eye(3), _vec3(p))

    @staticmethod
    def new(rot, pos) -> "SpatialTransform":
        return SpatialTransform(_mat3(rot), _vec3(pos))

    def compose(self, other: "SpatialTransform") -> "SpatialTransform":
        """self.compose(other): rot = self.rot @ other.rot, pos = other.pos + other.rot^T self.pos."""
        return SpatialTransform(self.rot @ other.rot, other.pos + other.rot.T @ self.pos)


@dataclasses.dataclass
class SpatialInertia:
    mass: float
    com: np.ndarray
    inertia: np.ndarray  # 3x3 about the COM

    @staticmethod
    def new(mass: float, com, inertia) -> "SpatialInertia":
        return SpatialInertia(float(mass), _vec3(com), _mat3(inertia))

    @staticmethod
    def sphere(mass: float, radius: float) -> "SpatialInertia":
        i = 0.4 * mass * radius * radius
        return SpatialInertia.new(mass, np.zeros(3), np.eye(3) * i)

    @staticmethod
    def point_mass(mass: float, com) -> "SpatialInertia":
        return SpatialInertia.new(mass, com, np.zeros((3, 3)))

    @staticmethod
    def rod(mass: float, half_len: float) -> "SpatialInertia":
        """Uniform rod hanging along -Y from the joint (the reference test fixture)."""
        length = 2.0 * half_len
        i = mass * length * length / 12.0
        return SpatialInertia.new(mass, [0.0, -half_len, 0.0], np.diag([i, 0.0, i]))


@dataclasses.dataclass
class Geometry:
    """One collision shape per body (the device contacts through collisions[0]; layout.rs:199-208)."""
    kind: int
    params: Sequence[float] = ()  # sphere (r); box (hx, hy, hz); capsule (r, length); cylinder (r, height); mesh aabb (min3, max3)
    origin: SpatialTransform = dataclasses.field(default_factory=SpatialTransform)

    @staticmethod
    def sphere(radius: float, origin: Optional[SpatialTransform] = None) -> "Geometry":
        return Geometry(G_SPHERE, (radius,), origin or SpatialTransform())

    @staticmethod
    def box(half_extents, origin: Optional[SpatialTransform] = None) -> "Geometry":
        return Geometry(G_BOX, tuple(half_extents), origin or SpatialTransform())

    @staticmethod
    def capsule(radius: float, length: float, origin: Optional[SpatialTransform] = None) -> "Geometry":
        return Geometry(G_CAPSULE, (radius, length), origin or SpatialTransform())

    @staticmethod
    def cylinder(radius: float, height: float, origin: Optional[SpatialTransform] = None) -> "Geometry":
        return Geometry(G_CYLINDER, (radius, height), origin or SpatialTransform())

    @staticmethod
    def mesh_aabb(lo, hi, origin: Optional[SpatialTransform] = None) -> "Geometry":
        return Geometry(G_MESH, tuple(lo) + tuple(hi), origin or SpatialTransform())


@dataclasses.dataclass
class Joint:
    jtype: int
    parent_to_joint: SpatialTransform = dataclasses.field(default_factory=SpatialTransform)
    axis: np.ndarray = dataclasses.field(default_factory=lambda: np.array([0.0, 0.0, 1.0]))
    damping: float = 0.0
    stiffness: float = 0.0
    spring_ref: float = 0.0
    armature: float = 0.0
    # Terms of the CPU model that the device body table does not carry
    # (joint.rs:27-104): the soft position limit and dry friction of a one-DOF joint.
    limits: Optional[Sequence[float]] = None
    limit_stiffness: float = DEFAULT_LIMIT_STIFFNESS
    limit_damping: float = DEFAULT_LIMIT_DAMPING
    friction_loss: float = 0.0
    name: str = ""

    def ndof(self) -> int:
        return joint_ndof(self.jtype)

    def limit_force(self, q: float, qd: float) -> float:
        """Soft joint-limit force (joint.rs:196-226): zero inside the range or on a
        multi-DOF joint; past a bound, a spring on the depth plus damping that
        only resists motion further into the limit."""
        if self.ndof() != 1 or self.limits is None:
            return 0.0
        lo, hi = self.limits
        if q < lo:
            depth, sign = lo - q, 1.0
        elif q > hi:
            depth, sign = q - hi, -1.0
        else:
            return 0.0
        return sign * (self.limit_stiffness * depth + self.limit_damping * max(-sign * qd, 0.0))


@dataclasses.dataclass
class Actuator:
    """Drives the first DOF of one joint (phyz_model::Actuator, model.rs:18-82):
    f = gear (gain clamp(ctrl) + bias_q q + bias_v v), then the force range."""
    name: str
    joint_name: str
    joint_idx: int  # body index: one joint per body
    gear: float = 1.0
    ctrl_range: Optional[Sequence[float]] = None
    gain: float = 1.0
    bias_q: float = 0.0
    bias_v: float = 0.0
    force_range: Optional[Sequence[float]] = None

    def clamp_ctrl(self, ctrl: float) -> float:
        if self.ctrl_range is None:
            return ctrl
        lo, hi = self.ctrl_range
        return min(max(ctrl, min(lo, hi)), max(lo, hi))

    def force_at(self, ctrl: float, q: float, v: float) -> float:
        f = self.gear * (self.gain * self.clamp_ctrl(ctrl) + self.bias_q * q + self.bias_v * v)
        if self.force_range is not None:
            lo, hi = self.force_range
            f = min(max(f, min(lo, hi)), max(lo, hi))
        return f

    @staticmethod
    def motor(name: str, joint_name: str, joint_idx: int, gear: float) -> "Actuator":
        return Actuator(name, joint_name, joint_idx, gear)

    @staticmethod
    def position(name: str, joint_name: str, joint_idx: int, gear: float, kp: float, kv: float) -> "Actuator":
        return Actuator(name, joint_name, joint_idx, gear, gain=kp, bias_q=-kp, bias_v=-kv)


@dataclasses.dataclass
class Body:
    name: str
    parent: int
    joint: Joint
    inertia: SpatialInertia
    geometry: Optional[Geometry] = None  # the contact shape (the first collision geom)
    collisions: List[Geometry] = dataclasses.field(default_factory=list)  # all collision geoms, in order


@dataclasses.dataclass
class Model:
    bodies: List[Body]
    gravity: np.ndarray
    dt: float
    nq: int
    nv: int
    q_offsets: List[int]
    v_offsets: List[int]
    actuators: List[Actuator] = dataclasses.field(default_factory=list)

    @property
    def nbodies(self) -> int:
        return len(self.bodies)

    @property
    def joints(self) -> List[Joint]:
        return [b.joint for b in self.bodies]

    def nu(self) -> int:
        """Number of actuators (MuJoCo's nu)."""
        return len(self.actuators)

    def nctrl(self) -> int:
        """Controls per world: one per actuator, or one per DOF without actuators."""
        return self.nu() if self.actuators else self.nv

    def has_joint_terms(self) -> bool:
        return any(b.joint.ndof() == 1 and (b.joint.limits is not None or b.joint.friction_loss > 0.0)
                   for b in self.bodies)

    def default_state(self):
        return np.zeros(self.nq), np.zeros(self.nv)


class ModelBuilder:
    """Builder with the reference's method names (model.rs:379-551)."""

    def __init__(self):
        self._bodies: List[Body] = []
        self._actuators: List[Actuator] = []
        self._gravity = np.array([0.0, 0.0, -GRAVITY])
        self._dt = 0.001

    def gravity(self, g) -> "ModelBuilder":
        self._gravity = _vec3(g)
        return self

    def dt(self, dt: float) -> "ModelBuilder":
        self._dt = float(dt)
        return self

    def add_body(self, name: str, parent: int, joint: Joint, inertia: SpatialInertia,
                 geometry: Optional[Geometry] = None) -> "ModelBuilder":
        self._bodies.append(Body(name, int(parent), joint, inertia, geometry))
        return self

    def add_revolute_body(self, name, parent, parent_to_joint, inertia, axis=(0.0, 0.0, 1.0), **kw):
        return self.add_body(name, parent, Joint(REVOLUTE, parent_to_joint, _vec3(axis), **kw), inertia)

    def add_prismatic_body(self, name, parent, parent_to_joint, axis, inertia, **kw):
        return self.add_body(name, parent, Joint(PRISMATIC, parent_to_joint, _vec3(axis), **kw), inertia)

    def add_spherical_body(self, name, parent, parent_to_joint, inertia, **kw):
        return self.add_body(name, parent, Joint(BALL, parent_to_joint, np.zeros(3), **kw), inertia)

    def add_actuator(self, actuator: Actuator) -> "ModelBuilder":
        self._actuators.append(actuator)
        return self

    def add_free_body(self, name, parent, parent_to_joint, inertia, geometry=None):
        return self.add_body(name, parent, Joint(FREE, parent_to_joint, np.zeros(3)), inertia, geometry)

    def add_fixed_body(self, name, parent, parent_to_joint, inertia, geometry=None):
        return self.add_body(name, parent, Joint(FIXED, parent_to_joint, np.zeros(3)), inertia, geometry)

    def build(self) -> Model:
        nq = nv = 0
        qo, vo = [], []
        for b in self._bodies:
            qo.append(nq)
            vo.append(nv)
            nq += b.joint.ndof()
            nv += b.joint.ndof()
        return Model(list(self._bodies), self._gravity.copy(), self._dt, nq, nv, qo, vo, list(self._actuators))


def pack_bodies(model: Model) -> np.ndarray:
    """Body table, nb x 36 f64, layout.rs:19-38 slot meanings (pack_bodies, layout.rs:103-156)."""
    nb = model.nbodies
    t = np.zeros((nb, BODY_STRIDE), dtype=np.float64)
    for i, b in enumerate(model.bodies):
        j = b.joint
        t[i, 0] = b.parent
        t[i, 1] = j.jtype
        t[i, 2] = model.q_offsets[i]
        t[i, 3] = model.v_offsets[i]
        t[i, 4] = b.inertia.mass
        t[i, 5:8] = b.inertia.com
        I = b.inertia.inertia
        t[i, 8:14] = [I[0, 0], I[1, 1], I[2, 2], I[0, 1], I[0, 2], I[1, 2]]
        t[i, 14:23] = j.parent_to_joint.rot.reshape(9)
        t[i, 23:26] = j.parent_to_joint.pos
        t[i, 26:29] = j.axis
        t[i, 29] = j.damping
        t[i, 30] = j.stiffness
        t[i, 31] = j.spring_ref
        t[i, 32] = j.armature
    return t


def pack_joint_terms(model: Model) -> np.ndarray:
    """Joint terms, nb x 8 f64: [limited, lo, hi, limit_k, limit_d, friction_loss, 0, 0]
    (an extension table: the reference's device body table has no such slots)."""
    t = np.zeros((model.nbodies, JOINT_TERMS_STRIDE), dtype=np.float64)
    for i, b in enumerate(model.bodies):
        j = b.joint
        lim = j.limits is not None and j.ndof() == 1
        t[i, 0] = 1.0 if lim else 0.0
        if lim:
            t[i, 1], t[i, 2] = j.limits
        t[i, 3], t[i, 4] = j.limit_stiffness, j.limit_damping
        t[i, 5] = j.friction_loss if j.ndof() == 1 else 0.0
    return t


def pack_actuators(model: Model) -> np.ndarray:
    """Actuators, nu x 16 f64: [body, gear, gain, bias_q, bias_v, has_ctrl_range,
    ctrl_lo, ctrl_hi, has_force_range, force_lo, force_hi, 0 ...]."""
    t = np.zeros((model.nu(), ACTUATOR_STRIDE), dtype=np.float64)
    for a, act in enumerate(model.actuators):
        t[a, 0:5] = [act.joint_idx, act.gear, act.gain, act.bias_q, act.bias_v]
        if act.ctrl_range is not None:
            t[a, 5:8] = [1.0, act.ctrl_range[0], act.ctrl_range[1]]
        if act.force_range is not None:
            t[a, 8:11] = [1.0, act.force_range[0], act.force_range[1]]
    return t


def pack_geometries(model: Model, stiffness: float = 0.0, damping: float = 0.0,
                    gains: Optional[Sequence] = None):
    """Geometry table, nb x 24 f64 (pack_geometries, layout.rs:182-280).

    Returns (table, collidable_count). `gains` is a per-body list of
    (stiffness, damping); otherwise the global pair is written to every body.
    """
    nb = model.nbodies
    g = np.zeros((nb, GEOM_STRIDE), dtype=np.float64)
    collidable = 0
    for i, b in enumerate(model.bodies):
        g[i, 13:22] = np.eye(3).reshape(9)
        geo = b.geometry
        if geo is not None and geo.kind != G_NONE:
            g[i, 10:13] = geo.origin.pos
            g[i, 13:22] = geo.origin.rot.reshape(9)
            g[i, 0] = geo.kind
            p = list(geo.params)
            g[i, 1:1 + len(p)] = p
            collidable += 1
        if gains is not None:
            g[i, 8], g[i, 9] = gains[i]
        else:
            g[i, 8], g[i, 9] = stiffness, damping
    return g, collidable


def model_from_tables(body: np.ndarray, geom: Optional[np.ndarray], gravity, dt: float, nq: int, nv: int,
                      joint_terms: Optional[np.ndarray] = None, actuators: Optional[np.ndarray] = None,
                      body_names: Optional[Sequence[str]] = None, joint_names: Optional[Sequence[str]] = None,
                      actuator_names: Optional[Sequence[str]] = None) -> Model:
    """The Model that pack_bodies / pack_geometries / pack_joint_terms /
    pack_actuators describe (their inverse, names optional)."""
    body = np.asarray(body, dtype=np.float64).reshape(-1, BODY_STRIDE)
    nb = body.shape[0]
    bodies, qo, vo = [], [], []
    for i in range(nb):
        r = body[i]
        I = np.array([[r[8], r[11], r[12]], [r[11], r[9], r[13]], [r[12], r[13], r[10]]])
        j = Joint(int(r[1]), SpatialTransform.new(r[14:23].reshape(3, 3), r[23:26]), r[26:29].copy(),
                  damping=float(r[29]), stiffness=float(r[30]), spring_ref=float(r[31]), armature=float(r[32]),
                  name="" if joint_names is None else str(joint_names[i]))
        if joint_terms is not None:
            t = np.asarray(joint_terms, dtype=np.float64).reshape(nb, JOINT_TERMS_STRIDE)[i]
            j.limits = (float(t[1]), float(t[2])) if t[0] != 0.0 else None
            j.limit_stiffness, j.limit_damping, j.friction_loss = float(t[3]), float(t[4]), float(t[5])
        geo = None
        if geom is not None:
            g = np.asarray(geom, dtype=np.float64).reshape(nb, GEOM_STRIDE)[i]
            if int(g[0]) != G_NONE:
                npar = {G_SPHERE: 1, G_BOX: 3, G_CAPSULE: 2, G_CYLINDER: 2, G_MESH: 6}[int(g[0])]
                geo = Geometry(int(g[0]), tuple(float(x) for x in g[1:1 + npar]),
                               SpatialTransform.new(g[13:22].reshape(3, 3), g[10:13]))
        name = f"body_{i}" if body_names is None else str(body_names[i])
        bodies.append(Body(name, int(r[0]), j, SpatialInertia.new(r[4], r[5:8], I), geo, [] if geo is None else [geo]))
        qo.append(int(r[2]))
        vo.append(int(r[3]))
    acts = []
    if actuators is not None:
        for a, r in enumerate(np.asarray(actuators, dtype=np.float64).reshape(-1, ACTUATOR_STRIDE)):
            jn = bodies[int(r[0])].joint.name
            acts.append(Actuator("" if actuator_names is None else str(actuator_names[a]), jn, int(r[0]), float(r[1]),
                                 (float(r[6]), float(r[7])) if r[5] != 0.0 else None, float(r[2]), float(r[3]),
                                 float(r[4]), (float(r[9]), float(r[10])) if r[8] != 0.0 else None))
    return Model(bodies, np.asarray(gravity, dtype=np.float64).copy(), float(dt), int(nq), int(nv), qo, vo, acts)


def uniform_frequency_gains(model: Model, omega: float, zeta: float):
    """BodyContactGains::uniform_frequency (contact_pipeline.rs:293-305): k = m w^2, d = 2 zeta m w."""
    return [(b.inertia.mass * omega * omega, 2.0 * zeta * b.inertia.mass * omega) for b in model.bodies]


@dataclasses.dataclass
class PdDof:
    q_index: int
    v_index: int
    kp: float
    kd: float
    max_force: float


def pack_pd_dofs(dofs: Sequence[PdDof]) -> np.ndarray:
    """PD table, n x 8 f64 (pack_pd_dofs, layout.rs:314-325)."""
    t = np.zeros((len(dofs), PD_DOF_STRIDE), dtype=np.float64)
    for i, d in enumerate(dofs):
        t[i, :5] = [d.q_index, d.v_index, d.kp, d.kd, d.max_force]
    return t


@dataclasses.dataclass
class BodyPlane:
    """A contact plane welded to a body: its local +Z face at `offset`, finite
    over +-half_x, +-half_y, reaching `max_depth` into the body; `exclude` lists
    bodies that never touch it (BodyPlane, crates/phyz-gpu/src/contact_pipeline.rs:300-353)."""
    body: int
    offset: float
    max_depth: float
    half_x: float
    half_y: float
    exclude: Sequence[int] = ()

    def row(self) -> np.ndarray:
        return np.array([self.body, self.offset, self.max_depth, self.half_x, self.half_y], dtype=np.float64)


@dataclasses.dataclass
class Heightfield:
    """Terrain nodes heights[iy][ix] at origin + (ix, iy) * cell, origin.z added
    to every height (phyz_model::Heightfield, crates/phyz-model/src/heightfield.rs)."""
    origin: Sequence[float]
    cell: float
    nx: int
    ny: int
    heights: np.ndarray

    def header(self) -> np.ndarray:
        return np.array([self.nx, self.ny, *self.origin, self.cell], dtype=np.float64)

    def nodes(self) -> np.ndarray:
        # Heights are f32 in the reference's type; carry exactly those values.
        return np.ascontiguousarray(np.asarray(self.heights, dtype=np.float32).astype(np.float64).ravel())

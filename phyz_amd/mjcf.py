"""MJCF (MuJoCo XML) models into phyz_amd Models, with phyz-mjcf's semantics.

Follows crates/phyz-mjcf/src (the reference loader) element by element:

* ``<default>`` classes with nesting and ``childclass`` inheritance
  (defaults.rs:1-120, parser.rs:401-426): an element's own attributes win over
  its class chain, nearer classes over further ones.
* ``<compiler angle eulerseq meshdir assetdir>``, ``<option gravity timestep>``
  (parser.rs:428-464). The angle unit defaults to radians, as in the reference.
  With ``angle="degree"``, joint ``range`` and every actuator's ``ctrlrange``
  are converted to radians after parsing (parser.rs:376-398).
* Orientation in any of ``quat``, ``axisangle``, ``euler``, ``xyaxes``,
  ``zaxis``, in that precedence (orientation.rs:47-113). A body's orientation
  matrix is used as the ``parent_to_joint`` rotation as written; a geom's goes
  in transposed (parser.rs:729, 828).
* Bodies with several joints become a chain of one-joint links: the first link
  carries the body's placement, the others are coincident, and every link but
  the last carries a 1e-9 placeholder inertia (parser.rs:735-790).
* Geom-derived inertia from ``density`` (default 1000) or ``mass``, summed with
  the parallel-axis theorem (inertia.rs); an explicit ``<inertial>`` wins.
  ``fromto`` gives a capsule/cylinder its centre, length and the minimal
  rotation taking +Z onto the segment (parser.rs:600-617).
* Collision geoms in document order; the body's contact shape is its first
  collision geom with its offset, which is what the device contacts through
  (layout.rs:195-208). ``contype="0" conaffinity="0"`` geoms are visual only.
* ``<motor|position|velocity|general joint=...>`` actuators with MuJoCo's
  affine law (parser.rs:638-692).
* ``<include file>`` spliced before parsing, nesting capped at 16 (include.rs).
* STL (binary and ASCII) and OBJ mesh assets (assets.rs); a mesh geom
  collides through its body-frame AABB, as in the device table.
* Tendons, equality constraints, heightfield assets, unknown joint types,
  actuators without a joint and unloadable meshes are reported in
  ``unsupported()``, never silently dropped.
"""
from __future__ import annotations

import dataclasses
import math
import os
import struct
import xml.etree.ElementTree as ET
from typing import Dict, List, Optional, Tuple

import numpy as np

from .model import (BALL, FIXED, FREE, PRISMATIC, REVOLUTE, Actuator, Body, Geometry, Joint, Model, ModelBuilder,
                    SpatialInertia, SpatialTransform, G_MESH, G_NONE)

ROOT_CLASS = ""
MAX_INCLUDE_DEPTH = 16
PLACEHOLDER_LINK = 1e-9


class MjcfError(ValueError):
    """Anything that can go wrong loading an MJCF model (lib.rs MjcfError)."""


def _invalid_attr(element: str, attribute: str, value: str, reason: str) -> MjcfError:
    return MjcfError(f"<{element}> attribute '{attribute}' has invalid value {value!r}: {reason}")


def _missing_attr(element: str, attribute: str) -> MjcfError:
    return MjcfError(f"<{element}> is missing required attribute '{attribute}'")


# ── attributes over class defaults (attrs.rs) ───────────────────────────────
class Attrs:
    def __init__(self, own: Dict[str, str], defaults: Optional[Dict[str, str]] = None):
        self.own = dict(own)
        self.defaults = dict(defaults or {})

    def get(self, key: str) -> Optional[str]:
        if key in self.own:
            return self.own[key]
        return self.defaults.get(key)

    def str_or(self, key: str, fallback: str) -> str:
        v = self.get(key)
        return fallback if v is None else v

    def f64(self, key: str) -> Optional[float]:
        v = self.get(key)
        if v is None:
            return None
        try:
            return float(v.strip())
        except ValueError:
            return None

    def f64_or(self, key: str, fallback: float) -> float:
        v = self.f64(key)
        return fallback if v is None else v

    def floats(self, key: str) -> Optional[List[float]]:
        v = self.get(key)
        if v is None:
            return None
        out = []
        for tok in v.split():
            try:
                out.append(float(tok))
            except ValueError:
                pass
        return out

    def vec3(self, key: str) -> Optional[np.ndarray]:
        v = self.floats(key)
        return np.array(v, dtype=np.float64) if v is not None and len(v) == 3 else None

    def vec3_or(self, key: str, fallback) -> np.ndarray:
        v = self.vec3(key)
        return np.array(fallback, dtype=np.float64) if v is None else v

    def range(self, key: str) -> Optional[Tuple[float, float]]:
        v = self.floats(key)
        return (v[0], v[1]) if v is not None and len(v) == 2 else None

    def bool(self, key: str) -> Optional[bool]:
        v = self.get(key)
        if v in ("true", "1"):
            return True
        if v in ("false", "0"):
            return False
        return None


# ── <default> class tree (defaults.rs) ──────────────────────────────────────
class DefaultsManager:
    def __init__(self):
        self.classes: Dict[str, Tuple[Optional[str], Dict[str, Dict[str, str]]]] = {ROOT_CLASS: (None, {})}

    def declare(self, name: str, parent: Optional[str]):
        by_tag = self.classes.get(name, (None, {}))[1]
        self.classes[name] = (parent, by_tag)

    def set(self, cls: str, tag: str, attrs: Dict[str, str]):
        if cls not in self.classes:
            self.classes[cls] = (None, {})
        self.classes[cls][1].setdefault(tag, {}).update(attrs)

    def has(self, cls: str) -> bool:
        return cls in self.classes

    def resolve(self, tag: str, cls: Optional[str]) -> Dict[str, str]:
        chain = []
        cursor = ROOT_CLASS if cls is None else cls
        guard = 0
        while cursor is not None and cursor in self.classes and guard <= 64:
            parent, by_tag = self.classes[cursor]
            chain.append(by_tag)
            cursor = parent
            guard += 1
        out: Dict[str, str] = {}
        for by_tag in reversed(chain):
            out.update(by_tag.get(tag, {}))
        return out


# ── orientation (orientation.rs) ────────────────────────────────────────────
@dataclasses.dataclass
class AngleConfig:
    degrees: bool = False
    eulerseq: str = "xyz"

    def to_radians(self, a: float) -> float:
        return math.radians(a) if self.degrees else a


def quat_to_matrix(w: float, x: float, y: float, z: float) -> np.ndarray:
    """Rotation of the unit quaternion (w, x, y, z) (active, Hamilton)."""
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def _quat_axis_angle(axis, angle: float) -> np.ndarray:
    h = 0.5 * angle
    s = math.sin(h)
    return np.array([math.cos(h), axis[0] * s, axis[1] * s, axis[2] * s])


def _quat_mul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    aw, ax, ay, az = a
    bw, bx, by, bz = b
    return np.array([aw * bw - ax * bx - ay * by - az * bz, aw * bx + ax * bw + ay * bz - az * by,
                     aw * by - ax * bz + ay * bw + az * bx, aw * bz + ax * by - ay * bx + az * bw])


def rotation_z_to(d: np.ndarray) -> np.ndarray:
    """Minimal rotation taking +Z onto the unit vector d; antiparallel: pi about X."""
    c = float(d[2])
    if c > 1.0 - 1e-12:
        return np.eye(3)
    if c < -1.0 + 1e-12:
        return quat_to_matrix(*_quat_axis_angle([1.0, 0.0, 0.0], math.pi))
    axis = np.cross([0.0, 0.0, 1.0], d)
    axis = axis / np.linalg.norm(axis)
    return quat_to_matrix(*_quat_axis_angle(axis, math.acos(max(-1.0, min(1.0, c)))))


def _expect_n(element: str, key: str, v: List[float], n: int) -> List[float]:
    if len(v) != n:
        raw = " ".join(str(x) for x in v)
        raise _invalid_attr(element, key, raw, f"expected {n} numbers, found {len(v)}")
    return v


def parse_orientation(a: Attrs, element: str, cfg: AngleConfig) -> Optional[np.ndarray]:
    """The element's rotation matrix from quat / axisangle / euler / xyaxes / zaxis
    (that precedence), or None when it states no orientation."""
    v = a.floats("quat")
    if v is not None:
        q = np.array(_expect_n(element, "quat", v, 4))
        n = np.linalg.norm(q)
        if n < 1e-12:
            raise _invalid_attr(element, "quat", a.get("quat") or "", "quaternion has zero norm")
        return quat_to_matrix(*(q / n))
    v = a.floats("axisangle")
    if v is not None:
        aa = _expect_n(element, "axisangle", v, 4)
        axis = np.array(aa[:3])
        n = np.linalg.norm(axis)
        if n < 1e-12:
            raise _invalid_attr(element, "axisangle", a.get("axisangle") or "", "rotation axis is the zero vector")
        return quat_to_matrix(*_quat_axis_angle(axis / n, cfg.to_radians(aa[3])))
    v = a.floats("euler")
    if v is not None:
        e = _expect_n(element, "euler", v, 3)
        q = np.array([1.0, 0.0, 0.0, 0.0])
        for i, ch in enumerate(cfg.eulerseq):
            axis = {"x": [1.0, 0.0, 0.0], "y": [0.0, 1.0, 0.0], "z": [0.0, 0.0, 1.0]}.get(ch.lower())
            if axis is None:
                raise _invalid_attr("compiler", "eulerseq", cfg.eulerseq, f"'{ch}' is not one of x/y/z/X/Y/Z")
            step = _quat_axis_angle(axis, cfg.to_radians(e[i]))
            # lower case: about the moving (intrinsic) frame; upper case: the fixed frame
            q = _quat_mul(q, step) if ch.islower() else _quat_mul(step, q)
        return quat_to_matrix(*(q / np.linalg.norm(q)))
    v = a.floats("xyaxes")
    if v is not None:
        xy = _expect_n(element, "xyaxes", v, 6)
        raw = a.get("xyaxes") or ""
        x = np.array(xy[:3])
        if np.linalg.norm(x) < 1e-12:
            raise _invalid_attr(element, "xyaxes", raw, "x axis is the zero vector")
        x = x / np.linalg.norm(x)
        y = np.array(xy[3:]) - x * np.dot(x, xy[3:])
        if np.linalg.norm(y) < 1e-12:
            raise _invalid_attr(element, "xyaxes", raw, "y axis is parallel to the x axis")
        y = y / np.linalg.norm(y)
        return np.column_stack([x, y, np.cross(x, y)])
    v = a.floats("zaxis")
    if v is not None:
        z = np.array(_expect_n(element, "zaxis", v, 3))
        n = np.linalg.norm(z)
        if n < 1e-12:
            raise _invalid_attr(element, "zaxis", a.get("zaxis") or "", "z axis is the zero vector")
        return rotation_z_to(z / n)
    return None


# ── geom mass properties (inertia.rs) ───────────────────────────────────────
def shape_volume(kind: str, size: List[float]) -> float:
    if kind == "sphere":
        return 4.0 / 3.0 * math.pi * size[0] ** 3
    if kind == "capsule":
        r, h = size[0], size[1]
        return math.pi * r * r * (2.0 * h) + 4.0 / 3.0 * math.pi * r ** 3
    if kind == "cylinder":
        return math.pi * size[0] ** 2 * (2.0 * size[1])
    if kind == "box":
        return 8.0 * size[0] * size[1] * size[2]
    raise ValueError(kind)


def shape_principal_inertia(kind: str, size: List[float], mass: float) -> np.ndarray:
    """Principal moments about the shape's centre (local Z the symmetry axis)."""
    if kind == "sphere":
        i = 0.4 * mass * size[0] ** 2
        return np.array([i, i, i])
    if kind == "box":
        x, y, z = size[:3]
        return np.array([mass / 3.0 * (y * y + z * z), mass / 3.0 * (x * x + z * z), mass / 3.0 * (x * x + y * y)])
    if kind == "cylinder":
        r, hh = size[0], size[1]
        h = 2.0 * hh
        ixx = mass * (3.0 * r * r + h * h) / 12.0
        return np.array([ixx, ixx, 0.5 * mass * r * r])
    if kind == "capsule":
        # Mass split between the shaft and the two hemispherical caps by volume;
        # a hemisphere's moment about its own centroid is 83/320 m r^2 and the
        # centroid sits 3r/8 beyond the shaft end.
        r, hl = size[0], size[1]
        v_cyl = math.pi * r * r * (2.0 * hl)
        v_cap = 2.0 / 3.0 * math.pi * r ** 3
        total = v_cyl + 2.0 * v_cap
        if total <= 0.0:
            return np.zeros(3)
        rho = mass / total
        m_cyl, m_cap = rho * v_cyl, rho * v_cap
        h = 2.0 * hl
        izz = 0.5 * m_cyl * r * r + 2.0 * (0.4 * m_cap * r * r)
        d = hl + 3.0 / 8.0 * r
        cap_ixx = 83.0 / 320.0 * m_cap * r * r + m_cap * d * d
        ixx = m_cyl * (3.0 * r * r + h * h) / 12.0 + 2.0 * cap_ixx
        return np.array([ixx, ixx, izz])
    raise ValueError(kind)


def combine_mass_props(parts: List[Tuple[float, np.ndarray, np.ndarray]]) -> Optional[SpatialInertia]:
    """Masses add, the COM is the mass-weighted mean, inertias shift to it by the
    parallel-axis theorem. parts: (mass, com, inertia about own com), body frame."""
    total = sum(p[0] for p in parts)
    if total <= 0.0:
        return None
    com = sum(p[0] * p[1] for p in parts) / total
    I = np.zeros((3, 3))
    for m, c, Ic in parts:
        d = c - com
        I = I + Ic + m * (np.dot(d, d) * np.eye(3) - np.outer(d, d))
    return SpatialInertia.new(total, com, I)


# ── meshes (assets.rs) ──────────────────────────────────────────────────────
@dataclasses.dataclass
class MeshAsset:
    name: str
    file: Optional[str]
    resolved_path: Optional[str]
    scale: np.ndarray
    vertices: Optional[np.ndarray] = None  # (n, 3)
    faces: Optional[np.ndarray] = None     # (m, 3)
    load_error: Optional[str] = None


def _load_stl(data: bytes):
    if len(data) >= 84:
        n = struct.unpack_from("<I", data, 80)[0]
        if 84 + n * 50 == len(data):
            verts = np.zeros((3 * n, 3))
            for i in range(n):
                base = 84 + i * 50 + 12  # skip the facet normal
                verts[3 * i:3 * i + 3] = np.array(struct.unpack_from("<9f", data, base)).reshape(3, 3)
            return verts, np.arange(3 * n).reshape(n, 3)
    if data.startswith(b"solid"):
        verts, faces, pending = [], [], []
        for lineno, line in enumerate(data.decode("utf-8").splitlines(), 1):
            line = line.strip()
            if line.startswith("vertex"):
                nums = line[len("vertex"):].split()
                if len(nums) != 3:
                    raise ValueError(f"line {lineno}: vertex needs 3 numbers")
                verts.append([float(x) for x in nums])
                pending.append(len(verts) - 1)
            elif line.startswith("endfacet"):
                if len(pending) == 3:
                    faces.append(pending)
                pending = []
        if not faces:
            raise ValueError("no facets found")
        return np.array(verts), np.array(faces)
    raise ValueError("file is neither a valid binary nor ASCII STL")


def _load_obj(text: str):
    verts, faces = [], []
    for lineno, line in enumerate(text.splitlines(), 1):
        line = line.strip()
        if line.startswith("v "):
            nums = line[2:].split()[:3]
            if len(nums) != 3:
                raise ValueError(f"line {lineno}: vertex needs 3 numbers")
            verts.append([float(x) for x in nums])
        elif line.startswith("f "):
            idx = []
            for tok in line[2:].split():
                k = int(tok.split("/")[0])
                idx.append(k - 1 if k > 0 else len(verts) + k)
            for t in range(1, len(idx) - 1):  # fan
                faces.append([idx[0], idx[t], idx[t + 1]])
    if not verts:
        raise ValueError("no vertices found")
    return np.array(verts), np.array(faces, dtype=np.int64).reshape(-1, 3)


def load_mesh_file(path: str):
    ext = os.path.splitext(path)[1].lower().lstrip(".")
    if ext == "stl":
        with open(path, "rb") as f:
            return _load_stl(f.read())
    if ext == "obj":
        with open(path) as f:
            return _load_obj(f.read())
    raise ValueError(f"unsupported mesh format '{ext}' for {path} (STL and OBJ are supported)")


# ── parsed elements ─────────────────────────────────────────────────────────
@dataclasses.dataclass
class UnsupportedFeature:
    tag: str
    detail: str


@dataclasses.dataclass
class SensorElement:
    name: str
    kind: str
    target: str


@dataclasses.dataclass
class _JointEl:
    name: str
    jtype: int
    pos: np.ndarray
    axis: np.ndarray
    range: Optional[Tuple[float, float]]
    limited: Optional[bool]
    damping: float
    armature: float
    stiffness: float
    spring_ref: float
    friction_loss: float


@dataclasses.dataclass
class _GeomEl:
    name: str
    kind: str
    size: List[float]
    pos: np.ndarray
    rot: np.ndarray  # geom -> body
    density: float
    mass: Optional[float]
    collides: bool
    mesh: Optional[str]
    friction: Optional[float]

    def mass_props(self):
        if self.kind not in ("sphere", "capsule", "cylinder", "box"):
            return None
        need = {"sphere": 1, "capsule": 2, "cylinder": 2, "box": 3}[self.kind]
        if len(self.size) < need:
            return None
        m = self.mass if self.mass is not None else self.density * shape_volume(self.kind, self.size)
        I = self.rot @ np.diag(shape_principal_inertia(self.kind, self.size, m)) @ self.rot.T
        return (m, self.pos.copy(), I)


@dataclasses.dataclass
class _BodyEl:
    name: str
    pos: np.ndarray
    rot: np.ndarray
    parent: Optional[int]
    childclass: Optional[str]
    inertial: Optional[SpatialInertia] = None
    joints: List[_JointEl] = dataclasses.field(default_factory=list)
    geoms: List[_GeomEl] = dataclasses.field(default_factory=list)


@dataclasses.dataclass
class _ActEl:
    name: str
    joint_name: str
    gear: float
    ctrl_range: Optional[Tuple[float, float]]
    force_range: Optional[Tuple[float, float]]
    gain: float
    bias_q: float
    bias_v: float


_JOINT_TYPES = {"hinge": REVOLUTE, "slide": PRISMATIC, "ball": BALL, "free": FREE}


class MjcfLoader:
    """MJCF loader with the reference's surface (parser.rs MjcfLoader):
    from_file / from_xml_str, build_model(), unsupported(), sensors(),
    meshes(), armature_joints()."""

    def __init__(self, xml: str, model_dir: Optional[str]):
        self.defaults = DefaultsManager()
        self.bodies: List[_BodyEl] = []
        self.actuators: List[_ActEl] = []
        self._sensors: List[SensorElement] = []
        self._meshes: List[MeshAsset] = []
        self._unsupported: List[UnsupportedFeature] = []
        self.gravity = np.array([0.0, 0.0, -9.81])
        self.timestep = 0.002
        self.angles = AngleConfig()
        self.coordinate = "local"
        self.model_dir = model_dir
        self.meshdir: Optional[str] = None
        root = _expand_includes(xml, model_dir, 0)
        self._walk(root, default_cls=None, body=None, section=None)
        if self.angles.degrees:
            for b in self.bodies:
                for j in b.joints:
                    if j.range is not None:
                        j.range = (math.radians(j.range[0]), math.radians(j.range[1]))
            for a in self.actuators:
                if a.ctrl_range is not None:
                    a.ctrl_range = (math.radians(a.ctrl_range[0]), math.radians(a.ctrl_range[1]))

    @staticmethod
    def from_file(path: str) -> "MjcfLoader":
        with open(path) as f:
            xml = f.read()
        return MjcfLoader(xml, os.path.dirname(os.path.abspath(path)))

    @staticmethod
    def from_xml_str(xml: str) -> "MjcfLoader":
        return MjcfLoader(xml, None)

    def unsupported(self) -> List[UnsupportedFeature]:
        return list(self._unsupported)

    def sensors(self) -> List[SensorElement]:
        return list(self._sensors)

    def meshes(self) -> List[MeshAsset]:
        return list(self._meshes)

    def armature_joints(self) -> List[str]:
        return [j.name for b in self.bodies for j in b.joints if j.armature != 0.0]

    def _note(self, tag: str, detail: str):
        f = UnsupportedFeature(tag, detail)
        if f not in self._unsupported:
            self._unsupported.append(f)

    # ── document walk ──
    def _walk(self, el: ET.Element, default_cls: Optional[str], body: Optional[int], section: Optional[str]):
        for child in el:
            if not isinstance(child.tag, str):
                continue  # comments
            tag = child.tag
            if tag == "default":
                name = child.get("class", ROOT_CLASS)
                self.defaults.declare(name, default_cls)
                self._walk(child, name, body, section)
                continue
            if default_cls is not None:
                self.defaults.set(default_cls, tag, dict(child.attrib))
                continue
            if tag == "compiler":
                self._parse_compiler(child)
            elif tag == "option":
                a = Attrs(child.attrib)
                g = a.vec3("gravity")
                if g is not None:
                    self.gravity = g
                self.timestep = a.f64_or("timestep", self.timestep)
            elif tag in ("worldbody", "actuator", "sensor", "asset"):
                self._walk(child, None, None, tag)
            elif tag == "mesh" and section == "asset":
                self._parse_mesh(child)
            elif tag == "hfield" and section == "asset":
                self._note("hfield", "heightfields are parsed but phyz-collision has no heightfield shape, "
                                     "so the geom is dropped")
            elif tag == "equality":
                self._note("equality", "equality constraints are ignored; closed kinematic loops will behave as "
                                       "open chains")
            elif tag == "tendon":
                self._note("tendon", "tendons are ignored; coupled joints move independently")
            elif tag == "body" and section == "worldbody":
                idx = self._parse_body(child, body)
                self._walk(child, None, idx, section)
            elif tag in ("joint", "freejoint") and section == "worldbody" and body is not None:
                self._parse_joint(child, body, tag)
            elif tag == "inertial" and section == "worldbody" and body is not None:
                self._parse_inertial(child, body)
            elif tag == "geom" and section == "worldbody" and body is not None:
                self._parse_geom(child, body)
            elif tag in ("motor", "position", "velocity", "general") and section == "actuator":
                self._parse_actuator(child, tag)
            elif section == "sensor":
                a = Attrs(child.attrib)
                target = a.get("joint") or a.get("site") or a.get("body") or a.get("objname") or ""
                self._sensors.append(SensorElement(a.str_or("name", f"{tag}_{target}"), tag, target))
            else:
                self._walk(child, None, body, section)

    def _attrs_for(self, el: ET.Element, tag: str, body: Optional[int]) -> Attrs:
        explicit = el.get("class")
        cls = explicit if explicit is not None else self._inherited_class(body)
        return Attrs(el.attrib, self.defaults.resolve(tag, cls))

    def _inherited_class(self, body: Optional[int]) -> Optional[str]:
        while body is not None:
            b = self.bodies[body]
            if b.childclass is not None:
                return b.childclass
            body = b.parent
        return None

    def _parse_compiler(self, el: ET.Element):
        a = Attrs(el.attrib)
        if a.get("angle") is not None:
            self.angles.degrees = a.get("angle") == "degree"
        seq = a.get("eulerseq")
        if seq is not None:
            if len(seq) != 3 or any(c not in "xyzXYZ" for c in seq):
                raise _invalid_attr("compiler", "eulerseq", seq, "expected exactly 3 characters from x/y/z/X/Y/Z")
            self.angles.eulerseq = seq
        if a.get("coordinate") is not None:
            self.coordinate = a.get("coordinate")
        if a.get("assetdir") is not None:
            self.meshdir = a.get("assetdir")
        if a.get("meshdir") is not None:
            self.meshdir = a.get("meshdir")

    def _asset_dir(self) -> Optional[str]:
        if self.model_dir is not None and self.meshdir is not None:
            return os.path.join(self.model_dir, self.meshdir)
        return self.model_dir if self.model_dir is not None else self.meshdir

    def _parse_mesh(self, el: ET.Element):
        a = Attrs(el.attrib)
        file = a.get("file")
        name = a.get("name")
        if name is None:
            if file is None:
                raise _missing_attr("mesh", "name")
            name = os.path.splitext(os.path.basename(file))[0]
        scale = a.vec3_or("scale", [1.0, 1.0, 1.0])
        d = self._asset_dir()
        path = None if file is None else (os.path.join(d, file) if d is not None else file)
        m = MeshAsset(name, file, path, scale)
        if path is None:
            m.load_error = "mesh has no 'file' attribute"
        else:
            try:
                v, f = load_mesh_file(path)
                m.vertices, m.faces = v * scale, f
            except (OSError, ValueError, UnicodeDecodeError, struct.error) as e:
                m.load_error = f"{path}: {e}"
        if m.load_error is not None:
            self._note("mesh", f"mesh '{m.name}' not loaded: {m.load_error}")
        self._meshes.append(m)

    def _parse_body(self, el: ET.Element, parent: Optional[int]) -> int:
        a = self._attrs_for(el, "body", parent)
        rot = parse_orientation(a, "body", self.angles)
        self.bodies.append(_BodyEl(a.str_or("name", f"body_{len(self.bodies)}"), a.vec3_or("pos", [0.0, 0.0, 0.0]),
                                   np.eye(3) if rot is None else rot, parent, a.get("childclass")))
        return len(self.bodies) - 1

    def _parse_joint(self, el: ET.Element, body: int, tag: str):
        a = self._attrs_for(el, tag, body)
        if tag == "freejoint":
            jt = FREE
        else:
            t = a.get("type") or "hinge"
            if t not in _JOINT_TYPES:
                self._note("joint", f"joint type '{t}' is unknown; treated as hinge")
            jt = _JOINT_TYPES.get(t, REVOLUTE)
        axis = a.vec3("axis")
        axis = np.array([0.0, 0.0, 1.0]) if axis is None else axis / np.linalg.norm(axis)
        limited = a.bool("limited")
        self.bodies[body].joints.append(_JointEl(
            a.str_or("name", f"joint_{body}"), jt, a.vec3_or("pos", [0.0, 0.0, 0.0]), axis,
            None if limited is False else a.range("range"), limited, a.f64_or("damping", 0.0),
            a.f64_or("armature", 0.0), a.f64_or("stiffness", 0.0), a.f64_or("springref", 0.0),
            a.f64_or("frictionloss", 0.0)))

    def _parse_inertial(self, el: ET.Element, body: int):
        a = self._attrs_for(el, "inertial", body)
        pos = a.vec3_or("pos", [0.0, 0.0, 0.0])
        mass = a.f64_or("mass", 1.0)
        full = a.floats("fullinertia")
        if full is not None and len(full) == 6:
            xx, yy, zz, xy, xz, yz = full
            I = np.array([[xx, xy, xz], [xy, yy, yz], [xz, yz, zz]])
        else:
            I = np.diag(a.vec3_or("diaginertia", [0.001, 0.001, 0.001]))
            q = a.floats("quat")
            if q is not None and len(q) == 4:
                qq = np.array(q) / np.linalg.norm(q)
                R = quat_to_matrix(*qq)
                I = R @ I @ R.T
        self.bodies[body].inertial = SpatialInertia.new(mass, pos, I)

    def _parse_geom(self, el: ET.Element, body: int):
        a = self._attrs_for(el, "geom", body)
        kind = a.str_or("type", "sphere")
        mesh = a.get("mesh")
        if kind == "mesh" or mesh is not None:
            named = mesh or ""
            if not any(m.name == named and m.vertices is not None for m in self._meshes):
                self._note("geom", "mesh geoms whose asset could not be loaded are dropped; the body loses that "
                                   "collision shape and its inertia contribution")
                return
        size = a.floats("size")
        size = [0.05] if size is None else size
        pos = a.vec3_or("pos", [0.0, 0.0, 0.0])
        rot = parse_orientation(a, "geom", self.angles)
        rot = np.eye(3) if rot is None else rot
        ft = a.floats("fromto")
        if ft is not None and len(ft) == 6:
            p0, p1 = np.array(ft[:3]), np.array(ft[3:])
            axis = p1 - p0
            length = math.sqrt(float(np.dot(axis, axis)))
            pos = 0.5 * (p0 + p1)
            size = [size[0] if size else 0.05, 0.5 * length]
            if length > 1e-12:
                rot = rotation_z_to(axis / length)
        collides = not (a.f64_or("contype", 1.0) == 0.0 and a.f64_or("conaffinity", 1.0) == 0.0)
        fr = a.floats("friction")
        self.bodies[body].geoms.append(_GeomEl(a.str_or("name", f"geom_{body}"), kind, size, pos, rot,
                                               a.f64_or("density", 1000.0), a.f64("mass"), collides, mesh,
                                               fr[0] if fr else None))

    def _parse_actuator(self, el: ET.Element, tag: str):
        a = self._attrs_for(el, tag, None)
        joint = a.str_or("joint", "")
        if not joint:
            self._note(tag, "actuator without a `joint` target (site/tendon actuators are not supported)")
            return
        g = a.floats("gear")
        gear = g[0] if g else 1.0
        kp = a.f64_or("kp", 1.0)
        kv = a.f64_or("kv", 0.0)
        if tag == "position":
            gain, bq, bv = kp, -kp, -kv
        elif tag == "velocity":
            gain, bq, bv = max(kv, 1.0), 0.0, -max(kv, 1.0)
        elif tag == "general":
            gp = a.floats("gainprm") or []
            bp = a.floats("biasprm") or []
            if gp or bp:
                gain = gp[0] if gp else 1.0
                bq = bp[1] if len(bp) > 1 else 0.0
                bv = bp[2] if len(bp) > 2 else 0.0
            else:
                gain, bq, bv = 1.0, 0.0, 0.0
        else:
            gain, bq, bv = 1.0, 0.0, 0.0
        name = a.get("name") or f"{tag}_{joint}"
        self.actuators.append(_ActEl(name, joint, gear, a.range("ctrlrange"), a.range("forcerange"), gain, bq, bv))

    # ── model ──
    def _body_inertia(self, b: _BodyEl) -> SpatialInertia:
        if b.inertial is not None:
            return b.inertial
        parts = [p for p in (g.mass_props() for g in b.geoms) if p is not None]
        I = combine_mass_props(parts) if parts else None
        if I is not None:
            return I
        return SpatialInertia.new(1.0, np.zeros(3), np.diag([0.001, 0.001, 0.001]))

    def _geometry(self, g: _GeomEl) -> Optional[Geometry]:
        s = g.size
        origin = SpatialTransform.new(g.rot.T, g.pos)
        if g.kind == "mesh" or g.mesh is not None:
            m = next((m for m in self._meshes if m.name == g.mesh and m.vertices is not None), None)
            if m is None or len(m.vertices) == 0:
                return None
            return Geometry(G_MESH, tuple(m.vertices.min(axis=0)) + tuple(m.vertices.max(axis=0)), origin)
        if g.kind == "sphere":
            return Geometry.sphere(s[0] if s else 0.05, origin)
        if g.kind == "capsule":
            return Geometry.capsule(s[0] if s else 0.05, (s[1] if len(s) > 1 else 0.05) * 2.0, origin)
        if g.kind == "cylinder":
            return Geometry.cylinder(s[0] if s else 0.05, (s[1] if len(s) > 1 else 0.05) * 2.0, origin)
        if g.kind == "box":
            return Geometry.box(s[:3] if len(s) >= 3 else (0.05, 0.05, 0.05), origin)
        if g.kind == "plane":
            # Kept in the collision list (it can be a body's first collision
            # geom); it never contacts the ground, so it packs as no shape.
            return Geometry(G_NONE, (), origin)
        return None

    def build_model(self) -> Model:
        bld = ModelBuilder().gravity(self.gravity).dt(self.timestep)
        body_map: Dict[int, int] = {}
        joint_map: Dict[str, int] = {}
        nxt = 0
        for bi, b in enumerate(self.bodies):
            parent = body_map.get(b.parent, -1) if b.parent is not None else -1
            placement = SpatialTransform.new(b.rot, b.pos)
            inertia = self._body_inertia(b)
            if not b.joints:
                bld.add_fixed_body(b.name, parent, placement, inertia)
                body_map[bi] = nxt
                nxt += 1
                continue
            last = len(b.joints) - 1
            for k, je in enumerate(b.joints):
                base = placement if k == 0 else SpatialTransform.identity()
                ptj = base.compose(SpatialTransform.from_translation(je.pos))
                j = Joint(je.jtype, ptj, je.axis.copy(),
                          damping=je.damping, stiffness=je.stiffness, spring_ref=je.spring_ref,
                          armature=je.armature, limits=None if je.limited is False else je.range,
                          friction_loss=je.friction_loss, name=je.name)
                link_inertia = inertia if k == last else SpatialInertia.new(
                    PLACEHOLDER_LINK, np.zeros(3), np.eye(3) * PLACEHOLDER_LINK)
                joint_map[je.name] = nxt
                bld.add_body(b.name if len(b.joints) == 1 else f"{b.name}_{k}", parent if k == 0 else nxt - 1, j,
                             link_inertia)
                if k == last:
                    body_map[bi] = nxt
                nxt += 1
        model = bld.build()
        for bi, b in enumerate(self.bodies):
            mb = model.bodies[body_map[bi]]
            for g in b.geoms:
                geo = self._geometry(g)
                if geo is not None and g.collides:
                    mb.collisions.append(geo)
            mb.geometry = mb.collisions[0] if mb.collisions else None
        for a in self.actuators:
            if a.joint_name in joint_map:
                model.actuators.append(Actuator(a.name, a.joint_name, joint_map[a.joint_name], a.gear, a.ctrl_range,
                                                a.gain, a.bias_q, a.bias_v, a.force_range))
        return model


def _expand_includes(xml: str, model_dir: Optional[str], depth: int) -> ET.Element:
    """Parse and splice every <include file> (the children of the included
    file's root take its place), depth-first, at most 16 levels deep."""
    try:
        root = ET.fromstring(xml)
    except ET.ParseError as e:
        raise MjcfError(f"XML parse error: {e}") from None
    _splice(root, model_dir, depth)
    return root


def _splice(el: ET.Element, model_dir: Optional[str], depth: int):
    i = 0
    while i < len(el):
        child = el[i]
        if child.tag == "include":
            file = child.get("file")
            if file is None:
                raise _missing_attr("include", "file")
            if depth + 1 >= MAX_INCLUDE_DEPTH:
                raise MjcfError(f"Invalid MJCF: <include> nesting exceeded {MAX_INCLUDE_DEPTH} levels at '{file}'; "
                                "the includes are probably cyclic")
            path = os.path.join(model_dir, file) if model_dir is not None else file
            try:
                with open(path) as f:
                    content = f.read()
            except OSError as e:
                raise MjcfError(f"Invalid MJCF: <include file=\"{file}\"> could not be read: {e}") from None
            sub = _expand_includes(content, os.path.dirname(os.path.abspath(path)), depth + 1)
            el.remove(child)
            for k, c in enumerate(list(sub)):
                el.insert(i + k, c)
            i += len(sub)
            continue
        _splice(child, model_dir, depth)
        i += 1

"""MJCF (MuJoCo XML) models as phyz_amd Models.

The element semantics are phyz-mjcf's (crates/phyz-mjcf/src, element handling
in parser.rs:300-800): what a model file means has to come out the same. The
code is organised around this build's needs, in three stages:

1. Read. `_DefaultTables` flattens every ``<default>`` class into one
   attribute table per element tag before anything else is read (a class's
   table is its parent's overlaid with its own settings, so a lookup is a
   dictionary read, not a walk up the class chain). `_Reader` then walks the
   document once: each element's attributes are its class table overlaid with
   its own, converted by the per-tag schema `_SCHEMA`, and land in flat
   records (`_BodyRec`, `_JointRec`, `_GeomRec`, `_ActuatorRec`).
2. Mass and frames. Every orientation spelling becomes a unit quaternion and
   then one rotation matrix (`_orientation`). A body's mass properties come
   from an explicit ``<inertial>`` or from its geoms through `_MassSum`.
3. Assemble (`build_model`). Each body becomes one link per joint (a body with
   several joints is a chain of coincident links, all but the last with a
   1e-9 placeholder mass), then actuators bind to their joint's link.

Supported: default classes with nesting and childclass; ``<compiler angle
eulerseq>`` (with ``angle="degree"`` joint ranges and actuator ctrlranges are
converted to radians); ``<option gravity timestep>``; quat / axisangle /
euler / xyaxes / zaxis orientations (that precedence); ``fromto``; geom-
derived inertia (density or mass) or an explicit inertial; hinge, slide, ball
and free joints with limits, damping, armature, stiffness, springref and
frictionloss; motor, position, velocity and general actuators on joints;
sensors (recorded, not simulated); ``<include file>`` (spliced into the tree
before anything is read, paths relative to the including file, nesting capped
at 16 levels, which also stops cycles: include.rs); ``<asset><mesh>`` from
binary or ASCII STL and OBJ files, resolved through ``<compiler meshdir>`` (or
``assetdir``) against the model's directory, scaled per axis (assets.rs;
meshes()). A mesh geom whose asset loaded collides through its body-frame
bounding box, as the device's geometry table carries meshes (layout.rs:241-
257), and adds no mass, as in the reference. Reported by unsupported() and
skipped: meshes that do not load (and geoms that use them), heightfield
assets, tendons, equality constraints, unknown joint types and actuators
without a joint.
"""
from __future__ import annotations

import dataclasses
import math
import os
import struct
import xml.etree.ElementTree as ET
from typing import Dict, Iterator, List, Optional, Tuple

import numpy as np

from .model import (BALL, FIXED, FREE, PRISMATIC, REVOLUTE, Actuator, Geometry, Joint, Model, ModelBuilder,
                    SpatialInertia, SpatialTransform, G_NONE)

PLACEHOLDER_MASS = 1e-9  # mass and inertia of the leading links of a multi-joint body
MAX_INCLUDE_DEPTH = 16


class MjcfError(ValueError):
    """A model file that cannot be read."""


# ── attribute values ────────────────────────────────────────────────────────
def _number(text: Optional[str]) -> Optional[float]:
    if text is None:
        return None
    try:
        return float(text.strip())
    except ValueError:
        return None


def _numbers(text: Optional[str]) -> Optional[List[float]]:
    """Whitespace-separated numbers; tokens that are not numbers are skipped."""
    if text is None:
        return None
    out = []
    for tok in text.split():
        x = _number(tok)
        if x is not None:
            out.append(x)
    return out


def _flag(text: Optional[str]) -> Optional[bool]:
    return {"true": True, "1": True, "false": False, "0": False}.get(text) if text is not None else None


# A kind per attribute: "num" one number, "nums" any count, "v3" exactly
# three (else unset), "pair" exactly two, "flag" a boolean, "str" raw text.
_ORIENT = {"quat": "nums", "axisangle": "nums", "euler": "nums", "xyaxes": "nums", "zaxis": "nums"}
_SCHEMA: Dict[str, Dict[str, str]] = {
    "body": {"name": "str", "pos": "v3", "childclass": "str", **_ORIENT},
    "joint": {"name": "str", "type": "str", "pos": "v3", "axis": "v3", "range": "pair", "limited": "flag",
              "damping": "num", "armature": "num", "stiffness": "num", "springref": "num", "frictionloss": "num"},
    "inertial": {"pos": "v3", "mass": "num", "diaginertia": "v3", "fullinertia": "nums", "quat": "nums"},
    "geom": {"name": "str", "type": "str", "size": "nums", "pos": "v3", "fromto": "nums", "density": "num",
             "mass": "num", "contype": "num", "conaffinity": "num", "mesh": "str", **_ORIENT},
    "actuator": {"name": "str", "joint": "str", "gear": "nums", "ctrlrange": "pair", "forcerange": "pair",
                 "kp": "num", "kv": "num", "gainprm": "nums", "biasprm": "nums"},
    "mesh": {"name": "str", "file": "str", "scale": "v3"},
}
_SCHEMA["freejoint"] = _SCHEMA["joint"]
_CONVERT = {
    "num": _number,
    "nums": _numbers,
    "v3": lambda t: (lambda v: np.array(v) if v is not None and len(v) == 3 else None)(_numbers(t)),
    "pair": lambda t: (lambda v: (v[0], v[1]) if v is not None and len(v) == 2 else None)(_numbers(t)),
    "flag": _flag,
    "str": lambda t: t,
}
_ACTUATOR_TAGS = ("motor", "position", "velocity", "general")


def _typed(tag: str, raw: Dict[str, str]) -> Dict[str, object]:
    """Convert the attributes the schema knows; others are dropped."""
    schema = _SCHEMA["actuator" if tag in _ACTUATOR_TAGS else tag]
    out = {}
    for key, text in raw.items():
        kind = schema.get(key)
        if kind is not None:
            out[key] = _CONVERT[kind](text)
    return out


# ── default classes ─────────────────────────────────────────────────────────
class _DefaultTables:
    """Every class's effective default attributes per element tag. The
    unnamed top-level class is the root; a nested class inherits from the
    class it is written in, whatever the order of settings within it."""

    ROOT = ""

    def __init__(self, doc: ET.Element):
        self.parent: Dict[str, Optional[str]] = {self.ROOT: None}
        self.own: Dict[str, Dict[str, Dict[str, str]]] = {self.ROOT: {}}
        for el in doc:
            if el.tag == "default":
                self._collect(el, None)
        self.table: Dict[str, Dict[str, Dict[str, str]]] = {}
        for cls in self.own:
            self._flatten(cls, 0)

    def _collect(self, el: ET.Element, parent: Optional[str]):
        cls = el.get("class", self.ROOT)
        self.parent[cls] = parent
        settings = self.own.setdefault(cls, {})
        for child in el:
            if not isinstance(child.tag, str):
                continue
            if child.tag == "default":
                self._collect(child, cls)
            else:
                settings.setdefault(child.tag, {}).update(child.attrib)

    def _flatten(self, cls: str, depth: int) -> Dict[str, Dict[str, str]]:
        if cls in self.table:
            return self.table[cls]
        up = self.parent.get(cls)
        base = self._flatten(up, depth + 1) if up is not None and depth < 64 else {}
        merged = {tag: dict(attrs) for tag, attrs in base.items()}
        for tag, attrs in self.own.get(cls, {}).items():
            merged.setdefault(tag, {}).update(attrs)
        self.table[cls] = merged
        return merged

    def attrs(self, cls: Optional[str], tag: str, own: Dict[str, str]) -> Dict[str, str]:
        """The element's attributes: its class's defaults under its own."""
        base = self.table.get(self.ROOT if cls is None else cls, {}).get(tag, {})
        return {**base, **own}


# ── orientations (all through unit quaternions w, x, y, z) ──────────────────
def quat_to_matrix(w: float, x: float, y: float, z: float) -> np.ndarray:
    """Rotation matrix of the unit quaternion (w, x, y, z), active sense."""
    xx, yy, zz = x * x, y * y, z * z
    return np.array([[1 - 2 * (yy + zz), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (xx + zz), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (xx + yy)]])


def _quat_about(axis, angle: float) -> np.ndarray:
    return np.concatenate([[math.cos(0.5 * angle)], np.asarray(axis, dtype=np.float64) * math.sin(0.5 * angle)])


def _quat_product(a, b) -> np.ndarray:
    w = a[0] * b[0] - np.dot(a[1:], b[1:])
    v = a[0] * b[1:] + b[0] * a[1:] + np.cross(a[1:], b[1:])
    return np.concatenate([[w], v])


def _quat_z_onto(d: np.ndarray) -> np.ndarray:
    """The shortest rotation taking +Z onto the unit vector d (pi about X when
    d points down)."""
    cz = float(d[2])
    if cz > 1.0 - 1e-12:
        return np.array([1.0, 0.0, 0.0, 0.0])
    if cz < -1.0 + 1e-12:
        return _quat_about([1.0, 0.0, 0.0], math.pi)
    n = np.array([-d[1], d[0], 0.0])  # +Z x d
    return _quat_about(n / np.linalg.norm(n), math.acos(min(1.0, max(-1.0, cz))))


def _orientation(element: str, a: Dict[str, object], degrees: bool, eulerseq: str) -> Optional[np.ndarray]:
    """The rotation an element states, or None. One spelling counts, in the
    order quat, axisangle, euler, xyaxes, zaxis."""
    def bad(attr, why):
        return MjcfError(f"<{element} {attr}=...>: {why}")

    def need(attr, n):
        v = a[attr]
        if len(v) != n:
            raise bad(attr, f"needs {n} numbers, has {len(v)}")
        return np.array(v, dtype=np.float64)

    unit = math.radians if degrees else (lambda x: x)
    if a.get("quat") is not None:
        q = need("quat", 4)
        n = np.linalg.norm(q)
        if n < 1e-12:
            raise bad("quat", "a quaternion of zero norm has no rotation")
        return quat_to_matrix(*(q / n))
    if a.get("axisangle") is not None:
        v = need("axisangle", 4)
        n = np.linalg.norm(v[:3])
        if n < 1e-12:
            raise bad("axisangle", "the axis is the zero vector")
        return quat_to_matrix(*_quat_about(v[:3] / n, unit(v[3])))
    if a.get("euler") is not None:
        angles = need("euler", 3)
        q = np.array([1.0, 0.0, 0.0, 0.0])
        for ch, ang in zip(eulerseq, angles):
            step = _quat_about(np.eye(3)["xyz".index(ch.lower())], unit(ang))
            # lower case turns about the rotated frame's axis, upper case about the fixed one
            q = _quat_product(q, step) if ch.islower() else _quat_product(step, q)
        return quat_to_matrix(*(q / np.linalg.norm(q)))
    if a.get("xyaxes") is not None:
        v = need("xyaxes", 6)
        if np.linalg.norm(v[:3]) < 1e-12:
            raise bad("xyaxes", "the x axis is the zero vector")
        ex = v[:3] / np.linalg.norm(v[:3])
        ey = v[3:] - ex * np.dot(ex, v[3:])
        if np.linalg.norm(ey) < 1e-12:
            raise bad("xyaxes", "the y axis is parallel to the x axis")
        ey = ey / np.linalg.norm(ey)
        return np.column_stack([ex, ey, np.cross(ex, ey)])
    if a.get("zaxis") is not None:
        v = need("zaxis", 3)
        n = np.linalg.norm(v)
        if n < 1e-12:
            raise bad("zaxis", "the z axis is the zero vector")
        return quat_to_matrix(*_quat_z_onto(v / n))
    return None


# ── solid shapes ────────────────────────────────────────────────────────────
_SIZE_COUNT = {"sphere": 1, "capsule": 2, "cylinder": 2, "box": 3}


def shape_volume(kind: str, size: List[float]) -> float:
    """Volume of a solid given MJCF sizes (radius, half-length, half-extents)."""
    if kind == "sphere":
        return 4.0 / 3.0 * math.pi * size[0] ** 3
    if kind == "capsule":
        return math.pi * size[0] ** 2 * (2.0 * size[1] + 4.0 / 3.0 * size[0])
    if kind == "cylinder":
        return 2.0 * math.pi * size[0] ** 2 * size[1]
    if kind == "box":
        return 8.0 * size[0] * size[1] * size[2]
    raise ValueError(kind)


def shape_principal_inertia(kind: str, size: List[float], mass: float) -> np.ndarray:
    """Principal moments about the solid's centre, its local Z the symmetry axis."""
    if kind == "sphere":
        return np.full(3, 0.4 * mass * size[0] ** 2)
    if kind == "box":
        sq = np.asarray(size[:3], dtype=np.float64) ** 2
        return mass / 3.0 * (sq.sum() - sq)
    r, h = size[0], size[1]  # radius and half-length
    if kind == "cylinder":
        across = mass * (3.0 * r * r + 4.0 * h * h) / 12.0
        return np.array([across, across, 0.5 * mass * r * r])
    if kind == "capsule":
        # A shaft of length 2h and two hemispherical caps of the same density.
        # About a diameter of its flat face a solid hemisphere has 2/5 m r^2;
        # its centroid sits 3r/8 inside, so carried to the capsule's centre
        # (a distance h from the face) a cap adds m (2/5 r^2 + h^2 + 3/4 h r).
        v_shaft, v_cap = 2.0 * math.pi * r * r * h, 2.0 / 3.0 * math.pi * r ** 3
        if v_shaft + 2.0 * v_cap <= 0.0:
            return np.zeros(3)
        m_shaft = mass * v_shaft / (v_shaft + 2.0 * v_cap)
        m_cap = 0.5 * (mass - m_shaft)
        along = 0.5 * m_shaft * r * r + 2.0 * 0.4 * m_cap * r * r
        across = m_shaft * (3.0 * r * r + 4.0 * h * h) / 12.0 + 2.0 * m_cap * (0.4 * r * r + h * h + 0.75 * h * r)
        return np.array([across, across, along])
    raise ValueError(kind)


class _MassSum:
    """Mass properties of rigidly joined parts: masses add, the centre of mass
    is their weighted mean, inertias move to it by the parallel-axis theorem."""

    def __init__(self):
        self.parts: List[Tuple[float, np.ndarray, np.ndarray]] = []

    def add(self, mass: float, com: np.ndarray, inertia: np.ndarray):
        self.parts.append((mass, com, inertia))

    def total(self) -> Optional[SpatialInertia]:
        m = sum(p[0] for p in self.parts)
        if not self.parts or m <= 0.0:
            return None
        com = sum(p[0] * p[1] for p in self.parts) / m
        inertia = np.zeros((3, 3))
        for mi, ci, Ii in self.parts:
            d = ci - com
            inertia = inertia + Ii + mi * (np.dot(d, d) * np.eye(3) - np.outer(d, d))
        return SpatialInertia.new(m, com, inertia)


# ── includes (include.rs) ───────────────────────────────────────────────────
def _splice_includes(root: ET.Element, base_dir: Optional[str], depth: int = 0) -> ET.Element:
    """Replace every ``<include file>`` under `root` by the children of the
    named document's root element, in place and in order; the included
    document's own includes resolve against its directory."""
    for parent in list(root.iter()):
        kids = list(parent)
        if not any(isinstance(k.tag, str) and k.tag == "include" for k in kids):
            continue
        spliced: List[ET.Element] = []
        for k in kids:
            if not (isinstance(k.tag, str) and k.tag == "include"):
                spliced.append(k)
                continue
            name = k.get("file")
            if name is None:
                raise MjcfError("Invalid MJCF: <include> is missing required attribute 'file'")
            if depth + 1 >= MAX_INCLUDE_DEPTH:
                raise MjcfError(f"Invalid MJCF: <include> nesting exceeded {MAX_INCLUDE_DEPTH} levels at "
                                f"'{name}'; the includes are probably cyclic")
            path = name if base_dir is None else os.path.join(base_dir, name)
            try:
                with open(path) as f:
                    text = f.read()
            except OSError as e:
                raise MjcfError(f'Invalid MJCF: <include file="{name}"> could not be read: {e}') from None
            try:
                sub = ET.fromstring(text)
            except ET.ParseError as e:
                raise MjcfError(f'Invalid MJCF: <include file="{name}">: XML parse error: {e}') from None
            _splice_includes(sub, os.path.dirname(os.path.abspath(path)), depth + 1)
            spliced.extend(sub)
        parent[:] = spliced
    return root


# ── mesh assets (assets.rs) ─────────────────────────────────────────────────
@dataclasses.dataclass
class MeshAsset:
    """A ``<mesh>`` asset: `vertices` [n][3] (scaled) and `faces` [m][3], or
    None with the reason in `load_error`."""
    name: str
    file: Optional[str]
    resolved_path: Optional[str]
    scale: np.ndarray
    vertices: Optional[np.ndarray] = None
    faces: Optional[np.ndarray] = None
    load_error: Optional[str] = None


def _stl(data: bytes) -> Tuple[np.ndarray, np.ndarray]:
    """Binary STL when the size matches the header's facet count (80-byte
    header, u32 count, 50 bytes a facet), else ASCII when it starts 'solid'."""
    if len(data) >= 84:
        n = struct.unpack_from("<I", data, 80)[0]
        if 84 + 50 * n == len(data):
            rec = np.frombuffer(data, dtype=np.dtype([("normal", "<f4", 3), ("v", "<f4", (3, 3)), ("attr", "<u2")]),
                                count=n, offset=84)
            verts = rec["v"].reshape(-1, 3).astype(np.float64)
            return verts, np.arange(3 * n).reshape(n, 3)
    if not data.startswith(b"solid"):
        raise ValueError("file is neither a valid binary nor ASCII STL")
    verts, faces, facet = [], [], []
    for lineno, line in enumerate(data.decode("utf-8").splitlines(), start=1):
        words = line.split()
        if words[:1] == ["vertex"]:
            if len(words) != 4:
                raise ValueError(f"line {lineno}: vertex needs 3 numbers")
            facet.append(len(verts))
            verts.append([float(x) for x in words[1:]])
        elif words[:1] == ["endfacet"]:
            if len(facet) == 3:
                faces.append(facet)
            facet = []
    if not faces:
        raise ValueError("no facets found")
    return np.array(verts), np.array(faces)


def _obj(text: str) -> Tuple[np.ndarray, np.ndarray]:
    """OBJ 'v' and 'f' records; polygons fan into triangles; face indices
    1-based, negative ones counted back from the last vertex."""
    verts, faces = [], []
    for lineno, line in enumerate(text.splitlines(), start=1):
        words = line.split()
        if not words:
            continue
        if words[0] == "v":
            xyz = [float(x) for x in words[1:4]]
            if len(xyz) != 3:
                raise ValueError(f"line {lineno}: vertex needs 3 numbers")
            verts.append(xyz)
        elif words[0] == "f":
            idx = []
            for tok in words[1:]:
                k = int(tok.split("/")[0])
                if k == 0:
                    raise ValueError(f"line {lineno}: face index 0 is invalid")
                j = k - 1 if k > 0 else len(verts) + k
                if not 0 <= j < len(verts):
                    raise ValueError(f"line {lineno}: face index {k} out of range of {len(verts)} vertices")
                idx.append(j)
            faces.extend([idx[0], idx[t], idx[t + 1]] for t in range(1, len(idx) - 1))
    if not faces:
        raise ValueError("no faces found")
    return np.array(verts, dtype=np.float64), np.array(faces)


def load_mesh_file(path: str) -> Tuple[np.ndarray, np.ndarray]:
    """(vertices, faces) of an STL or OBJ file, by extension."""
    ext = os.path.splitext(path)[1][1:].lower()
    try:
        if ext == "stl":
            with open(path, "rb") as f:
                return _stl(f.read())
        if ext == "obj":
            with open(path) as f:
                return _obj(f.read())
    except (OSError, ValueError, UnicodeDecodeError) as e:
        raise ValueError(f"{path}: {e}") from None
    raise ValueError(f"unsupported mesh format '{ext}' for {path} (STL and OBJ are supported)")


# ── records ─────────────────────────────────────────────────────────────────
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
class _JointRec:
    name: str
    jtype: int
    pos: np.ndarray
    axis: np.ndarray
    limits: Optional[Tuple[float, float]]
    damping: float
    armature: float
    stiffness: float
    spring_ref: float
    friction_loss: float


@dataclasses.dataclass
class _GeomRec:
    kind: str
    size: List[float]
    pos: np.ndarray
    rot: np.ndarray  # geom frame -> body frame
    mass: float
    collides: bool
    mesh: Optional["MeshAsset"] = None  # a mesh geom's loaded asset


@dataclasses.dataclass
class _BodyRec:
    name: str
    parent: Optional[int]
    pos: np.ndarray
    rot: np.ndarray
    childclass: Optional[str]
    inertial: Optional[SpatialInertia] = None
    joints: List[_JointRec] = dataclasses.field(default_factory=list)
    geoms: List[_GeomRec] = dataclasses.field(default_factory=list)


@dataclasses.dataclass
class _ActuatorRec:
    name: str
    joint: str
    gear: float
    ctrl_range: Optional[Tuple[float, float]]
    force_range: Optional[Tuple[float, float]]
    gain: float
    bias_q: float
    bias_v: float


_JOINT_KIND = {"hinge": REVOLUTE, "slide": PRISMATIC, "ball": BALL, "free": FREE}

# Gain and biases of each actuator kind's affine law from kp, kv and the
# general kind's gainprm / biasprm (MuJoCo's actuator shortcuts).
def _actuator_law(tag: str, a: Dict[str, object]) -> Tuple[float, float, float]:
    kp = a.get("kp") if a.get("kp") is not None else 1.0
    kv = a.get("kv") if a.get("kv") is not None else 0.0
    if tag == "position":
        return kp, -kp, -kv
    if tag == "velocity":
        g = max(kv, 1.0)
        return g, 0.0, -g
    if tag == "general":
        gp, bp = a.get("gainprm") or [], a.get("biasprm") or []
        if gp or bp:
            return (gp[0] if gp else 1.0), (bp[1] if len(bp) > 1 else 0.0), (bp[2] if len(bp) > 2 else 0.0)
    return 1.0, 0.0, 0.0


# ── the document walk ───────────────────────────────────────────────────────
class _Reader:
    def __init__(self, doc: ET.Element, model_dir: Optional[str] = None):
        self.defaults = _DefaultTables(doc)
        self.model_dir = model_dir
        self.mesh_dir: Optional[str] = None
        self.meshes: List[MeshAsset] = []
        self.degrees = False
        self.eulerseq = "xyz"
        self.gravity = np.array([0.0, 0.0, -9.81])
        self.timestep = 0.002
        self.bodies: List[_BodyRec] = []
        self.actuators: List[_ActuatorRec] = []
        self.sensors: List[SensorElement] = []
        self.unsupported: List[UnsupportedFeature] = []
        for el in doc.iter("compiler"):
            self._compiler(el)
        for el in doc.iter("option"):
            g = _CONVERT["v3"](el.get("gravity"))
            if g is not None:
                self.gravity = g
            t = _number(el.get("timestep"))
            if t is not None:
                self.timestep = t
        self._top(doc)
        if self.degrees:  # ranges are written in degrees; the model works in radians
            for b in self.bodies:
                for j in b.joints:
                    if j.limits is not None:
                        j.limits = (math.radians(j.limits[0]), math.radians(j.limits[1]))
            for act in self.actuators:
                if act.ctrl_range is not None:
                    act.ctrl_range = (math.radians(act.ctrl_range[0]), math.radians(act.ctrl_range[1]))

    def note(self, tag: str, detail: str):
        f = UnsupportedFeature(tag, detail)
        if f not in self.unsupported:
            self.unsupported.append(f)

    def _compiler(self, el: ET.Element):
        if el.get("angle") is not None:
            self.degrees = el.get("angle") == "degree"
        # meshdir wins over the general assetdir, whatever their order.
        for key in ("assetdir", "meshdir"):
            if el.get(key) is not None and (key == "meshdir" or el.get("meshdir") is None):
                self.mesh_dir = el.get(key)
        seq = el.get("eulerseq")
        if seq is not None:
            if len(seq) != 3 or any(c not in "xyzXYZ" for c in seq):
                raise MjcfError(f"<compiler eulerseq={seq!r}>: three of x, y, z, X, Y, Z expected")
            self.eulerseq = seq

    def _children(self, el: ET.Element) -> Iterator[ET.Element]:
        return (c for c in el if isinstance(c.tag, str))

    def _top(self, el: ET.Element):
        for c in self._children(el):
            if c.tag == "worldbody":
                self._bodies_in(c, None)
            elif c.tag == "actuator":
                for a in self._children(c):
                    self._actuator(a)
            elif c.tag == "sensor":
                for s in self._children(c):
                    target = s.get("joint") or s.get("site") or s.get("body") or s.get("objname") or ""
                    self.sensors.append(SensorElement(s.get("name") or f"{s.tag}_{target}", s.tag, target))
            elif c.tag == "asset":
                for a in self._children(c):
                    if a.tag == "mesh":
                        self._mesh(a)
                    elif a.tag == "hfield":
                        self.note("hfield", "heightfield assets are not loaded; the ground is the contact "
                                            "pass's own plane or heightfield")
            elif c.tag == "tendon":
                self.note("tendon", "tendons are ignored; coupled joints move independently")
            elif c.tag == "equality":
                self.note("equality", "equality constraints are ignored; closed loops act as open chains")
            elif c.tag not in ("default", "compiler", "option"):
                self._top(c)

    def _asset_dir(self) -> Optional[str]:
        if self.model_dir is not None and self.mesh_dir is not None:
            return os.path.join(self.model_dir, self.mesh_dir)
        return self.model_dir if self.model_dir is not None else self.mesh_dir

    def _mesh(self, el: ET.Element):
        a = self._attrs(el, None)
        file = a.get("file")
        name = a.get("name") or (os.path.splitext(os.path.basename(file))[0] if file else None)
        if name is None:
            raise MjcfError("Invalid MJCF: <mesh> is missing required attribute 'name'")
        scale = a.get("scale") if a.get("scale") is not None else np.ones(3)
        d = self._asset_dir()
        path = None if file is None else (file if d is None else os.path.join(d, file))
        m = MeshAsset(name, file, path, np.asarray(scale, dtype=np.float64))
        if path is None:
            m.load_error = "mesh has no 'file' attribute"
        else:
            try:
                v, f = load_mesh_file(path)
                m.vertices, m.faces = v * m.scale, f
            except ValueError as e:
                m.load_error = str(e)
        if m.load_error is not None:
            self.note("mesh", f"mesh '{name}' not loaded: {m.load_error}")
        self.meshes.append(m)

    def _class_of(self, el: ET.Element, body: Optional[int]) -> Optional[str]:
        """An explicit class, else the nearest enclosing body's childclass."""
        if el.get("class") is not None:
            return el.get("class")
        while body is not None:
            if self.bodies[body].childclass is not None:
                return self.bodies[body].childclass
            body = self.bodies[body].parent
        return None

    def _attrs(self, el: ET.Element, body: Optional[int]) -> Dict[str, object]:
        tag = el.tag
        raw = self.defaults.attrs(self._class_of(el, body), tag, dict(el.attrib))
        return _typed(tag, raw)

    def _bodies_in(self, el: ET.Element, body: Optional[int]):
        for c in self._children(el):
            if c.tag == "body":
                a = self._attrs(c, body)
                rot = _orientation("body", a, self.degrees, self.eulerseq)
                self.bodies.append(_BodyRec(a.get("name") or f"body_{len(self.bodies)}", body,
                                            a["pos"] if a.get("pos") is not None else np.zeros(3),
                                            np.eye(3) if rot is None else rot, a.get("childclass")))
                self._bodies_in(c, len(self.bodies) - 1)
            elif body is not None and c.tag in ("joint", "freejoint"):
                self.bodies[body].joints.append(self._joint(c, body))
            elif body is not None and c.tag == "inertial":
                self.bodies[body].inertial = self._inertial(c, body)
            elif body is not None and c.tag == "geom":
                g = self._geom(c, body)
                if g is not None:
                    self.bodies[body].geoms.append(g)
            else:
                self._bodies_in(c, body)

    def _joint(self, el: ET.Element, body: int) -> _JointRec:
        a = self._attrs(el, body)
        if el.tag == "freejoint":
            kind = FREE
        else:
            t = a.get("type") or "hinge"
            if t not in _JOINT_KIND:
                self.note("joint", f"joint type '{t}' is unknown; read as a hinge")
            kind = _JOINT_KIND.get(t, REVOLUTE)
        axis = a.get("axis")
        axis = np.array([0.0, 0.0, 1.0]) if axis is None else axis / np.linalg.norm(axis)
        num = lambda k: a.get(k) if a.get(k) is not None else 0.0  # noqa: E731
        return _JointRec(a.get("name") or f"joint_{body}", kind,
                         a["pos"] if a.get("pos") is not None else np.zeros(3), axis,
                         None if a.get("limited") is False else a.get("range"),
                         num("damping"), num("armature"), num("stiffness"), num("springref"), num("frictionloss"))

    def _inertial(self, el: ET.Element, body: int) -> SpatialInertia:
        a = self._attrs(el, body)
        full = a.get("fullinertia")
        if full is not None and len(full) == 6:
            xx, yy, zz, xy, xz, yz = full
            inertia = np.array([[xx, xy, xz], [xy, yy, yz], [xz, yz, zz]])
        else:
            diag = a.get("diaginertia")
            inertia = np.diag(np.full(3, 0.001) if diag is None else diag)
            q = a.get("quat")
            if q is not None and len(q) == 4:
                R = quat_to_matrix(*(np.array(q) / np.linalg.norm(q)))
                inertia = R @ inertia @ R.T
        mass = a.get("mass") if a.get("mass") is not None else 1.0
        return SpatialInertia.new(mass, a["pos"] if a.get("pos") is not None else np.zeros(3), inertia)

    def _geom(self, el: ET.Element, body: int) -> Optional[_GeomRec]:
        a = self._attrs(el, body)
        kind = a.get("type") or "sphere"
        mesh = None
        if kind == "mesh" or a.get("mesh") is not None:
            mesh = next((m for m in self.meshes if m.name == (a.get("mesh") or "") and m.vertices is not None
                         and len(m.vertices)), None)
            if mesh is None:
                self.note("geom", "mesh geoms whose asset could not be loaded are dropped; the body loses that "
                                  "collision shape")
                return None
            kind = "mesh"
        size = a.get("size")
        size = [0.05] if size is None else size
        pos = a["pos"] if a.get("pos") is not None else np.zeros(3)
        rot = _orientation("geom", a, self.degrees, self.eulerseq)
        rot = np.eye(3) if rot is None else rot
        seg = a.get("fromto")
        if seg is not None and len(seg) == 6:
            p0, p1 = np.array(seg[:3]), np.array(seg[3:])
            d = p1 - p0
            length = math.sqrt(float(np.dot(d, d)))
            pos = 0.5 * (p0 + p1)
            size = [size[0] if size else 0.05, 0.5 * length]
            if length > 1e-12:
                rot = quat_to_matrix(*_quat_z_onto(d / length))
        off = lambda k: a.get(k) == 0.0  # noqa: E731
        if a.get("mass") is not None:
            mass = a["mass"]
        elif kind in _SIZE_COUNT and len(size) >= _SIZE_COUNT[kind]:
            mass = (a.get("density") if a.get("density") is not None else 1000.0) * shape_volume(kind, size)
        else:
            mass = 0.0
        if mesh is not None:
            mass = 0.0  # a mesh's volume is not integrated: it adds no mass (the reference's rule)
        return _GeomRec(kind, size, pos, rot, mass, not (off("contype") and off("conaffinity")), mesh)

    def _actuator(self, el: ET.Element):
        if el.tag not in _ACTUATOR_TAGS:
            return
        a = self._attrs(el, None)
        joint = a.get("joint") or ""
        if not joint:
            self.note(el.tag, "an actuator needs a joint target (site and tendon actuators are not supported)")
            return
        gain, bias_q, bias_v = _actuator_law(el.tag, a)
        gear = a.get("gear")
        self.actuators.append(_ActuatorRec(a.get("name") or f"{el.tag}_{joint}", joint, gear[0] if gear else 1.0,
                                           a.get("ctrlrange"), a.get("forcerange"), gain, bias_q, bias_v))


# ── bodies into links ───────────────────────────────────────────────────────
def _body_inertia(b: _BodyRec) -> SpatialInertia:
    if b.inertial is not None:
        return b.inertial
    acc = _MassSum()
    for g in b.geoms:
        if g.kind in _SIZE_COUNT and len(g.size) >= _SIZE_COUNT[g.kind]:
            acc.add(g.mass, g.pos.copy(), g.rot @ np.diag(shape_principal_inertia(g.kind, g.size, g.mass)) @ g.rot.T)
    return acc.total() or SpatialInertia.new(1.0, np.zeros(3), np.diag([0.001, 0.001, 0.001]))


def _collision_shape(g: _GeomRec) -> Optional[Geometry]:
    s = g.size
    origin = SpatialTransform.new(g.rot.T, g.pos)  # body frame -> geom frame
    radius = s[0] if s else 0.05
    half = s[1] if len(s) > 1 else 0.05
    if g.kind == "sphere":
        return Geometry.sphere(radius, origin)
    if g.kind == "capsule":
        return Geometry.capsule(radius, 2.0 * half, origin)
    if g.kind == "cylinder":
        return Geometry.cylinder(radius, 2.0 * half, origin)
    if g.kind == "box":
        return Geometry.box(s[:3] if len(s) >= 3 else (0.05, 0.05, 0.05), origin)
    if g.kind == "plane":  # may be a body's first collision geom; it never meets the ground
        return Geometry(G_NONE, (), origin)
    if g.kind == "mesh":  # the body-frame bounding box of the mesh's vertices, as the device table holds it
        return Geometry.mesh_aabb(g.mesh.vertices.min(axis=0), g.mesh.vertices.max(axis=0), origin)
    return None


class MjcfLoader:
    """An MJCF document, read: from_file / from_xml_str, build_model(),
    unsupported(), sensors() (the reference's MjcfLoader surface)."""

    def __init__(self, xml: str, model_dir: Optional[str] = None):
        try:
            doc = ET.fromstring(xml)
        except ET.ParseError as e:
            raise MjcfError(f"XML parse error: {e}") from None
        self._r = _Reader(_splice_includes(doc, model_dir), model_dir)

    @staticmethod
    def from_file(path: str) -> "MjcfLoader":
        """A model file; its includes and mesh files resolve against its directory."""
        with open(path) as f:
            return MjcfLoader(f.read(), os.path.dirname(os.path.abspath(path)))

    @staticmethod
    def from_xml_str(xml: str) -> "MjcfLoader":
        return MjcfLoader(xml)

    def unsupported(self) -> List[UnsupportedFeature]:
        return list(self._r.unsupported)

    def sensors(self) -> List[SensorElement]:
        return list(self._r.sensors)

    def meshes(self) -> List[MeshAsset]:
        """The ``<mesh>`` assets in document order, loaded or with their error."""
        return list(self._r.meshes)

    def _links(self) -> Iterator[Tuple[int, str, int, Joint, SpatialInertia]]:
        """(body record, link name, parent link, joint, inertia) per link, in
        document order; a body without joints is one fixed link."""
        last_link: Dict[int, int] = {}
        n = 0
        for bi, b in enumerate(self._r.bodies):
            parent = -1 if b.parent is None else last_link[b.parent]
            placement = SpatialTransform.new(b.rot, b.pos)
            inertia = _body_inertia(b)
            if not b.joints:
                yield bi, b.name, parent, Joint(FIXED, placement, np.zeros(3)), inertia
                last_link[bi] = n
                n += 1
                continue
            for k, j in enumerate(b.joints):
                first, final = k == 0, k == len(b.joints) - 1
                frame = (placement if first else SpatialTransform.identity()).compose(
                    SpatialTransform.from_translation(j.pos))
                joint = Joint(j.jtype, frame, j.axis.copy(), damping=j.damping, stiffness=j.stiffness,
                              spring_ref=j.spring_ref, armature=j.armature, limits=j.limits,
                              friction_loss=j.friction_loss, name=j.name)
                mass = inertia if final else SpatialInertia.new(PLACEHOLDER_MASS, np.zeros(3),
                                                                 np.eye(3) * PLACEHOLDER_MASS)
                yield (bi, b.name if len(b.joints) == 1 else f"{b.name}_{k}", parent if first else n - 1, joint,
                       mass)
                last_link[bi] = n
                n += 1

    def build_model(self) -> Model:
        r = self._r
        builder = ModelBuilder().gravity(r.gravity).dt(r.timestep)
        owner: List[int] = []  # body record of each link
        for bi, name, parent, joint, inertia in self._links():
            builder.add_body(name, parent, joint, inertia)
            owner.append(bi)
        model = builder.build()
        link_of_joint = {link.joint.name: k for k, link in enumerate(model.bodies) if link.joint.name}
        for k, link in enumerate(model.bodies):
            if k + 1 < len(owner) and owner[k + 1] == owner[k]:
                continue  # the body's shapes go on its last link
            shapes = (_collision_shape(g) for g in r.bodies[owner[k]].geoms if g.collides)
            link.collisions = [s for s in shapes if s is not None]
            link.geometry = link.collisions[0] if link.collisions else None
        for a in r.actuators:
            if a.joint in link_of_joint:
                model.actuators.append(Actuator(a.name, a.joint, link_of_joint[a.joint], a.gear, a.ctrl_range, a.gain,
                                                a.bias_q, a.bias_v, a.force_range))
        return model

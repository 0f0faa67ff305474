"""The MJCF loader (phyz_amd.mjcf) and the CPU-model force terms it carries
(actuators, soft joint limits, dry friction) in the oracle.

Loader: the articulation the reference's own benchmark-model tests assert
(crates/phyz-mjcf/tests/benchmark_models.rs), the packed fixture
(phyz_amd/data/mjcf_models.npz), and the element semantics of
crates/phyz-mjcf/src, each checked against a closed form or an independent
construction (inertia by voxel integration, orientations by explicit
rotation products).

Force terms: known answers of crates/phyz-mjcf/tests/dynamics.rs (a geared
motor on a single link gives qdd = gear ctrl / I, clamped by ctrlrange; a
limited pendulum stays in its band) plus closed forms for the position servo,
the force range, the gated limit damping and the tanh friction.
"""
import math
import os
import struct

import numpy as np
import pytest

from oracle.oracle import Oracle
from phyz_amd import workloads as W
from phyz_amd.mjcf import MjcfError, MjcfLoader, quat_to_matrix, shape_principal_inertia, shape_volume
from phyz_amd.model import (FIXED, FREE, G_CAPSULE, G_MESH, G_SPHERE, REVOLUTE, pack_actuators, pack_bodies,
                            pack_geometries, pack_joint_terms)

REF_MODELS = "/root/reference/models"
need_ref = pytest.mark.skipif(not os.path.isdir(REF_MODELS), reason="reference model files not present")


def load(xml):
    return MjcfLoader.from_xml_str(xml)


def single_link(extra_joint="", actuator="", inertial='<inertial mass="1.0" diaginertia="0.25 0.25 0.25"/>',
                gravity="0 0 0"):
    return f"""<mujoco><option gravity="{gravity}"/><worldbody>
      <body name="link" pos="0 0 0">{inertial}<joint name="j" type="hinge" axis="0 0 1" {extra_joint}/></body>
    </worldbody><actuator>{actuator}</actuator></mujoco>"""


# ── the reference's benchmark models ────────────────────────────────────────
@need_ref
def test_benchmark_models_articulation():
    """The counts the reference asserts exactly (benchmark_models.rs)."""
    def m(name):
        return MjcfLoader.from_file(os.path.join(REF_MODELS, name)).build_model()
    ant = m("ant.xml")
    assert (ant.nq, ant.nv, ant.nbodies, ant.nu()) == (14, 14, 9, 8)
    assert all(b.inertia.mass > 0 for b in ant.bodies)
    assert sum(b.geometry is not None for b in ant.bodies) >= 9
    ch = m("half_cheetah.xml")
    assert ch.nv == 12 and ch.nu() == 6
    assert next(a for a in ch.actuators if a.joint_name == "ffoot").gear == 30.0  # per-joint gear beats the default
    hu = m("humanoid.xml")
    assert hu.nv == 23 and hu.nu() == 17
    assert next(b for b in hu.bodies if b.name.startswith("right_lower_arm")).inertia.mass > 0
    hand = m("shadow_hand.xml")
    assert hand.nv == 24 and hand.nu() == 20
    assert hand.actuators[0].gain > 0 and hand.actuators[0].bias_q < 0  # position servo
    for name in ("ant.xml", "half_cheetah.xml", "humanoid.xml", "shadow_hand.xml"):
        assert MjcfLoader.from_file(os.path.join(REF_MODELS, name)).unsupported() == []


@need_ref
@pytest.mark.parametrize("name", ["ant", "humanoid", "shadow_hand", "half_cheetah", "simple_arm"])
def test_tables_are_what_the_loader_makes_of_the_reference_models(name):
    z = np.load(W.MJCF_TABLES)
    m = MjcfLoader.from_file(os.path.join(REF_MODELS, f"{name}.xml")).build_model()
    assert np.array_equal(pack_bodies(m), z[f"{name}/body"])
    assert np.array_equal(pack_geometries(m)[0], z[f"{name}/geom"])
    assert np.array_equal(pack_joint_terms(m), z[f"{name}/joint_terms"])
    assert np.array_equal(pack_actuators(m).reshape(-1), z[f"{name}/actuators"].reshape(-1))


@pytest.mark.parametrize("name", ["ant", "humanoid", "shadow_hand", "half_cheetah", "simple_arm"])
def test_tables_round_trip_through_model_from_tables(name):
    z = np.load(W.MJCF_TABLES)
    m = W.mjcf_model(name)
    assert np.array_equal(pack_bodies(m), z[f"{name}/body"])
    assert np.array_equal(pack_geometries(m)[0], z[f"{name}/geom"])
    assert np.array_equal(pack_joint_terms(m), z[f"{name}/joint_terms"])
    assert np.array_equal(pack_actuators(m).reshape(-1), z[f"{name}/actuators"].reshape(-1))


def test_mjcf_ant_facts():
    """The ant file's own numbers through the fixture: degree ranges converted,
    ctrlrange converted too (the reference converts every actuator's
    ctrlrange under angle="degree"), gear 150, capsule legs from fromto, the
    torso a 0.25 m water sphere."""
    m = W.mjcf_model("ant")
    torso = m.bodies[0]
    assert torso.joint.jtype == FREE
    assert torso.inertia.mass == pytest.approx(1000 * 4 / 3 * math.pi * 0.25 ** 3, rel=1e-12)
    hip = m.bodies[1]
    assert hip.joint.limits == pytest.approx((-math.radians(30), math.radians(30)))
    assert hip.joint.damping == 1.0 and hip.joint.armature == 0.01
    a = m.actuators[0]
    assert a.gear == 150.0 and a.ctrl_range == pytest.approx((-math.radians(1), math.radians(1)))
    leg = m.bodies[2].geometry
    assert leg.kind == G_CAPSULE
    assert leg.params == pytest.approx((0.08, math.sqrt(0.4 ** 2 + 0.4 ** 2)))
    np.testing.assert_allclose(leg.origin.pos, [0.2, 0.2, 0.0])


# ── element semantics ───────────────────────────────────────────────────────
def test_defaults_classes_childclass_and_precedence():
    xml = """<mujoco><default>
        <joint damping="0.1" armature="2"/>
        <geom density="500"/>
        <default class="a"><joint damping="3"/>
          <default class="b"><joint stiffness="7"/></default></default>
      </default>
      <worldbody>
        <body name="r" childclass="b"><joint name="j0"/><geom type="sphere" size="0.1"/>
          <body name="c"><joint name="j1" class="a"/><joint name="j2" damping="9"/></body>
        </body>
        <body name="plain"><joint name="j3"/></body>
      </worldbody></mujoco>"""
    m = load(xml).build_model()
    j = {b.joint.name: b.joint for b in m.bodies}
    assert (j["j0"].damping, j["j0"].stiffness, j["j0"].armature) == (3.0, 7.0, 2.0)  # b -> a -> root
    assert (j["j1"].damping, j["j1"].stiffness) == (3.0, 0.0)                           # explicit class beats childclass
    assert (j["j2"].damping, j["j2"].stiffness) == (9.0, 7.0)                           # own attribute wins
    assert (j["j3"].damping, j["j3"].stiffness, j["j3"].armature) == (0.1, 0.0, 2.0)   # root class only
    r = next(b for b in m.bodies if b.name == "r")
    assert r.inertia.mass == pytest.approx(500 * 4 / 3 * math.pi * 0.1 ** 3)


def _voxel_inertia(inside, lo, hi, n=140):
    """Mass properties of a uniform solid of density 1 by midpoint voxels."""
    axes = [np.linspace(lo[k], hi[k], n, endpoint=False) + (hi[k] - lo[k]) / (2 * n) for k in range(3)]
    X, Y, Z = np.meshgrid(*axes, indexing="ij")
    sel = inside(X, Y, Z)
    dv = np.prod([(hi[k] - lo[k]) / n for k in range(3)])
    p = np.stack([X[sel], Y[sel], Z[sel]], axis=1)
    m = sel.sum() * dv
    com = p.mean(axis=0)
    d = p - com
    I = (np.eye(3) * (d * d).sum() - d.T @ d) * dv
    return m, com, I


def test_capsule_inertia_against_voxel_integration():
    r, h = 0.1, 0.15  # radius, half shaft
    def inside(x, y, z):
        zc = np.clip(z, -h, h)
        return x * x + y * y + (z - zc) ** 2 <= r * r
    m, com, I = _voxel_inertia(inside, [-r, -r, -h - r], [r, r, h + r])
    assert m == pytest.approx(shape_volume("capsule", [r, h]), rel=2e-3)
    p = shape_principal_inertia("capsule", [r, h], m)
    np.testing.assert_allclose(np.diag(I), p, rtol=4e-3)
    # a zero-length capsule is exactly a sphere
    s = shape_principal_inertia("sphere", [r], 1.0)
    np.testing.assert_allclose(shape_principal_inertia("capsule", [r, 0.0], 1.0), s, rtol=1e-14)


@pytest.mark.parametrize("r,h", [(0.08, 0.28), (0.046, 0.0), (0.5, 0.01), (0.01, 3.0)])
def test_capsule_inertia_is_cylinder_plus_two_hemispheres(r, h):
    """The textbook composition: a cylinder of length 2h plus two solid
    hemispheres, each with 83/320 m r^2 about its own centroid, which sits 3r/8
    beyond the shaft's end (parallel-axis theorem), at one density."""
    rho = 1.0 / shape_volume("capsule", [r, h])
    mc, ms = rho * math.pi * r * r * 2 * h, rho * 2 / 3 * math.pi * r ** 3
    assert mc + 2 * ms == pytest.approx(1.0, rel=1e-14)
    izz = mc * r * r / 2 + 2 * (2 / 5) * ms * r * r
    ixx = mc * (3 * r * r + (2 * h) ** 2) / 12 + 2 * (83 / 320 * ms * r * r + ms * (h + 3 * r / 8) ** 2)
    np.testing.assert_allclose(shape_principal_inertia("capsule", [r, h], 1.0), [ixx, ixx, izz], rtol=1e-13)


def test_box_and_cylinder_inertia_closed_forms():
    np.testing.assert_allclose(shape_principal_inertia("box", [0.1, 0.2, 0.3], 6.0),
                               [6 / 12 * (0.4 ** 2 + 0.6 ** 2), 6 / 12 * (0.2 ** 2 + 0.6 ** 2), 6 / 12 * (0.2 ** 2 + 0.4 ** 2)])
    np.testing.assert_allclose(shape_principal_inertia("cylinder", [0.1, 0.2], 2.0),
                               [2 * (3 * 0.01 + 0.16) / 12, 2 * (3 * 0.01 + 0.16) / 12, 0.5 * 2 * 0.01])


def test_geom_inertia_combines_with_parallel_axis_and_explicit_mass_wins():
    xml = """<mujoco><worldbody><body name="b"><joint/>
        <geom type="sphere" size="0.1" pos="0.3 0 0" mass="2"/>
        <geom type="sphere" size="0.1" pos="-0.1 0 0" mass="6"/>
      </body><body name="e"><inertial mass="3" pos="0 0 1" diaginertia="1 2 3"/><geom type="sphere" size="5"/><joint/></body>
      </worldbody></mujoco>"""
    m = load(xml).build_model()
    b = m.bodies[0].inertia
    assert b.mass == 8.0
    np.testing.assert_allclose(b.com, [0.0, 0.0, 0.0], atol=1e-15)
    i0 = 0.4 * 0.01
    # about the combined COM (origin): spheres at x = 0.3 (2 kg) and -0.1 (6 kg)
    np.testing.assert_allclose(np.diag(b.inertia), [8 * i0, 8 * i0 + 2 * 0.09 + 6 * 0.01, 8 * i0 + 2 * 0.09 + 6 * 0.01])
    e = m.bodies[1].inertia
    assert e.mass == 3.0 and np.allclose(e.com, [0, 0, 1]) and np.allclose(np.diag(e.inertia), [1, 2, 3])


def test_fromto_sets_centre_length_and_axis():
    xml = """<mujoco><worldbody><body name="b"><joint/>
        <geom type="capsule" fromto="0.1 0.2 0.3  0.1 0.6 0.3" size="0.03"/>
        <geom type="capsule" fromto="0 0 1  0 0 0" size="0.03"/></body></worldbody></mujoco>"""
    m = load(xml).build_model()
    g, g2 = m.bodies[0].collisions
    assert g.params == pytest.approx((0.03, 0.4))
    np.testing.assert_allclose(g.origin.pos, [0.1, 0.4, 0.3])
    # origin.rot is body -> shape; its transpose maps the shape's +Z onto the segment
    np.testing.assert_allclose(g.origin.rot.T @ [0, 0, 1], [0, 1, 0], atol=1e-12)
    np.testing.assert_allclose(g2.origin.rot.T @ [0, 0, 1], [0, 0, -1], atol=1e-12)  # antiparallel
    assert m.bodies[0].geometry is g  # the contact shape is the first collision geom


def test_multi_joint_body_becomes_a_chain():
    xml = """<mujoco><worldbody><body name="t" pos="1 2 3">
        <joint name="a" type="hinge" axis="1 0 0"/><joint name="b" type="slide" axis="0 1 0" pos="0 0 0.5"/>
        <geom type="sphere" size="0.1"/></body></worldbody>
        <actuator><motor joint="b" gear="3"/></actuator></mujoco>"""
    m = load(xml).build_model()
    assert [b.name for b in m.bodies] == ["t_0", "t_1"]
    assert m.bodies[1].parent == 0
    np.testing.assert_allclose(m.bodies[0].joint.parent_to_joint.pos, [1, 2, 3])
    np.testing.assert_allclose(m.bodies[1].joint.parent_to_joint.pos, [0, 0, 0.5])
    assert m.bodies[0].inertia.mass == 1e-9 and m.bodies[1].inertia.mass > 1.0
    assert m.bodies[1].geometry is not None and m.bodies[0].geometry is None
    assert m.actuators[0].joint_idx == 1 and m.actuators[0].gear == 3.0


def test_orientation_spellings_agree():
    R = quat_to_matrix(math.cos(math.pi / 4), 0, 0, math.sin(math.pi / 4))  # 90 deg about z
    xml = """<mujoco><compiler angle="degree"/><worldbody>
        <body name="q" quat="0.7071067811865476 0 0 0.7071067811865476"/>
        <body name="e" euler="0 0 90"/><body name="aa" axisangle="0 0 1 90"/>
        <body name="xy" xyaxes="0 1 0 -1 0 0"/><body name="z" zaxis="1 0 0"/>
      </worldbody></mujoco>"""
    m = load(xml).build_model()
    rot = {b.name: b.joint.parent_to_joint.rot for b in m.bodies}
    for k in ("q", "e", "aa", "xy"):
        np.testing.assert_allclose(rot[k], R, atol=1e-12)
    np.testing.assert_allclose(rot["z"] @ [0, 0, 1], [1, 0, 0], atol=1e-12)


def test_euler_sequences_intrinsic_and_extrinsic():
    def rx(a):
        return np.array([[1, 0, 0], [0, math.cos(a), -math.sin(a)], [0, math.sin(a), math.cos(a)]])

    def ry(a):
        return np.array([[math.cos(a), 0, math.sin(a)], [0, 1, 0], [-math.sin(a), 0, math.cos(a)]])
    a, b = 0.3, -0.7
    for seq, want in (("xyz", rx(a) @ ry(b)), ("XYZ", ry(b) @ rx(a))):
        xml = f"""<mujoco><compiler eulerseq="{seq}"/><worldbody><body name="b" euler="{a} {b} 0"/></worldbody></mujoco>"""
        np.testing.assert_allclose(load(xml).build_model().bodies[0].joint.parent_to_joint.rot, want, atol=1e-12)


@pytest.mark.parametrize("attr,msg", [('euler="1 2"', "needs 3 numbers"), ('quat="0 0 0 0"', "zero norm"),
                                      ('axisangle="0 0 0 1"', "zero vector"), ('xyaxes="1 0 0 2 0 0"', "parallel")])
def test_degenerate_orientations_are_errors(attr, msg):
    with pytest.raises(MjcfError) as e:
        load(f"<mujoco><worldbody><body name='b' {attr}/></worldbody></mujoco>")
    assert "body" in str(e.value) and msg in str(e.value)


def test_degree_compiler_converts_ranges_and_ctrlranges():
    xml = """<mujoco><compiler angle="{u}"/><worldbody><body><joint name="j" range="-30 60"/></body></worldbody>
             <actuator><motor joint="j" ctrlrange="-1 2"/></actuator></mujoco>"""
    d = load(xml.format(u="degree")).build_model()
    r = load(xml.format(u="radian")).build_model()
    assert d.bodies[0].joint.limits == pytest.approx((math.radians(-30), math.radians(60)))
    assert d.actuators[0].ctrl_range == pytest.approx((math.radians(-1), math.radians(2)))
    assert r.bodies[0].joint.limits == (-30.0, 60.0) and r.actuators[0].ctrl_range == (-1.0, 2.0)


def test_actuator_kinds_use_the_affine_law():
    xml = """<mujoco><worldbody><body><joint name="j"/></body></worldbody><actuator>
        <motor joint="j" gear="5"/><position joint="j" kp="4" kv="0.5"/><velocity joint="j" kv="3"/>
        <general joint="j" gainprm="2" biasprm="0 -1 -0.25" forcerange="-1 1"/><motor gear="2"/>
      </actuator></mujoco>"""
    L = load(xml)
    a = L.build_model().actuators
    assert [(x.gear, x.gain, x.bias_q, x.bias_v) for x in a] == [(5, 1, 0, 0), (1, 4, -4, -0.5), (1, 3, 0, -3),
                                                                  (1, 2, -1, -0.25)]
    assert a[3].force_range == (-1.0, 1.0)
    assert a[1].force_at(0.3, 0.1, 2.0) == pytest.approx(4 * (0.3 - 0.1) - 0.5 * 2.0)
    assert a[3].force_at(10.0, 0.0, 0.0) == 1.0
    assert any("joint" in u.detail for u in L.unsupported())  # the motor without a joint


def test_joint_attributes_limited_false_freejoint_and_sensors():
    xml = """<mujoco><worldbody>
        <body name="f"><freejoint/></body>
        <body name="h"><joint name="j" range="-0.5 0.5" damping="0.1" armature="0.05" stiffness="3" springref="0.2" frictionloss="0.7"/></body>
        <body name="u"><joint name="k" range="-0.5 0.5" limited="false"/></body>
      </worldbody><sensor><jointpos joint="j"/></sensor></mujoco>"""
    L = load(xml)
    m = L.build_model()
    assert m.bodies[0].joint.jtype == FREE and m.nv == 8
    j = m.bodies[1].joint
    assert j.limits == (-0.5, 0.5) and (j.damping, j.armature, j.stiffness, j.spring_ref, j.friction_loss) == (
        0.1, 0.05, 3.0, 0.2, 0.7)
    assert m.bodies[2].joint.limits is None
    assert [(s.kind, s.target) for s in L.sensors()] == [("jointpos", "j")]


def test_visual_only_geoms_add_inertia_but_do_not_collide():
    xml = """<mujoco><worldbody><body><joint/><geom type="sphere" size="0.1" contype="0" conaffinity="0"/>
        <geom type="box" size="0.1 0.1 0.1"/></body><body><joint/></body></worldbody></mujoco>"""
    m = load(xml).build_model()
    assert [g.kind for g in m.bodies[0].collisions] == [2]
    assert m.bodies[0].inertia.mass == pytest.approx(1000 * (4 / 3 * math.pi * 1e-3 + 8e-3))
    assert m.bodies[1].inertia.mass == 1.0  # no geoms: the placeholder point mass


def test_unsupported_features_are_reported():
    xml = """<mujoco><asset><hfield name="h" size="1 1 1 1"/></asset><worldbody><body><joint type="weird"/></body>
      </worldbody><tendon/><equality/></mujoco>"""
    tags = {u.tag for u in load(xml).unsupported()}
    assert tags == {"hfield", "joint", "tendon", "equality"}


def test_includes_splice_defaults_and_bodies(tmp_path):
    """include.rs: an included file's children land where the <include> stood
    (its defaults apply to the including file's bodies too); nested includes
    resolve against their own directory; a cycle stops at the depth cap; a
    missing file or attribute is an error that names it."""
    (tmp_path / "parts").mkdir()
    (tmp_path / "parts" / "leg.xml").write_text("""<mujocoinclude><body name="nested_leg"><joint/>
        <geom type="sphere" size="0.05"/></body></mujocoinclude>""")
    (tmp_path / "child.xml").write_text("""<mujoco><default><joint damping="3.25"/></default>
        <worldbody><body name="included_child"><joint/><include file="parts/leg.xml"/></body></worldbody></mujoco>""")
    (tmp_path / "main.xml").write_text("""<mujoco><include file="child.xml"/>
        <worldbody><body name="own"><joint/></body></worldbody></mujoco>""")
    m = MjcfLoader.from_file(str(tmp_path / "main.xml")).build_model()
    assert [b.name for b in m.bodies] == ["included_child", "nested_leg", "own"]
    assert m.bodies[1].parent == 0
    assert all(b.joint.damping == 3.25 for b in m.bodies)
    (tmp_path / "a.xml").write_text('<mujoco><include file="b.xml"/></mujoco>')
    (tmp_path / "b.xml").write_text('<mujoco><include file="a.xml"/></mujoco>')
    with pytest.raises(MjcfError, match="cyclic"):
        MjcfLoader.from_file(str(tmp_path / "a.xml"))
    with pytest.raises(MjcfError, match="does_not_exist.xml"):
        MjcfLoader.from_xml_str('<mujoco><include file="does_not_exist.xml"/></mujoco>')
    with pytest.raises(MjcfError, match="missing required attribute 'file'"):
        MjcfLoader.from_xml_str("<mujoco><include/></mujoco>")
    assert MjcfLoader.from_xml_str("<mujoco><worldbody/></mujoco>").unsupported() == []


TET = np.array([[0, 0, 0], [1, 0, 0], [0, 1, 0], [0, 0, 1]], dtype=float)
TET_FACES = [(0, 2, 1), (0, 1, 3), (0, 3, 2), (1, 2, 3)]


def test_mesh_files_obj_and_stl():
    """assets.rs loaders: OBJ polygons fan into triangles, index forms v, v/vt,
    v//vn and negative indices; binary STL by its size, ASCII STL by 'solid';
    garbage is an error, not a crash."""
    from phyz_amd.mjcf import _obj, _stl
    v, f = _obj("v 0 0 0\nv 1 0 0\nv 1 1 0\nv 0 1 0\nf 1 2 3 4\n")
    assert v.shape == (4, 3) and f.tolist() == [[0, 1, 2], [0, 2, 3]]
    v, f = _obj("v 0 0 0\nv 1 0 0\nv 0 1 0\nf 1/1/1 2//2 -1\n")
    assert f.tolist() == [[0, 1, 2]]
    with pytest.raises(ValueError):
        _obj("v 0 0 0\nf 1 2 3\n")
    ascii_stl = b"solid t\n facet normal 0 0 1\n  outer loop\n   vertex 0 0 0\n   vertex 1 0 0\n" \
                b"   vertex 0 1 0\n  endloop\n endfacet\nendsolid t\n"
    v, f = _stl(ascii_stl)
    assert v.shape == (3, 3) and f.tolist() == [[0, 1, 2]]
    binary = b"solid-looking header".ljust(80, b"\0") + struct.pack("<I", 1) + struct.pack("<3f", 0, 0, 1) + \
        struct.pack("<9f", 0, 0, 0, 1, 0, 0, 0, 1, 0) + b"\0\0"
    v, f = _stl(binary)
    assert v.shape == (3, 3) and v[1, 0] == 1.0
    with pytest.raises(ValueError):
        _stl(b"not a mesh at all")


def test_mesh_assets_obj_and_binary_stl(tmp_path):
    """<asset><mesh> through <compiler meshdir> (which wins over assetdir),
    the name defaulting to the file stem, per-axis scale; a mesh geom
    collides through its body-frame bounding box and adds no mass; an
    unloadable mesh is reported and its geom dropped."""
    (tmp_path / "meshes").mkdir()
    (tmp_path / "meshes" / "t.obj").write_text("".join(f"v {a} {b} {c}\n" for a, b, c in TET) +
                                               "".join(f"f {a + 1} {b + 1} {c + 1}\n" for a, b, c in TET_FACES))
    with open(tmp_path / "meshes" / "t.stl", "wb") as f:
        f.write(b"\0" * 80 + struct.pack("<I", 4))
        for tri in TET_FACES:
            f.write(struct.pack("<3f", 0, 0, 0) + b"".join(struct.pack("<3f", *TET[k] * 2) for k in tri) + b"\0\0")
    (tmp_path / "m.xml").write_text("""<mujoco><compiler meshdir="meshes" assetdir="elsewhere"/>
        <asset><mesh file="t.obj"/><mesh name="s" file="t.stl" scale="1 2 3"/>
        <mesh name="gone" file="missing.stl"/></asset>
        <worldbody><body><joint/><geom type="mesh" mesh="t"/></body>
        <body><joint/><geom type="mesh" mesh="s" pos="0 0 0.5"/><geom type="sphere" size="0.1"/></body>
        <body><joint/><geom type="mesh" mesh="gone"/><geom type="sphere" size="0.1"/></body></worldbody></mujoco>""")
    L = MjcfLoader.from_file(str(tmp_path / "m.xml"))
    ms = {m.name: m for m in L.meshes()}
    assert list(ms) == ["t", "s", "gone"]
    assert ms["t"].vertices.shape == (4, 3) and ms["t"].faces.shape == (4, 3)
    assert ms["s"].vertices.shape == (12, 3) and np.allclose(ms["s"].vertices.max(axis=0), [2, 4, 6])
    assert ms["gone"].vertices is None and "missing.stl" in ms["gone"].load_error
    m = L.build_model()
    g0, g1 = m.bodies[0].geometry, m.bodies[1].geometry
    assert g0.kind == G_MESH and g0.params == (0, 0, 0, 1, 1, 1)
    assert g1.kind == G_MESH and g1.params == (0, 0, 0, 2, 4, 6) and np.allclose(g1.origin.pos, [0, 0, 0.5])
    assert len(m.bodies[1].collisions) == 2
    assert m.bodies[0].inertia.mass == 1.0  # the mesh adds no mass: the body takes the default
    sphere = 1000 * 4 / 3 * math.pi * 1e-3
    assert m.bodies[1].inertia.mass == pytest.approx(sphere)
    assert m.bodies[2].geometry.kind == G_SPHERE and len(m.bodies[2].collisions) == 1
    assert {u.tag for u in L.unsupported()} == {"mesh", "geom"}
    geom, collidable = pack_geometries(m)
    assert collidable == 3 and int(geom[0, 0]) == G_MESH and list(geom[0, 1:7]) == [0, 0, 0, 1, 1, 1]


# ── force terms in the oracle ───────────────────────────────────────────────
def qdd_for(xml, ctrl, q=0.0, v=0.0):
    m = load(xml).build_model()
    o = Oracle(m)
    return o.aba([q], [v], [ctrl])[0], o


def test_geared_motor_torque_and_ctrlrange_clamp():
    xml = single_link(actuator='<motor name="m" joint="j" gear="100" ctrlrange="-1 1"/>')
    assert qdd_for(xml, 0.5)[0] == pytest.approx(50.0 / 0.25, abs=1e-9)
    assert qdd_for(xml, 7.5)[0] == pytest.approx(100.0 / 0.25, abs=1e-9)
    assert qdd_for(xml, -7.5)[0] == pytest.approx(-100.0 / 0.25, abs=1e-9)


def test_position_servo_and_force_range():
    xml = single_link(actuator='<position joint="j" kp="40" kv="3" gear="2"/>')
    q, v, c = 0.2, -0.5, 0.7
    assert qdd_for(xml, c, q, v)[0] == pytest.approx(2 * (40 * (c - q) - 3 * v) / 0.25, rel=1e-12)
    xml = single_link(actuator='<general joint="j" gainprm="10" forcerange="-2 3"/>')
    assert qdd_for(xml, 1.0)[0] == pytest.approx(3.0 / 0.25)
    assert qdd_for(xml, -1.0)[0] == pytest.approx(-2.0 / 0.25)


def test_soft_limit_force_is_gated_spring_damper():
    xml = single_link('range="-0.3 0.3"')
    I = 0.25
    # past the upper bound, moving further out: spring + damping
    assert qdd_for(xml, 0.0, 0.31, 0.5)[0] == pytest.approx(-(1000 * 0.01 + 60 * 0.5) / I, rel=1e-9)
    # past the bound but moving back in: spring only
    assert qdd_for(xml, 0.0, 0.31, -0.5)[0] == pytest.approx(-(1000 * 0.01) / I, rel=1e-9)
    assert qdd_for(xml, 0.0, -0.35, -0.2)[0] == pytest.approx((1000 * 0.05 + 60 * 0.2) / I, rel=1e-9)
    assert qdd_for(xml, 0.0, 0.29, 5.0)[0] == 0.0  # inside the band


def test_friction_loss_is_smoothed_coulomb():
    xml = single_link('frictionloss="0.7"')
    for v in (2e-3, -5e-4, 0.3):
        assert qdd_for(xml, 0.0, 0.0, v)[0] == pytest.approx(-0.7 * math.tanh(v / 1e-3) / 0.25, rel=1e-12)


def test_limit_holds_a_falling_link():
    """A pendulum started at its limit moving outward stays in the band
    (dynamics.rs mjcf_joint_limit_stops_the_link), integrated here with the
    oracle's step at dt 1e-4."""
    xml = """<mujoco><option gravity="0 -9.81 0" timestep="0.0001"/><worldbody><body name="l">
        <inertial mass="1.0" pos="0 -0.5 0" diaginertia="0.083 0.083 0.083"/>
        <joint name="j" type="hinge" axis="0 0 1" range="-0.3 0.3"/></body></worldbody></mujoco>"""
    m = load(xml).build_model()
    o = Oracle(m)
    q, v, c = np.array([[0.3]]), np.array([[1.0]]), np.zeros((1, 1))
    lo = hi = 0.3
    for _ in range(20):
        o.step_batch(q, v, c, 1000)
        lo, hi = min(lo, q[0, 0]), max(hi, q[0, 0])
        assert np.isfinite(q).all()
    assert -0.4 < lo and hi < 0.4


def test_models_without_actuators_take_ctrl_per_dof():
    xml = single_link()
    assert qdd_for(xml, 0.75)[0] == pytest.approx(0.75 / 0.25)


# ── the C ABI's validation (host-only simulators, no GPU) ───────────────────
def test_abi_actuator_and_joint_term_validation():
    from phyz_amd.model import PdDof
    from phyz_amd.sim import BatchSim, PhzError
    m = W.mjcf_model("ant")
    s = BatchSim(m, 8, "f32", device=-1)
    assert s.nctrl == 8
    with pytest.raises(PhzError, match="actuators"):
        s.enable_pd_control([PdDof(6, 6, 1.0, 0.1, 1.0)])
    with pytest.raises(PhzError, match="noise control 8 out of range"):
        s.enable_control_noise(1, 1, -1.0, 1.0, [8])
    bad = pack_actuators(m)
    bad[0, 0] = 0  # the free root: first DOF is fine (6 DOF joint)
    s.set_actuators(bad)
    fixed = W.mjcf_model("shadow_hand")
    s2 = BatchSim(fixed, 8, "f32", device=-1, model_terms=False)
    assert s2.nctrl == fixed.nv
    t = pack_actuators(fixed)
    t[0, 0] = 0  # the forearm is welded: no DOF
    with pytest.raises(PhzError, match="has no DOF"):
        s2.set_actuators(t)
    s2.enable_pd_control([PdDof(0, 0, 1.0, 0.1, 1.0)])
    with pytest.raises(PhzError, match="cannot also have PD"):
        s2.set_actuators(pack_actuators(fixed))
    jt = pack_joint_terms(fixed)
    jt[3, 3] = -1.0
    with pytest.raises(PhzError, match=">= 0"):
        s2.set_joint_terms(jt)
    s.set_actuators(None)
    assert s.nctrl == m.nv

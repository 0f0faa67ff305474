"""Small test models, the shapes of the reference's own parity fixtures
(crates/phyz-gpu/tests/cuda_vs_cpu.rs:33-165, joint_offset_vs_cpu.rs:28-41,
contact_drop.rs:19-32, ground_contact.rs), plus geometry variants."""
from __future__ import annotations

import math

import numpy as np

from phyz_amd.model import (BALL, FREE, PRISMATIC, REVOLUTE, Geometry, Joint, ModelBuilder, PdDof, SpatialInertia,
                            SpatialTransform, rotation_axis_angle)

G = 9.81


def iso(mass, i):
    return SpatialInertia.new(mass, np.zeros(3), np.eye(3) * i)


def double_pendulum_offset():
    return (ModelBuilder().gravity([0, -G, 0]).dt(0.001)
            .add_revolute_body("upper", -1, SpatialTransform.identity(), SpatialInertia.rod(1.0, 0.5))
            .add_revolute_body("lower", 0, SpatialTransform.from_translation([0, -1.0, 0]), SpatialInertia.rod(1.0, 0.5))
            .build())


def arm_6dof():
    length = 0.3
    inertia = SpatialInertia.new(0.5, [0, 0, -length / 2], np.diag([0.00375, 0.00375, 0.001]))
    b = ModelBuilder().gravity([0, 0, -G]).dt(0.001).add_revolute_body("j1", -1, SpatialTransform.identity(), inertia)
    for k in range(1, 6):
        b.add_revolute_body(f"j{k + 1}", k - 1, SpatialTransform.from_translation([0, 0, -length]), inertia)
    return b.build()


def free_base_with_limb():
    return (ModelBuilder().gravity([0, 0, -G]).dt(0.001)
            .add_body("torso", -1, Joint(FREE, SpatialTransform.identity(), np.zeros(3)), iso(5.0, 0.3))
            .add_revolute_body("limb", 0, SpatialTransform.from_translation([0.2, 0, 0]), iso(1.0, 0.05))
            .build())


def ball_joint_model():
    return (ModelBuilder().gravity([0, 0, -G]).dt(0.001)
            .add_body("ball", -1, Joint(BALL, SpatialTransform.identity(), np.zeros(3)),
                      SpatialInertia.new(1.0, [0, 0, -0.3], np.diag([0.05, 0.05, 0.02])))
            .build())


def prismatic_model():
    return (ModelBuilder().gravity([0, 0, -G]).dt(0.001)
            .add_prismatic_body("slider", -1, SpatialTransform.identity(), [0, 0, 1.0], iso(1.0, 0.1))
            .build())


def pd_link():
    inertia = SpatialInertia.new(1.0, [0, 0, -0.5], np.eye(3) * 0.1)
    m = ModelBuilder().gravity([0, 0, -G]).dt(0.002).add_revolute_body("link", -1, SpatialTransform.identity(), inertia).build()
    return m, [PdDof(0, 0, 30.0, 2.0, 25.0)]


def free_shape(geom, mass=1.0, inertia=None, dt=0.001):
    I = np.diag([0.02, 0.03, 0.025]) if inertia is None else inertia
    return (ModelBuilder().gravity([0, 0, -G]).dt(dt)
            .add_free_body("body", -1, SpatialTransform.identity(), SpatialInertia.new(mass, [0.01, -0.02, 0.005], I), geom)
            .build())


def shapes():
    """Free bodies with each collision shape, off-centre instance origins."""
    off = SpatialTransform.new(rotation_axis_angle([1, 1, 0], 0.3), [0.02, -0.01, 0.03])
    return {
        "sphere": free_shape(Geometry.sphere(0.1)),
        "box": free_shape(Geometry.box([0.1, 0.08, 0.06])),
        "capsule": free_shape(Geometry.capsule(0.05, 0.3, off)),
        "cylinder": free_shape(Geometry.cylinder(0.06, 0.2, off)),
        "mesh": free_shape(Geometry.mesh_aabb([-0.1, -0.05, -0.08], [0.12, 0.06, 0.05], off)),
    }


def random_tree(seed, njoints=8, with_free_root=True):
    """A random tree over every joint type with passive springs, damping and armature."""
    rng = np.random.default_rng(seed)

    def rinertia():
        A = rng.normal(size=(3, 3))
        return SpatialInertia.new(rng.uniform(0.5, 2), rng.normal(size=3) * 0.3, (A @ A.T + 0.1 * np.eye(3)) * 0.1)

    def rrot():
        return rotation_axis_angle(rng.normal(size=3), rng.uniform(-3, 3))

    b = ModelBuilder().gravity(rng.normal(size=3) * 5).dt(0.002)
    if with_free_root:
        b.add_body("root", -1, Joint(FREE, SpatialTransform.new(rrot(), rng.normal(size=3)), np.zeros(3)), rinertia())
    else:
        b.add_revolute_body("root", -1, SpatialTransform.identity(), rinertia())
    types = [REVOLUTE, PRISMATIC, BALL, 2, REVOLUTE, BALL, FREE, REVOLUTE, PRISMATIC, REVOLUTE]
    for i in range(njoints):
        t = types[i % len(types)]
        parent = int(rng.integers(0, i + 1))
        ax = rng.normal(size=3)
        ax /= np.linalg.norm(ax)
        j = Joint(t, SpatialTransform.new(rrot(), rng.normal(size=3) * 0.5), ax,
                  damping=float(rng.uniform(0, 0.5)), stiffness=float(rng.uniform(0, 2)) if t in (0, 1) else 0.0,
                  spring_ref=0.1, armature=float(rng.uniform(0, 0.1)))
        b.add_body(f"b{i}", parent, j, rinertia())
    return b.build()


def trunk_and_two_feet():
    """Free trunk with two hinged feet, offset centres of mass (cuda_vs_cpu.rs:1418-1443)."""
    def off(m, c):
        return SpatialInertia.new(m, c, np.diag([0.1, 0.1, 0.1]))
    return (ModelBuilder().gravity([0, 0, -9.81]).dt(0.001)
            .add_body("trunk", -1, Joint(FREE, SpatialTransform.identity(), np.zeros(3)), off(8.0, [0.02, 0.0, 0.15]))
            .add_revolute_body("left_foot", 0, SpatialTransform.from_translation([0.0, 0.12, -0.6]),
                               off(1.5, [0.03, 0.0, -0.02]))
            .add_revolute_body("right_foot", 0, SpatialTransform.from_translation([0.0, -0.12, -0.6]),
                               off(1.5, [-0.03, 0.01, -0.02]))
            .build())


def deck_and_feet():
    """A free box deck on the ground with a free sphere foot and a free box foot
    standing on it (the skateboard case of contact_pipeline.rs:300-353): plane
    body 0, face at its local +Z half-thickness."""
    def box_inertia(m, h):
        hx, hy, hz = h
        return SpatialInertia.new(m, np.zeros(3), np.diag([m * (hy * hy + hz * hz) / 3, m * (hx * hx + hz * hz) / 3,
                                                           m * (hx * hx + hy * hy) / 3]))
    free = lambda: Joint(FREE, SpatialTransform.identity(), np.zeros(3))
    return (ModelBuilder().gravity([0, 0, -G]).dt(0.001)
            .add_body("deck", -1, free(), box_inertia(2.0, (0.4, 0.1, 0.02)), Geometry.box([0.4, 0.1, 0.02]))
            .add_body("foot_sphere", -1, free(), SpatialInertia.sphere(0.5, 0.05), Geometry.sphere(0.05))
            .add_body("foot_box", -1, free(), box_inertia(0.4, (0.05, 0.03, 0.02)), Geometry.box([0.05, 0.03, 0.02]))
            .build())


DECK_PLANE = (0, 0.02, 0.05, 0.4, 0.1)  # body, offset, max_depth, half_x, half_y


def bumpy_heightfield(nx=9, ny=9, cell=0.25, amp=0.08):
    """(nx, ny, ox, oy, oz, cell, heights) centred on the origin: smooth bumps."""
    xs = (np.arange(nx) - (nx - 1) / 2) * cell
    ys = (np.arange(ny) - (ny - 1) / 2) * cell
    h = amp * np.sin(2.1 * xs)[None, :] * np.cos(1.7 * ys)[:, None] + 0.03 * ys[:, None]
    return (nx, ny, float(xs[0]), float(ys[0]), 0.01, cell, np.asarray(h, dtype=np.float32).astype(np.float64))

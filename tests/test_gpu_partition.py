"""Partitioned step kernels (several waves per world group) against the oracle
and against the one-lane-per-world kernel.

The host splits a tree over the waves of a workgroup (PHZ_PARTITION: 0 one lane
per world, auto, or forced). Each mode must give the oracle's per-step qdd and
agree with the others on short f64 rollouts (the only difference between them
is the summation order of articulated-inertia contributions at branch points).
"""
import os

import numpy as np
import pytest

from phyz_amd import workloads as W
from phyz_amd.model import (BALL, FIXED, PRISMATIC, REVOLUTE, Geometry, Joint, ModelBuilder, SpatialInertia,
                            SpatialTransform, pack_geometries, rotation_axis_angle)
from phyz_amd.sim import BatchSim
from tests import models as TM
from tests.helpers import as_precision, oracle_for, rel_err_rows
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu


def fixed_base_three_arms():
    """A welded base with three branches (revolute, prismatic, ball joints),
    contact spheres on the branch tips."""
    rng = np.random.default_rng(31)
    b = ModelBuilder().gravity([0, 0, -9.81]).dt(0.001)
    b.add_fixed_body("base", -1, SpatialTransform.from_translation([0, 0, 0.6]), SpatialInertia.sphere(2.0, 0.2))
    for k, jt in enumerate((REVOLUTE, PRISMATIC, BALL)):
        parent = 0
        for j in range(3):
            ax = rng.normal(size=3)
            ax /= np.linalg.norm(ax)
            t = jt if j == 0 else REVOLUTE
            ptj = SpatialTransform.new(rotation_axis_angle(rng.normal(size=3), 0.4), [0.15, 0.05 * k, -0.1])
            geo = Geometry.sphere(0.05, SpatialTransform.from_translation([0.1, 0, -0.05])) if j == 2 else None
            idx = len(b._bodies)
            b.add_body(f"a{k}_{j}", parent, Joint(t, ptj, ax, damping=0.2, armature=0.01),
                       SpatialInertia.new(0.5, [0.05, 0, 0], np.diag([1e-3, 2e-3, 2e-3])), geo)
            parent = idx
    return b.build()


def _sim(model, n, prec, mode, contact=None, noise=None, groups=None):
    env = {"PHZ_PARTITION": mode}
    if groups is not None:
        env["PHZ_MAX_GROUPS"] = str(groups)
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        s = BatchSim(model, n, prec)
        if contact is not None:
            s.enable_ground_contact(*contact)
        if noise is not None:
            s.enable_control_noise(*noise)
        s.compile()
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k)
            else:
                os.environ[k] = v
    return s


UNMERGED_WAVES = {"humanoid": 4, "hand": 5}  # parts below the trunk

CASES = {
    "random_tree_free": (lambda: TM.random_tree(21, 12, True), None, "2"),
    "fixed_base_arms": (fixed_base_three_arms, (0.0, 2e3, 20.0, 0.8), "1"),
    "ant": (lambda: W.config(3).model, (0.0, 1e4, 100.0, 1.0), "2"),
    "humanoid": (lambda: W.config(4).model, (0.0, 1e4, 100.0, 1.0), "auto"),
    "hand": (lambda: W.config(5).model, None, "auto"),
}


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("prec", ["f64", "f32"])
def test_partitioned_step_matches_oracle(name, prec):
    _step_matches_oracle(name, prec)


def _step_matches_oracle(name, prec, groups=None):
    make, contact, mode = CASES[name]
    m = make()
    n = 100
    rng = np.random.default_rng(5)
    q = rng.normal(size=(n, m.nq)) * 0.3
    for i, b in enumerate(m.bodies):
        if b.joint.jtype == 4:  # free joint: lift the base above the ground
            q[:, m.q_offsets[i] + 5] = 0.6 + 0.3 * rng.random(n)
    v = rng.normal(size=(n, m.nv)) * 0.5
    noise = (77, 0, 0.0, 0.5, list(range(m.nv)))
    geom = pack_geometries(m, contact[1], contact[2])[0] if contact else None
    orc = Oracle(m, contact=None if contact is None else (geom, contact[0], contact[3]))
    # Warm into contact on the oracle, then compare one device step.
    c = np.zeros((n, m.nv))
    orc.step_batch(q, v, c, 150, threads=8)
    q, v = as_precision(q, prec), as_precision(v, prec)
    s = _sim(m, n, prec, mode, contact, noise, groups)
    info = s.kernel_info()
    if groups is not None:  # f64 plans keep one subtree per wave whatever the cap
        assert info["block"] == 64 * (groups if prec == "f32" else UNMERGED_WAVES[name])
    s.load_states(q, v, np.zeros((n, m.nv)))
    s.step()
    ctrl = as_precision(s.readback_controls(), prec)
    qdd = s.readback_qdd()
    want = np.zeros_like(qdd)
    for k in range(n):
        ext = orc.contact(q[k], v[k])[0] if contact else None
        want[k] = orc.aba(q[k], v[k], ctrl[k], ext)
    e = rel_err_rows(qdd, want)
    print(f"{name} {prec} mode {mode} groups {groups}: block {info['block']}, qdd err {e.max():.3e}", flush=True)
    if prec == "f64":
        assert e.max() <= 1e-10
    else:
        assert e.max() <= 1e-4
    # The control stream is identical whatever the partition.
    s0 = _sim(m, n, prec, "0", contact, noise)
    s0.load_states(q, v, np.zeros((n, m.nv)))
    s0.step()
    a, b = s0.readback_controls(), s.readback_controls()
    bad = a != b
    if bad.any():
        ulp = np.abs(a.astype(np.float32).view(np.int32).astype(np.int64) - b.astype(np.float32).view(np.int32)).max()
        print(f"controls differ in {bad.sum()} of {bad.size}: dofs {np.where(bad.any(axis=0))[0].tolist()}, "
              f"worlds {np.where(bad.any(axis=1))[0][:12].tolist()}..., max {ulp} ulp (f32); rng states equal: "
              f"{np.array_equal(s0.readback_rng(), s.readback_rng())}; kernels {s0.kernel_info()} / {info}", flush=True)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("name", ["humanoid", "hand", "fixed_base_arms", "random_tree_free"])
def test_partition_modes_agree_on_rollouts(name):
    make, contact, mode = CASES[name]
    m = make()
    n = 130
    rng = np.random.default_rng(8)
    q = rng.normal(size=(n, m.nq)) * 0.2
    for i, b in enumerate(m.bodies):
        if b.joint.jtype == 4:
            q[:, m.q_offsets[i] + 5] = 1.0
    v = rng.normal(size=(n, m.nv)) * 0.2
    outs = []
    for md in ("0", mode):
        s = _sim(m, n, "f64", md, contact, (3, 0, 0.0, 0.3, list(range(m.nv))))
        s.load_states(q, v)
        s.step_many(50)
        outs.append(s.readback_states())
        if contact:
            outs[-1] = outs[-1] + (s.readback_contacts(),)
    d = max(np.abs(outs[0][0] - outs[1][0]).max(), np.abs(outs[0][1] - outs[1][1]).max())
    print(f"{name}: 50-step f64 state difference between partitions {d:.3e}", flush=True)
    assert d <= 1e-9
    if contact:
        assert np.array_equal(outs[0][2][:, :, 0], outs[1][2][:, :, 0])


@pytest.mark.parametrize("name,groups", [("humanoid", 2), ("hand", 4), ("hand", 2)])
def test_merged_groups_match(name, groups):
    """Plans with fewer waves than the tree has parts merge subtrees into one
    wave's code (f32 only: f64 plans keep one subtree per wave under any cap).
    PHZ_MAX_GROUPS forces those plans at a small size: one step gives the
    oracle's qdd in both precisions, f64 rollouts under the cap equal the
    one-lane-per-world kernel's, and a repeated rollout is bit-identical."""
    for prec in ("f64", "f32"):
        _step_matches_oracle(name, prec, groups)
    make, contact, mode = CASES[name]
    m = make()
    n = 130
    rng = np.random.default_rng(9)
    q = rng.normal(size=(n, m.nq)) * 0.2
    for i, b in enumerate(m.bodies):
        if b.joint.jtype == 4:
            q[:, m.q_offsets[i] + 5] = 1.0
    v = rng.normal(size=(n, m.nv)) * 0.2
    noise = (3, 0, 0.0, 0.3, list(range(m.nv)))
    outs = []
    for md, g in (("0", None), (mode, groups), (mode, groups)):
        s = _sim(m, n, "f64", md, contact, noise, g)
        s.load_states(q, v)
        s.step_many(50)
        outs.append(s.readback_states())
    (q0, v0), (qa, va), (qr, vr) = outs
    assert np.array_equal(qa.view(np.uint64), qr.view(np.uint64)) and np.array_equal(va.view(np.uint64), vr.view(np.uint64))
    d = max(np.abs(q0 - qa).max(), np.abs(v0 - va).max())
    print(f"{name} {groups} waves: 50-step f64 state difference {d:.3e}", flush=True)
    assert d <= 1e-9

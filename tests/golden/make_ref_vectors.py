"""Write tests/golden/ref_step_vectors.npz: input/output vectors of the
reference's own step kernels (crates/phyz-gpu/cuda/phyz_kernels.cu compiled as
host C++ by oracle/Makefile into oracle/_ref), for the test models of
tests/models.py and the five benchmark workloads.

Run in a tree where /root/reference is present (after `make -C oracle`):
    python tests/golden/make_ref_vectors.py

Each case stores the f64 body / geometry / PD tables, gravity, dt, the f32
inputs (q, v, ctrl, targets) and the reference's f32 outputs after `steps`
steps: q, v, ctrl, the last step's qdd, ext forces and contact rows.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from phyz_amd import workloads as W  # noqa: E402
from phyz_amd.model import pack_bodies, pack_geometries, pack_pd_dofs, uniform_frequency_gains  # noqa: E402
from tests import models as TM  # noqa: E402
from tests.helpers import oracle_for  # noqa: E402
from tests.ref_host import RefStepper, available  # noqa: E402
from oracle.oracle import Oracle  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_step_vectors.npz")


def f32(a):
    return np.asarray(a, dtype=np.float32).astype(np.float64)


def run_case(store, name, model, q, v, ctrl, steps=1, geom=None, ground_h=0.0, mu=0.0, pd=None, targets=None):
    table = pack_bodies(model)
    nworld = q.shape[0]
    q, v, ctrl = f32(q), f32(v), f32(ctrl)
    if targets is not None:
        targets = f32(targets)
    rs = RefStepper(table, model.nq, model.nv, model.gravity, model.dt, nworld, geom64=geom, ground_h=ground_h, mu=mu,
                    pd64=pd)
    q32, v32, c32 = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, v, ctrl))
    t32 = None if targets is None else np.ascontiguousarray(targets, dtype=np.float32)
    for _ in range(steps):
        qdd, ext, rows = rs.step(q32, v32, c32, t32)
    p = name + "/"
    store[p + "table"] = table
    store[p + "gravity"] = np.asarray(model.gravity, dtype=np.float64)
    store[p + "dt"] = np.array([model.dt])
    store[p + "dims"] = np.array([model.nbodies, model.nq, model.nv, steps])
    store[p + "geom"] = geom if geom is not None else np.zeros((0, 24))
    store[p + "contact"] = np.array([ground_h, mu])
    store[p + "pd"] = pd if pd is not None else np.zeros((0, 8))
    store[p + "targets"] = targets if targets is not None else np.zeros((nworld, 0))
    store[p + "q0"], store[p + "v0"], store[p + "ctrl0"] = q, v, ctrl
    store[p + "q"], store[p + "v"], store[p + "ctrl"] = (a.astype(np.float64) for a in (q32, v32, c32))
    store[p + "qdd"] = qdd.astype(np.float64)
    store[p + "ext"] = ext.astype(np.float64)
    store[p + "rows"] = rows.astype(np.float64)
    print(f"{name}: {nworld} worlds x {steps} steps")


def warm_states(model, nworld, steps, seed, geom=None, mu=0.0, z=(0.15, 0.3)):
    """Drop free bodies with random orientation and velocity; return oracle states after `steps`."""
    rng = np.random.default_rng(seed)
    q = np.zeros((nworld, model.nq))
    q[:, 0:3] = rng.normal(size=(nworld, 3)) * 0.8
    q[:, 5] = rng.uniform(*z, size=nworld)
    v = rng.normal(size=(nworld, model.nv)) * 0.5
    c = np.zeros((nworld, model.nv))
    orc = Oracle(model, contact=None if geom is None else (geom, 0.0, mu))
    orc.step_batch(q, v, c, steps, threads=8)
    return q, v, c


def main():
    if not available():
        raise SystemExit("oracle/_ref/libphyz_ref_host.so missing: run `make -C oracle` with the reference tree present")
    store = {}
    rng = np.random.default_rng(20261201)

    m = TM.double_pendulum_offset()
    q = np.array([[0.3, 0.2], [0.4, -0.3]])
    v = np.array([[0.1, -0.1], [0.0, 0.0]])
    run_case(store, "double_pendulum_1", m, q, v, np.zeros((2, 2)))
    run_case(store, "double_pendulum_200", m, q, v, np.zeros((2, 2)), steps=200)

    m = TM.arm_6dof()
    run_case(store, "arm_6dof", m, np.array([[0.1, -0.2, 0.3, -0.1, 0.2, -0.3]]), np.zeros((1, 6)), np.zeros((1, 6)))
    m = TM.prismatic_model()
    run_case(store, "prismatic", m, np.array([[0.2]]), np.array([[-0.5]]), np.zeros((1, 1)))
    m = TM.ball_joint_model()
    run_case(store, "ball", m, np.array([[0.3, -0.2, 0.1]]), np.array([[0.5, -0.4, 0.3]]), np.zeros((1, 3)))
    m = TM.free_base_with_limb()
    run_case(store, "free_limb", m, np.array([[0.2, -0.1, 0.3, 0.1, 0.2, 0.5, 0.4]]),
             np.array([[0.3, 0, 0, -0.2, 0, 0, 1.0]]), np.zeros((1, 7)))

    m, dofs = TM.pd_link()
    q = np.full((4, 1), 0.3)
    run_case(store, "pd_link_100", m, q, np.zeros((4, 1)), np.zeros((4, 1)), steps=100, pd=pack_pd_dofs(dofs),
             targets=np.full((4, 1), 0.8))

    for k, seed in ((3, 11), (7, 12)):
        m = TM.random_tree(seed, njoints=k)
        n = 4
        q = rng.normal(size=(n, m.nq)) * 0.6
        run_case(store, f"random_tree_{k}", m, q, rng.normal(size=(n, m.nv)), rng.normal(size=(n, m.nv)))

    # Contact: a 1 kg sphere on the ground at omega 200 (cuda_vs_cpu.rs:319-367), and every shape.
    for name, m in TM.shapes().items():
        gains = uniform_frequency_gains(m, 200.0, 1.0) if name == "sphere" else uniform_frequency_gains(m, 50.0, 1.0)
        geom, _ = pack_geometries(m, gains=gains)
        q, v, c = warm_states(m, 16, 250, seed=sum(map(ord, name)), geom=geom, mu=0.8)
        run_case(store, f"contact_{name}", m, q, v, c, geom=geom, mu=0.8)

    for idx in W.ALL:
        w = W.config(idx)
        orc = oracle_for(w)
        n = 24
        q, v, c, tg = w.initial_state(n)
        orc.step_batch(q, v, c, 200, targets=tg, rng=orc.rng_states(n), threads=8)
        geom = None
        if w.contact is not None:
            geom, _ = pack_geometries(w.model, w.contact.stiffness, w.contact.damping)
        run_case(store, f"workload_{w.name}", w.model, q, v, c, geom=geom,
                 ground_h=0.0 if w.contact is None else w.contact.ground_height,
                 mu=0.0 if w.contact is None else w.contact.friction, pd=w.pd_table(), targets=tg)

    np.savez_compressed(OUT, **store)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()

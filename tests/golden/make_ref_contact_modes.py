"""Write tests/golden/ref_contact_modes.npz: the reference's own contact pass
(crates/phyz-gpu/cuda/phyz_kernels.cu:804-1132, compiled as host C++ into
oracle/_ref) on heightfield terrain, with a body-attached plane, and in
impulse mode (leading ABA, then [contact, ABA] x 16 sweeps per step,
crates/phyz-gpu/src/cuda/mod.rs:899-928), from states the oracle brought into
contact.

Run where /root/reference is present (after `make -C oracle`):
    python tests/golden/make_ref_contact_modes.py

Each case stores the f64 tables, the contact configuration, the f32 inputs
(q, v, ctrl; solver state zero) and the reference's f32 outputs after `steps`
steps: q, v, the last qdd, ext forces, the full 56-slot contact state.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from phyz_amd import workloads as W  # noqa: E402
from phyz_amd.model import pack_bodies, pack_geometries, uniform_frequency_gains  # noqa: E402
from tests import models as TM  # noqa: E402
from tests.ref_host import RefStepper, available  # noqa: E402
from oracle.oracle import ContactCfg, Oracle  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_contact_modes.npz")
IMPULSE_ERP = lambda dt: dt / (2.0 * 0.02 * 1.0 + dt)  # noqa: E731  solref_erp_from(0.02, 1.0, dt)


def f32(a):
    return np.asarray(a, dtype=np.float32).astype(np.float64)


def geometry(model, omega, plane=None):
    g, _ = pack_geometries(model, gains=uniform_frequency_gains(model, omega, 1.0))
    if plane is not None:
        g[plane[0], 7] = 1.0
    return g


def settle(model, geom, mu, cfg, nworld, steps, seed, z=(0.15, 0.3), xy=0.0):
    """Random poses dropped onto the terrain and stepped by the oracle."""
    rng = np.random.default_rng(seed)
    q = np.zeros((nworld, model.nq))
    v = rng.normal(size=(nworld, model.nv)) * 0.3
    for i, b in enumerate(model.bodies):
        if b.joint.jtype == 4:
            o = model.q_offsets[i]
            q[:, o:o + 3] = rng.normal(size=(nworld, 3)) * 0.5
            q[:, o + 3:o + 5] = rng.uniform(-xy, xy, size=(nworld, 2))
            q[:, o + 5] = rng.uniform(*z, size=nworld)
    c = np.zeros((nworld, model.nv))
    orc = Oracle(model, contact=(geom, 0.0, mu), contact_cfg=cfg)
    ext = np.zeros((nworld, model.nbodies, 6))
    cs = np.zeros((nworld, model.nbodies, 56))
    orc.step_batch(q, v, c, steps, threads=8, ext_state=ext, cs_state=cs)
    return q, v, c


def run_case(store, name, model, q, v, ctrl, geom, mu, cfg, steps):
    table = pack_bodies(model)
    nworld = q.shape[0]
    q, v, ctrl = f32(q), f32(v), f32(ctrl)
    rs = RefStepper(table, model.nq, model.nv, model.gravity, model.dt, nworld, geom64=geom, ground_h=0.0, mu=mu,
                    cfg=cfg)
    q32, v32, c32 = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, v, ctrl))
    for _ in range(steps):
        qdd, ext, rows = rs.step(q32, v32, c32)
    p = name + "/"
    store[p + "table"] = table
    store[p + "gravity"] = np.asarray(model.gravity, dtype=np.float64)
    store[p + "dt"] = np.array([model.dt])
    store[p + "dims"] = np.array([model.nbodies, model.nq, model.nv, steps])
    store[p + "geom"] = geom
    store[p + "mu"] = np.array([mu])
    store[p + "mode"] = np.array([cfg.solve_mode, cfg.sweeps])
    store[p + "prm"] = cfg.prm
    store[p + "plane"] = np.asarray(cfg.plane if cfg.plane is not None else [-1, 0, 0, 0, 0], dtype=np.float64)
    if cfg.heightfield is not None:
        nx, ny, ox, oy, oz, cell, h = cfg.heightfield
        store[p + "hf"] = np.array([nx, ny, ox, oy, oz, cell])
        store[p + "hf_heights"] = np.asarray(h, dtype=np.float64)
    else:
        store[p + "hf"] = np.zeros(6)
        store[p + "hf_heights"] = np.zeros(0)
    store[p + "q0"], store[p + "v0"], store[p + "ctrl0"] = q, v, ctrl
    store[p + "q"], store[p + "v"] = q32.astype(np.float64), v32.astype(np.float64)
    store[p + "qdd"] = qdd.astype(np.float64)
    store[p + "ext"] = ext.astype(np.float64)
    store[p + "cs"] = rs.cstate.reshape(nworld, model.nbodies, 56).astype(np.float64)
    print(f"{name}: {nworld} worlds x {steps} steps")


def main():
    if not available():
        raise SystemExit("oracle/_ref/libphyz_ref_host.so missing: run `make -C oracle` with the reference tree present")
    store = {}
    hf = TM.bumpy_heightfield()
    shapes = TM.shapes()
    for name in ("sphere", "box", "capsule", "cylinder"):
        m = shapes[name]
        geom = geometry(m, 50.0)
        for mode in (0, 1):
            for terr in ("flat", "hf"):
                if mode == 0 and terr == "flat":
                    continue  # penalty on flat ground: ref_step_vectors.npz
                cfg = ContactCfg(solve_mode=mode, erp=IMPULSE_ERP(m.dt) if mode else 0.001 / 0.041,
                                 heightfield=hf if terr == "hf" else None)
                q, v, c = settle(m, geom, 0.8, cfg, 12, 300, seed=len(name) * 7 + mode, xy=0.8 if terr == "hf" else 0.0)
                tag = f"{'impulse' if mode else 'penalty'}_{terr}_{name}"
                run_case(store, tag + "_1", m, q, v, c, geom, 0.8, cfg, 1)
                run_case(store, tag + "_10", m, q, v, c, geom, 0.8, cfg, 10)
    m = TM.deck_and_feet()
    geom = geometry(m, 50.0, TM.DECK_PLANE)
    for mode in (0, 1):
        cfg = ContactCfg(solve_mode=mode, erp=IMPULSE_ERP(m.dt) if mode else 0.001 / 0.041, plane=TM.DECK_PLANE)
        rng = np.random.default_rng(40 + mode)
        n = 8
        q = np.zeros((n, m.nq))
        q[:, 5] = 0.02
        for k, (o, z) in enumerate(((6, 0.09), (12, 0.06))):  # feet just above the deck's top face (z = 0.04)
            q[:, o:o + 3] = rng.normal(size=(n, 3)) * 0.2
            q[:, o + 3] = rng.uniform(-0.3, 0.3, size=n)
            q[:, o + 4] = rng.uniform(-0.05, 0.05, size=n)
            q[:, o + 5] = z
        v = rng.normal(size=(n, m.nv)) * 0.1
        c = np.zeros((n, m.nv))
        orc = Oracle(m, contact=(geom, 0.0, 0.8), contact_cfg=cfg)
        orc.step_batch(q, v, c, 150, threads=8, ext_state=np.zeros((n, 3, 6)), cs_state=np.zeros((n, 3, 56)))
        tag = f"{'impulse' if mode else 'penalty'}_plane_deck"
        run_case(store, tag + "_1", m, q, v, c, geom, 0.8, cfg, 1)
        run_case(store, tag + "_10", m, q, v, c, geom, 0.8, cfg, 10)
    w = W.config(3)
    geom = geometry(w.model, 60.0)
    cfg = ContactCfg(solve_mode=1, erp=IMPULSE_ERP(w.model.dt))
    q, v, c, _ = w.initial_state(12)
    orc = Oracle(w.model, contact=(geom, 0.0, 1.0), contact_cfg=cfg)
    orc.step_batch(q, v, c, 300, threads=8, ext_state=np.zeros((12, 9, 6)), cs_state=np.zeros((12, 9, 56)))
    run_case(store, "impulse_flat_ant_1", w.model, q, v, c, geom, 1.0, cfg, 1)
    run_case(store, "impulse_flat_ant_5", w.model, q, v, c, geom, 1.0, cfg, 5)
    np.savez_compressed(OUT, **store)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()

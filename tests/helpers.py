"""Shared test helpers: oracle construction for a workload, tolerance metrics."""
from __future__ import annotations

import numpy as np

from oracle.oracle import ContactCfg, Oracle
from phyz_amd.model import pack_geometries


def oracle_for(workload, f32_uniform: bool = False) -> Oracle:
    w = workload
    contact = None
    if w.contact is not None:
        g, _ = w.geometry_table()
        contact = (g, w.contact.ground_height, w.contact.friction)
    noise = None
    if w.noise is not None:
        noise = (w.noise.seed, w.noise.dist, w.noise.a, w.noise.b, w.noise.dofs)
    return Oracle(w.model, contact=contact, pd=w.pd_table(), noise=noise, contact_cfg=contact_cfg_for(w))


def contact_cfg_for(w):
    """The oracle's ContactCfg for a workload's terrain / impulse settings (None: flat penalty)."""
    if w.contact is None or (w.heightfield is None and w.impulse_sweeps == 0):
        return None
    hf = None
    if w.heightfield is not None:
        h = w.heightfield
        hf = (h.nx, h.ny, *h.origin, h.cell, h.nodes())
    if w.impulse_sweeps > 0:
        return ContactCfg(solve_mode=1, sweeps=w.impulse_sweeps, erp=w.impulse_erp(), heightfield=hf)
    return ContactCfg(solve_mode=0, heightfield=hf)


def as_precision(a: np.ndarray, precision: str) -> np.ndarray:
    """Round host f64 data the way the device stores it."""
    if precision == "f32":
        return np.asarray(a, dtype=np.float32).astype(np.float64)
    return np.asarray(a, dtype=np.float64).copy()


def rel_err_rows(got: np.ndarray, want: np.ndarray, floor: float = 1e-12) -> np.ndarray:
    """Per-world normwise error max|got - want| / max(max|want|, floor)."""
    d = np.abs(got - want).max(axis=-1)
    s = np.maximum(np.abs(want).max(axis=-1), floor)
    return d / s


def abs_err_rows(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    return np.abs(got - want).max(axis=-1)


def wrap_angle_diff(a, b):
    d = a - b
    return (d + np.pi) % (2 * np.pi) - np.pi


def late_step_errors(w, sim, prec: str, idx):
    """One more device step of the worlds `idx` from the sim's current state,
    against the oracle: the device's own torques (read back after the step)
    drive an oracle without the control stream; impulse mode starts from the
    device's carried contact forces and warm-start impulses. Returns the
    per-world qdd errors (normwise, relative to max|qdd| of the f64 oracle)
    and, in impulse mode, the carried-state errors."""
    import dataclasses
    imp = w.impulse_sweeps > 0
    qg, vg = sim.readback_states()
    if imp:
        cs0, ext0 = sim.readback_contact_state()
        cs0, ext0 = np.ascontiguousarray(cs0[idx]), np.ascontiguousarray(ext0[idx])
    sim.step()
    ctrl = as_precision(sim.readback_controls(), prec)
    qdd = sim.readback_qdd()
    extra = {}
    if not imp and w.heightfield is None:
        orc = oracle_for(w)
        ext = [orc.contact(qg[k], vg[k])[0] if w.contact is not None else None for k in idx]
        want = np.stack([orc.aba(qg[k], vg[k], ctrl[k], ext[i]) for i, k in enumerate(idx)])
    else:
        orc = oracle_for(dataclasses.replace(w, noise=None))
        q, v, c = (np.ascontiguousarray(a[idx]) for a in (qg, vg, ctrl))
        want, _ = orc.step_batch(q, v, c, 1, threads=8, ext_state=ext0 if imp else None,
                                 cs_state=cs0 if imp else None)
        if imp:
            cs1, ext1 = sim.readback_contact_state()
            es = max(float(np.abs(ext0).max()), 1.0)
            extra["contact_force_rel_err_max"] = float(np.abs(ext1[idx] - ext0).max() / es)
            isc = max(float(np.abs(cs0[:, :, 8:]).max()), 1e-6)
            extra["impulse_rel_err_max"] = float(np.abs(cs1[idx, :, 8:] - cs0[:, :, 8:]).max() / isc)
    return rel_err_rows(qdd[idx], want), extra

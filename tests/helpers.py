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

"""ctypes wrapper over oracle/liboracle.so — TEST INFRASTRUCTURE ONLY.

Used by tests/, by __graft_entry__.smoke() as the checker, and by bench.py's
cpu_baseline leg. The product (phyz_amd) never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libphyz_ref_host.so")

_lib = None

dp = C.POINTER(C.c_double)
fp = C.POINTER(C.c_float)
u64p = C.POINTER(C.c_uint64)


def build(quiet: bool = True) -> None:
    """Compile the oracle (and oracle/_ref where the reference tree exists)."""
    out = subprocess.run(["make", "-C", HERE, "all"], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_model_create.restype = C.c_void_p
        L.orc_model_create.argtypes = [dp, C.c_int, C.c_int, C.c_int, dp, C.c_double, C.c_char_p, C.c_int]
        L.orc_model_destroy.argtypes = [C.c_void_p]
        L.orc_set_contact.argtypes = [C.c_void_p, dp, C.c_double, C.c_double]
        L.orc_set_pd.argtypes = [C.c_void_p, dp, C.c_int]
        L.orc_set_noise.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_double, C.c_double, C.POINTER(C.c_int), C.c_int]
        L.orc_aba.argtypes = [C.c_void_p, dp, dp, dp, dp, dp, C.c_int]
        L.orc_aba_f32.argtypes = [C.c_void_p, fp, fp, fp, fp, fp]
        L.orc_rnea.argtypes = [C.c_void_p, dp, dp, dp, dp, dp]
        L.orc_qdd_f32.argtypes = [C.c_void_p, fp, fp, fp, fp]
        L.orc_crba.argtypes = [C.c_void_p, dp, dp]
        L.orc_generalized_forces.argtypes = [C.c_void_p, dp, dp, dp, dp]
        L.orc_fk.argtypes = [C.c_void_p, dp, dp, dp]
        L.orc_fk_batch.argtypes = [C.c_void_p, C.c_int, dp, dp, dp, C.c_int]
        L.orc_contact.argtypes = [C.c_void_p, dp, dp, dp, dp]
        L.orc_integrate.argtypes = [C.c_void_p, dp, dp, dp]
        L.orc_world_seed.restype = C.c_uint64
        L.orc_world_seed.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_quat_exp_log.argtypes = [dp, dp, dp]
        L.orc_step_batch.argtypes = [C.c_void_p, C.c_int, C.c_int, dp, dp, dp, dp, u64p, dp, dp, C.c_int, C.c_int, dp, dp]
        L.orc_set_contact_cfg.argtypes = [C.c_void_p, C.c_int, C.c_int, dp, C.c_int, dp, C.c_int, C.c_int, dp, dp]
        L.orc_contact_pass.argtypes = [C.c_void_p, dp, dp, dp, dp, dp]
        L.orc_set_joint_terms.argtypes = [C.c_void_p, dp]
        L.orc_set_actuators.argtypes = [C.c_void_p, dp, C.c_int]
        L.orc_count_ops.argtypes = [C.c_void_p, dp, dp, dp, dp, C.c_uint64, C.c_int, u64p, dp, dp]
        _lib = L
    return _lib


def _d(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.float64 and a.flags.c_contiguous
    return a.ctypes.data_as(dp)


PHASES = ("noise", "pd", "contact", "aba", "integrate")
COUNTERS = ("add", "mul", "div", "sqrt", "trans", "other")


class Oracle:
    """f64 CPU restatement of one model's step (see oracle/phz_oracle.hpp)."""

    def __init__(self, model=None, contact=None, pd=None, noise=None, tables=None, contact_cfg=None):
        """From a phyz_amd.model.Model, or from raw tables=(body_table, nq, nv, gravity, dt).

        contact = (geometry table, ground height, friction); contact_cfg (a
        ContactCfg) adds impulse mode, the body-attached plane and heightfield
        terrain to it."""
        L = lib()
        if tables is not None:
            table, nq, nv, gravity, dt = tables
            self.model = None
            self.nb, self.nq, self.nv = table.shape[0], int(nq), int(nv)
        else:
            from phyz_amd.model import pack_bodies
            table, gravity, dt = pack_bodies(model), model.gravity, model.dt
            self.model = model
            self.nb, self.nq, self.nv = model.nbodies, model.nq, model.nv
        table = np.ascontiguousarray(table, dtype=np.float64)
        g = np.ascontiguousarray(gravity, dtype=np.float64)
        err = C.create_string_buffer(256)
        h = L.orc_model_create(_d(table), self.nb, self.nq, self.nv, _d(g), float(dt), err, 256)
        if not h:
            raise ValueError(err.value.decode())
        self._h = C.c_void_p(h)
        self.n_pd = 0
        self.noise = None
        if contact is not None:
            geom, ground_h, mu = contact
            L.orc_set_contact(self._h, _d(np.ascontiguousarray(geom, dtype=np.float64)), float(ground_h), float(mu))
        if pd is not None:
            t = np.ascontiguousarray(pd, dtype=np.float64)
            self.n_pd = t.shape[0]
            L.orc_set_pd(self._h, _d(t), self.n_pd)
        if noise is not None:
            seed, dist, a, b, dofs = noise
            arr = (C.c_int * len(dofs))(*dofs)
            L.orc_set_noise(self._h, int(seed), int(dist), float(a), float(b), arr, len(dofs))
            self.noise = noise
        self.cfg = contact_cfg
        if contact_cfg is not None:
            contact_cfg.apply(L, self._h)
        self.nctrl = self.nv
        if model is not None:
            from phyz_amd.model import pack_actuators, pack_joint_terms
            if model.has_joint_terms():
                self.set_joint_terms(pack_joint_terms(model))
            if model.actuators:
                self.set_actuators(pack_actuators(model))

    def set_joint_terms(self, table):
        """Limits and friction loss, nb x 8 (phyz_amd.model.pack_joint_terms)."""
        t = np.ascontiguousarray(table, dtype=np.float64).reshape(self.nb, 8)
        lib().orc_set_joint_terms(self._h, _d(t))

    def set_actuators(self, table):
        """Actuators, nu x 16 (phyz_amd.model.pack_actuators); ctrl becomes nu wide."""
        t = np.ascontiguousarray(table, dtype=np.float64).reshape(-1, 16)
        if lib().orc_set_actuators(self._h, _d(t), t.shape[0]):
            raise ValueError("actuator on a body without a moving joint")
        self.nctrl = t.shape[0] if t.shape[0] else self.nv

    def __del__(self):
        if getattr(self, "_h", None) is not None and _lib is not None:
            _lib.orc_model_destroy(self._h)
            self._h = None

    # ── single-world calls ──
    def aba(self, q, v, ctrl, ext=None, dense=False):
        out = np.zeros(self.nv)
        lib().orc_aba(self._h, _d(np.ascontiguousarray(q, dtype=np.float64)), _d(np.ascontiguousarray(v, dtype=np.float64)),
                      _d(np.ascontiguousarray(ctrl, dtype=np.float64)),
                      _d(None if ext is None else np.ascontiguousarray(ext, dtype=np.float64)), _d(out), 1 if dense else 0)
        return out

    def aba_f32(self, q, v, ctrl, ext=None):
        f = lambda a: np.ascontiguousarray(a, dtype=np.float32)
        out = np.zeros(self.nv, dtype=np.float32)
        qq, vv, cc = f(q), f(v), f(ctrl)
        ee = None if ext is None else f(ext)
        lib().orc_aba_f32(self._h, qq.ctypes.data_as(fp), vv.ctypes.data_as(fp), cc.ctypes.data_as(fp),
                          None if ee is None else ee.ctypes.data_as(fp), out.ctypes.data_as(fp))
        return out

    def qdd_f32(self, q, v, ctrl):
        """One step's qdd (with contact when enabled) computed in f32 arithmetic."""
        f = lambda a: np.ascontiguousarray(a, dtype=np.float32)
        out = np.zeros(self.nv, dtype=np.float32)
        qq, vv, cc = f(q), f(v), f(ctrl)
        lib().orc_qdd_f32(self._h, qq.ctypes.data_as(fp), vv.ctypes.data_as(fp), cc.ctypes.data_as(fp),
                          out.ctypes.data_as(fp))
        return out.astype(np.float64)

    def rnea(self, q, v, qdd, ext=None):
        out = np.zeros(self.nv)
        lib().orc_rnea(self._h, _d(np.ascontiguousarray(q, dtype=np.float64)), _d(np.ascontiguousarray(v, dtype=np.float64)),
                       _d(np.ascontiguousarray(qdd, dtype=np.float64)),
                       _d(None if ext is None else np.ascontiguousarray(ext, dtype=np.float64)), _d(out))
        return out

    def crba(self, q):
        out = np.zeros((self.nv, self.nv))
        lib().orc_crba(self._h, _d(np.ascontiguousarray(q, dtype=np.float64)), _d(out))
        return out

    def generalized_forces(self, q, v, ctrl):
        out = np.zeros(self.nv)
        lib().orc_generalized_forces(self._h, _d(np.ascontiguousarray(q, dtype=np.float64)),
                                     _d(np.ascontiguousarray(v, dtype=np.float64)),
                                     _d(np.ascontiguousarray(ctrl, dtype=np.float64)), _d(out))
        return out

    def fk(self, q, v):
        out = np.zeros((self.nb, 18))
        lib().orc_fk(self._h, _d(np.ascontiguousarray(q, dtype=np.float64)), _d(np.ascontiguousarray(v, dtype=np.float64)), _d(out))
        return out

    def fk_batch(self, q, v, threads=1):
        """fk over world-major states: [nworld][nb][18]."""
        q = np.ascontiguousarray(q, dtype=np.float64)
        v = np.ascontiguousarray(v, dtype=np.float64)
        out = np.zeros((q.shape[0], self.nb, 18))
        lib().orc_fk_batch(self._h, q.shape[0], _d(q), _d(v), _d(out), int(threads))
        return out

    def contact(self, q, v):
        ext = np.zeros((self.nb, 6))
        rows = np.zeros((self.nb, 8))
        rc = lib().orc_contact(self._h, _d(np.ascontiguousarray(q, dtype=np.float64)),
                               _d(np.ascontiguousarray(v, dtype=np.float64)), _d(ext), _d(rows))
        if rc != 0:
            raise RuntimeError("contact not enabled on this oracle")
        return ext, rows

    def integrate(self, q, v, qdd):
        q = np.array(q, dtype=np.float64)
        v = np.array(v, dtype=np.float64)
        lib().orc_integrate(self._h, _d(q), _d(v), _d(np.ascontiguousarray(qdd, dtype=np.float64)))
        return q, v

    # ── batch stepping ──
    def rng_states(self, nworld: int) -> np.ndarray:
        if self.noise is None:
            return None
        seed = int(self.noise[0])
        return np.array([lib().orc_world_seed(seed, w) for w in range(nworld)], dtype=np.uint64)

    def contact_pass(self, q, v, cs=None):
        """One contact pass at velocity v (the free velocity in impulse mode).
        cs: nb x 56 solver state, updated in place. Returns (ext, rows)."""
        ext = np.zeros((self.nb, 6))
        rows = np.zeros((self.nb, 8))
        if cs is not None:
            assert cs.dtype == np.float64 and cs.flags.c_contiguous and cs.size == self.nb * 56
        lib().orc_contact_pass(self._h, _d(np.ascontiguousarray(q, dtype=np.float64)),
                               _d(np.ascontiguousarray(v, dtype=np.float64)), _d(ext), _d(cs), _d(rows))
        return ext, rows

    def step_batch(self, q, v, ctrl, nsteps, targets=None, rng=None, threads=1, dense=False, want_contacts=False,
                   ext_state=None, cs_state=None):
        """Advance world-major (q, v, ctrl) in place by nsteps. Returns (qdd_last, contact_rows|None).
        ext_state [nworld][nb][6] / cs_state [nworld][nb][56]: impulse-mode solver state, in and out."""
        nworld = q.shape[0]
        assert q.dtype == np.float64 and q.flags.c_contiguous
        qdd = np.zeros((nworld, self.nv))
        rows = np.zeros((nworld, self.nb, 8)) if want_contacts else None
        tg = None
        if self.n_pd:
            tg = np.ascontiguousarray(targets, dtype=np.float64)
        rp = None
        if rng is not None:
            assert rng.dtype == np.uint64 and rng.flags.c_contiguous
            rp = rng.ctypes.data_as(u64p)
        for a in (ext_state, cs_state):
            if a is not None:
                assert a.dtype == np.float64 and a.flags.c_contiguous
        lib().orc_step_batch(self._h, nworld, int(nsteps), _d(q), _d(v), _d(ctrl), _d(tg), rp, _d(qdd),
                             _d(rows), int(threads), 1 if dense else 0, _d(ext_state), _d(cs_state))
        return qdd, rows

    def count_ops(self, q, v, ctrl, targets=None, rng_state=1, dense=False, ext_state=None, cs_state=None):
        """Per-phase operation counts of one world-step: {phase: {counter: n}}.
        ext_state [nb][6] / cs_state [nb][56]: impulse-mode carried state (default zero)."""
        c = np.zeros(len(PHASES) * len(COUNTERS), dtype=np.uint64)
        tg = np.ascontiguousarray(targets if targets is not None else np.zeros(max(self.n_pd, 1)), dtype=np.float64)
        e = None if ext_state is None else np.ascontiguousarray(np.asarray(ext_state, dtype=np.float64).reshape(self.nb, 6))
        s = None if cs_state is None else np.ascontiguousarray(np.asarray(cs_state, dtype=np.float64).reshape(self.nb, 56))
        lib().orc_count_ops(self._h, _d(np.ascontiguousarray(q, dtype=np.float64)), _d(np.ascontiguousarray(v, dtype=np.float64)),
                            _d(np.ascontiguousarray(ctrl, dtype=np.float64)), _d(tg), int(rng_state), 1 if dense else 0,
                            c.ctypes.data_as(u64p), _d(e), _d(s))
        c = c.reshape(len(PHASES), len(COUNTERS))
        return {p: {k: int(c[i, j]) for j, k in enumerate(COUNTERS)} for i, p in enumerate(PHASES)}


def world_seed(seed: int, world: int) -> int:
    return int(lib().orc_world_seed(int(seed), int(world)))


def quat_exp_log(w):
    q = np.zeros(4)
    l = np.zeros(3)
    lib().orc_quat_exp_log(_d(np.ascontiguousarray(w, dtype=np.float64)), _d(q), _d(l))
    return q, l


class ContactCfg:
    """Impulse mode, body-attached plane and heightfield terrain for the oracle
    (ContactParams, crates/phyz-gpu/src/contact_pipeline.rs:17-100; defaults of
    GroundContactParams::default, 197-222)."""

    def __init__(self, solve_mode=0, sweeps=16, restitution=0.0, restitution_threshold=0.05,
                 erp=0.001 / (2.0 * 0.02 + 0.001), margin=0.001, solimp=(0.9, 0.95, 0.001, 0.5, 2.0), plane=None,
                 heightfield=None):
        """plane: (body, offset, max_depth, half_x, half_y); heightfield: (nx, ny, ox, oy, oz, cell, heights)."""
        self.solve_mode, self.sweeps = int(solve_mode), int(sweeps)
        self.prm = np.array([restitution, restitution_threshold, erp, margin, *solimp], dtype=np.float64)
        self.plane = plane
        self.heightfield = heightfield

    def apply(self, L, h):
        pb, pl = -1, np.zeros(4)
        if self.plane is not None:
            pb = int(self.plane[0])
            pl = np.array(self.plane[1:5], dtype=np.float64)
        nx = ny = 0
        hf = np.zeros(4)
        heights = None
        if self.heightfield is not None:
            nx, ny, ox, oy, oz, cell, hh = self.heightfield
            hf = np.array([ox, oy, oz, cell], dtype=np.float64)
            heights = np.ascontiguousarray(np.asarray(hh, dtype=np.float64).ravel())
        L.orc_set_contact_cfg(h, self.solve_mode, self.sweeps, _d(self.prm), pb, _d(pl), int(nx), int(ny), _d(hf),
                              _d(heights))


# ── chaos classification (crates/phyz/src/determinism.rs:164-382) ───────────
def ulp_offset(x: float, n: int) -> float:
    """x moved n representable f64 steps toward +inf (n < 0: toward -inf), on
    the sign-magnitude total order; NaN and infinities unchanged
    (determinism.rs:180-224)."""
    x = float(x)
    if n == 0 or not np.isfinite(x):
        return x
    bits = int(np.array(x, dtype=np.float64).view(np.int64))
    key = bits if bits >= 0 else -(1 << 63) - bits
    lo, hi = -0x7FEFFFFFFFFFFFFF, 0x7FEFFFFFFFFFFFFF  # -f64::MAX, f64::MAX on the ordered line
    key = min(max(key + int(n), lo), hi)
    bits = key if key >= 0 else -(1 << 63) - key
    return float(np.array(bits, dtype=np.int64).view(np.float64))


def ulps_between(a: float, b: float) -> int:
    """Representable f64 steps from a to b (determinism.rs:201-207); i64::MAX
    when either is not finite."""
    if not (np.isfinite(a) and np.isfinite(b)):
        return (1 << 63) - 1

    def key(x):
        bits = int(np.array(float(x), dtype=np.float64).view(np.int64))
        return bits if bits >= 0 else -(1 << 63) - bits
    return max(min(key(b) - key(a), (1 << 63) - 1), -(1 << 63))


def state_distance(q0, v0, q1, v1) -> np.ndarray:
    """Per-world Euclidean distance over the stacked (q, v) vector; inf for a
    world where either state is not finite (determinism.rs:235-253)."""
    d = np.concatenate([np.asarray(q0) - np.asarray(q1), np.asarray(v0) - np.asarray(v1)], axis=-1)
    out = np.sqrt(np.sum(d * d, axis=-1))
    return np.where(np.isfinite(d).all(axis=-1), out, np.inf)


def one_ulp_divergence(orc: "Oracle", q, v, ctrl, nsteps: int, q_index=None, targets=None, ulps: int = 1,
                       threads: int = 8):
    """Two oracle rollouts of every world, nsteps each: one from (q, v), one
    with q[:, q_index] moved `ulps` representable steps (determinism.rs:333-382,
    per world, both rollouts replaying the same control stream). q_index None
    moves every coordinate of q, so no symmetry direction of the model (a
    hinge about the gravity axis) can hide a growing one. Returns (initial
    distance, final distance, final q, final v of the unperturbed rollout),
    one entry per world."""
    qa, va, ca = (np.array(a, dtype=np.float64, order="C") for a in (q, v, ctrl))
    qb, vb, cb = qa.copy(), va.copy(), ca.copy()
    cols = range(qb.shape[1]) if q_index is None else [q_index]
    for j in cols:
        qb[:, j] = [ulp_offset(x, ulps) for x in qb[:, j]]
    d0 = state_distance(qa, va, qb, vb)
    n = qa.shape[0]
    orc.step_batch(qa, va, ca, nsteps, targets=targets, rng=orc.rng_states(n), threads=threads)
    orc.step_batch(qb, vb, cb, nsteps, targets=targets, rng=orc.rng_states(n), threads=threads)
    return d0, state_distance(qa, va, qb, vb), qa, va

"""The reference's own kernels, compiled as host C++ (oracle/_ref), driven in
the reference's f32 wire format — TEST INFRASTRUCTURE ONLY.

oracle/Makefile builds crates/phyz-gpu/cuda/phyz_kernels.cu as host C++, the
reference's `cuda-host` build (crates/phyz-gpu/build.rs:7-19). Its entry points
phyz_host_{pd,contact,aba,integrate} (phyz_kernels.cu:1779-1802) and
phyz_host_{fk,obs,policy} (1809-1835) walk the grid serially. This module packs buffers exactly as crates/phyz-gpu/src/layout.rs
and crates/phyz-gpu/src/contact_pipeline.rs:60-100 do (f32, integer slots
bit-cast) and runs the reference step order of
crates/phyz-gpu/src/cuda/mod.rs:879-945 (PD, contact, ABA, integrate; in
impulse mode PD, ABA, then [contact, ABA] x sweeps, integrate).
"""
from __future__ import annotations

import ctypes as C
import os
import struct

import numpy as np

from oracle.oracle import REF_LIB_PATH

fp = C.POINTER(C.c_float)
_lib = None


def available() -> bool:
    return os.path.exists(REF_LIB_PATH)


def lib():
    global _lib
    if _lib is None:
        L = C.CDLL(REF_LIB_PATH)
        u = C.c_uint32
        L.phyz_host_pd.argtypes = [u, u, u, u, u, fp, fp, fp, fp, fp]
        L.phyz_host_contact.argtypes = [u, fp, fp, fp, fp, fp, fp, fp, fp, fp]
        L.phyz_host_aba.argtypes = [u, u, u, C.c_float, u, C.c_float, C.c_float, C.c_float, fp, fp, fp, fp, fp, fp]
        L.phyz_host_integrate.argtypes = [u, u, u, C.c_float, u, fp, fp, fp, fp]
        L.phyz_host_fk.argtypes = [u, u, u, u, fp, fp, fp, fp]
        L.phyz_host_obs.argtypes = [u, u, u, u, u, u, u, fp, fp, fp, fp, fp, fp, fp]
        L.phyz_host_policy.argtypes = [u, u, u, u, u, u, C.c_float, u, C.c_float, u, u, fp, fp, fp, fp, fp, fp, fp,
                                       fp, fp, fp, fp]
        _lib = L
    return _lib


def _bits_i32(x: int) -> float:
    return struct.unpack("<f", struct.pack("<i", int(x)))[0]


def _bits_u32(x: int) -> float:
    return struct.unpack("<f", struct.pack("<I", int(x)))[0]


def pack_bodies_f32(table64: np.ndarray) -> np.ndarray:
    """layout.rs:103-156: f32 body table with parent/jtype/offsets bit-cast."""
    nb = table64.shape[0]
    t = np.zeros((nb, 36), dtype=np.float32)
    for i in range(nb):
        t[i, 0] = _bits_i32(table64[i, 0])
        t[i, 1] = _bits_u32(table64[i, 1])
        t[i, 2] = _bits_u32(table64[i, 2])
        t[i, 3] = _bits_u32(table64[i, 3])
        t[i, 4:33] = table64[i, 4:33].astype(np.float32)
    return t


def pack_cparams(nworld, nb, nv, ground_h, dt, mu, cfg=None) -> np.ndarray:
    """ContactParams::pack (contact_pipeline.rs:60-100). Without cfg: penalty mode,
    flat ground, defaults; cfg (oracle.oracle.ContactCfg) sets the solve mode,
    solver parameters, body-attached plane and heightfield header."""
    if cfg is not None:
        p = pack_cparams(nworld, nb, nv, ground_h, dt, mu)
        if cfg.plane is not None:
            p[6] = _bits_i32(int(cfg.plane[0]))
            p[7:11] = cfg.plane[1:5]
        if cfg.heightfield is not None:
            nx, ny, ox, oy, oz, cell, _ = cfg.heightfield
            p[11], p[12] = _bits_u32(nx), _bits_u32(ny)
            p[13:17] = [ox, oy, oz, cell]
        p[17] = _bits_u32(cfg.solve_mode)
        p[19:28] = cfg.prm
        return p
    p = np.zeros(32, dtype=np.float32)
    p[0] = _bits_u32(nworld)
    p[1] = _bits_u32(nb)
    p[2] = _bits_u32(nv)
    p[3] = ground_h
    p[4] = dt
    p[5] = mu
    p[6] = _bits_i32(-1)          # no body-attached plane
    p[11] = _bits_u32(0)          # hf_nx = 0: flat ground
    p[12] = _bits_u32(0)
    p[16] = 1.0                   # hf_cell
    p[17] = _bits_u32(0)          # solve_mode penalty
    p[20] = 0.05                  # restitution_threshold
    p[21] = 0.001 / (2.0 * 0.02 + 0.001)
    p[22] = 0.001                 # margin
    p[23:28] = [0.9, 0.95, 0.001, 0.5, 2.0]
    return p


class RefStepper:
    """Reference f32 kernels on the host for `nworld` worlds of one model."""

    def __init__(self, table64, nq, nv, gravity, dt, nworld, geom64=None, ground_h=0.0, mu=0.0, pd64=None, cfg=None):
        self.L = lib()
        self.nb = table64.shape[0]
        self.nq, self.nv, self.nworld = nq, nv, nworld
        self.gravity = np.asarray(gravity, dtype=np.float32)
        self.dt = np.float32(dt)
        self.bodies = np.ascontiguousarray(pack_bodies_f32(table64).reshape(-1))
        self.contact = geom64 is not None
        if self.contact:
            self.geom = np.ascontiguousarray(np.asarray(geom64, dtype=np.float32).reshape(-1))
            self.cparams = pack_cparams(nworld, self.nb, nv, ground_h, dt, mu, cfg)
        self.pd = None if pd64 is None else np.ascontiguousarray(np.asarray(pd64, dtype=np.float32).reshape(-1))
        self.npd = 0 if pd64 is None else len(pd64)
        self.ext = np.zeros(nworld * self.nb * 6, dtype=np.float32)
        self.cstate = np.zeros(nworld * self.nb * 56, dtype=np.float32)
        self.hf = np.zeros(1, dtype=np.float32)
        self.sweeps = 0
        if cfg is not None:
            if cfg.heightfield is not None:
                self.hf = np.ascontiguousarray(np.asarray(cfg.heightfield[6], dtype=np.float32).ravel())
            if cfg.solve_mode == 1:
                self.sweeps = cfg.sweeps
        self.qdd = np.zeros(nworld * nv, dtype=np.float32)

    @staticmethod
    def _p(a):
        return a.ctypes.data_as(fp)

    def step(self, q, v, ctrl, targets=None):
        """One reference step in place on f32 world-major arrays. Returns (qdd, ext, contact rows)."""
        L, P = self.L, self._p
        n = self.nworld
        if self.npd:
            L.phyz_host_pd(n * self.npd, n, self.nq, self.nv, self.npd, P(self.pd), P(q), P(v), P(targets), P(ctrl))
        g = self.gravity

        def contact():
            L.phyz_host_contact(n, P(self.cparams), P(self.bodies), P(self.geom), P(q), P(v), P(self.ext),
                                P(self.cstate), P(self.hf), P(self.qdd))

        def aba():
            L.phyz_host_aba(n, n, self.nv, self.dt, self.nb, float(g[0]), float(g[1]), float(g[2]), P(self.bodies),
                            P(q), P(v), P(ctrl), P(self.qdd), P(self.ext))

        if self.contact and self.sweeps > 0:
            # Impulse mode (mod.rs:899-928): leading ABA, then [contact, ABA] x sweeps.
            aba()
            for _ in range(self.sweeps):
                contact()
                aba()
        else:
            if self.contact:
                contact()
            aba()
        L.phyz_host_integrate(n * self.nb, n, self.nv, self.dt, self.nb, P(q), P(v), P(self.qdd), P(self.bodies))
        rows = self.cstate.reshape(n, self.nb, 56)[:, :, :8].copy()
        return self.qdd.reshape(n, self.nv).copy(), self.ext.reshape(n, self.nb, 6).copy(), rows


class RefControl:
    """The reference's FK readout, observation and policy passes on the host
    (phyz_host_fk / phyz_host_obs / phyz_host_policy) for `nworld` worlds: f32
    buffers in the reference's layouts (policy_pipeline.rs:285-297 for the op
    table, [mass, com] per body, the policy weights W1 b1 W2 b2 W3 b3)."""

    def __init__(self, table64, model, spec, weights, std, n_dofs, nworld):
        from phyz_amd.policy import pack_obs_ops
        self.L = lib()
        self.nb, self.nq, self.nv, self.nworld = table64.shape[0], model.nq, model.nv, nworld
        self.bodies = np.ascontiguousarray(pack_bodies_f32(table64).reshape(-1))
        ops, aux = pack_obs_ops(spec.obs)
        self.ops = np.ascontiguousarray(ops.astype(np.float32).reshape(-1))
        self.aux = np.ascontiguousarray(np.asarray(aux if len(aux) else [0.0], dtype=np.float32))
        self.com = np.ascontiguousarray(np.array([[b.inertia.mass, *b.inertia.com] for b in model.bodies],
                                                 dtype=np.float32).reshape(-1))
        self.spec = spec
        self.n_in, self.n_h, self.n_out, self.n_dofs = spec.n_in(), spec.hidden, spec.n_out(), n_dofs
        self.weights = np.ascontiguousarray(np.asarray(weights, dtype=np.float32))
        self.std = np.ascontiguousarray(np.asarray(std, dtype=np.float32))
        self.in_noise = np.ascontiguousarray(np.asarray(spec.input_noise, dtype=np.float32))
        self.slots = np.ascontiguousarray(np.asarray(spec.act_slots, dtype=np.float32))
        cs = spec.act_clamp_slots
        self.clamp_slots = np.ascontiguousarray(np.asarray(cs if cs is not None else [0.0], dtype=np.float32))

    P = staticmethod(lambda a: a.ctypes.data_as(fp))

    def fk(self, q32, v32):
        xf = np.zeros(self.nworld * self.nb * 18, dtype=np.float32)
        self.L.phyz_host_fk(self.nworld, self.nworld, self.nv, self.nb, self.P(self.bodies), self.P(q32),
                            self.P(v32), self.P(xf))
        return xf

    def obs(self, q32, v32, xf):
        o = np.zeros(self.nworld * self.n_in, dtype=np.float32)
        self.L.phyz_host_obs(self.nworld, self.nworld, self.nq, self.nv, self.nb, self.n_in, 0, self.P(self.ops),
                             self.P(self.aux), self.P(self.com), self.P(q32), self.P(v32), self.P(xf), self.P(o))
        return o

    def policy(self, obs, rng, z, base_targets):
        """One policy pass in place on obs (input noise), rng words and z.
        Returns (targets [nworld][n_dofs], out [nworld][n_out + 1])."""
        tg = np.zeros(self.nworld * self.n_dofs, dtype=np.float32)
        out = np.zeros(self.nworld * (self.n_out + 1), dtype=np.float32)
        sp = self.spec
        self.L.phyz_host_policy(self.nworld, self.nworld, self.n_in, self.n_h, self.n_out, self.n_dofs,
                                float(sp.act_clamp), 1 if sp.act_clamp_slots is not None else 0, float(sp.noise_rho),
                                0, 0, self.P(self.weights), self.P(self.std), self.P(self.in_noise), self.P(obs),
                                self.P(rng), self.P(z), self.P(self.slots), self.P(self.clamp_slots),
                                self.P(base_targets), self.P(tg), self.P(out))
        return tg.reshape(self.nworld, self.n_dofs), out.reshape(self.nworld, self.n_out + 1)

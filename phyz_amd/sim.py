"""BatchSim — Python binding with the reference's batched-simulator surface.

Method names, argument meaning and error behaviour follow
crates/phyz-gpu/src/cuda/mod.rs:430-1003 (BatchSim<B>): build from a model and
a world count, optionally enable ground contact and PD servos, then
load_states / set_controls / step / step_many / readback_states /
readback_contacts. Errors raise PhzError with the library's message, where the
reference returns Err(String) (try_step, enable_*) or panics (step).
Everything here calls the HIP library through its C ABI; there is no CPU path.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import numpy as np

from . import _lib
from .model import Model, PdDof, pack_actuators, pack_bodies, pack_geometries, pack_joint_terms, pack_pd_dofs
from .policy import XF_STRIDE, PolicySpec, pack_obs_ops

F32, F64 = 0, 1
NOISE_NORMAL, NOISE_UNIFORM = 0, 1


class PhzError(RuntimeError):
    pass


def _dp(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(_lib.dp)


def _rows(a, n, width, name) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float64))
    if a.shape != (n, width):
        raise ValueError(f"{name}: expected shape {(n, width)}, got {a.shape}")
    return a


class BatchSim:
    """`nworld` copies of one model stepped in lockstep on one MI355X."""

    def __init__(self, model: Model, nworld: int, precision: str = "f32", device: int = 0, model_terms: bool = True):
        """model_terms: apply the model's actuators, joint limits and friction
        loss (terms of the reference's CPU model that its device pass leaves
        out); ctrl then holds one control per actuator."""
        self._L = _lib.load()
        self.model = model
        self.nworld = int(nworld)
        self.precision = precision
        self.nb, self.nq, self.nv = model.nbodies, model.nq, model.nv
        self._npd = 0
        table = np.ascontiguousarray(pack_bodies(model))
        g = np.ascontiguousarray(model.gravity, dtype=np.float64)
        h = C.c_void_p()
        rc = self._L.phz_sim_create(_dp(table), self.nb, self.nq, self.nv, _dp(g), float(model.dt), self.nworld,
                                    F64 if precision == "f64" else F32, int(device), C.byref(h))
        if rc != 0:
            raise PhzError(self._L.phz_last_error(None).decode())
        self._h = h
        if model_terms:
            if model.has_joint_terms():
                self.set_joint_terms(pack_joint_terms(model))
            if model.actuators:
                self.set_actuators(pack_actuators(model))

    # ── model terms beyond the device body table ──
    def set_joint_terms(self, table: Optional[np.ndarray]):
        """Limits and friction loss per body, nb x 8 (phyz_amd.model.pack_joint_terms); None clears."""
        t = None if table is None else np.ascontiguousarray(np.asarray(table, dtype=np.float64).reshape(self.nb, 8))
        self._check(self._L.phz_set_joint_terms(self._h, _dp(t)))

    def set_actuators(self, table: Optional[np.ndarray]):
        """Actuators, nu x 16 (phyz_amd.model.pack_actuators); None or no rows clears.
        Controls become one per actuator (zeroed)."""
        t = None if table is None else np.ascontiguousarray(np.asarray(table, dtype=np.float64).reshape(-1, 16))
        n = 0 if t is None else t.shape[0]
        self._check(self._L.phz_set_actuators(self._h, _dp(t), n))

    @property
    def nctrl(self) -> int:
        """Controls per world: one per actuator, or one per DOF."""
        return int(self._L.phz_nctrl(self._h))

    # ── lifecycle ──
    def close(self):
        if getattr(self, "_h", None):
            self._L.phz_sim_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int):
        if rc != 0:
            raise PhzError(self._L.phz_last_error(self._h).decode())

    # ── model / configuration ──
    def set_model(self, model: Model):
        table = np.ascontiguousarray(pack_bodies(model))
        g = np.ascontiguousarray(model.gravity, dtype=np.float64)
        self._check(self._L.phz_set_model(self._h, _dp(table), model.nbodies, model.nq, model.nv, _dp(g), float(model.dt)))
        self.model = model

    def enable_ground_contact(self, ground_height: float, stiffness: float, damping: float, friction: float,
                              geometry: Optional[np.ndarray] = None) -> int:
        geom = pack_geometries(self.model)[0] if geometry is None else geometry
        geom = np.ascontiguousarray(geom, dtype=np.float64)
        n = C.c_uint32(0)
        self._check(self._L.phz_enable_ground_contact(self._h, float(ground_height), float(stiffness), float(damping),
                                                      float(friction), _dp(geom), C.byref(n)))
        return int(n.value)

    def enable_ground_contact_per_body(self, ground_height: float, friction: float, gains: Sequence,
                                       geometry: Optional[np.ndarray] = None) -> int:
        if len(gains) != self.nb:
            raise PhzError(f"body_gains has {len(gains)} entries but the model has {self.nb} bodies")
        geom = pack_geometries(self.model)[0] if geometry is None else geometry
        geom = np.ascontiguousarray(geom, dtype=np.float64)
        kd = np.ascontiguousarray(np.asarray(gains, dtype=np.float64).reshape(self.nb, 2))
        n = C.c_uint32(0)
        self._check(self._L.phz_enable_ground_contact_per_body(self._h, float(ground_height), float(friction), _dp(kd),
                                                               _dp(geom), C.byref(n)))
        return int(n.value)

    def _contact_args(self, gains, plane, heightfield, geometry):
        if len(gains) != self.nb:
            raise PhzError(f"body_gains has {len(gains)} entries but the model has {self.nb} bodies")
        geom = pack_geometries(self.model)[0] if geometry is None else geometry
        geom = np.ascontiguousarray(geom, dtype=np.float64)
        kd = np.ascontiguousarray(np.asarray(gains, dtype=np.float64).reshape(self.nb, 2))
        pl = None if plane is None else np.ascontiguousarray(plane.row())
        ex = (C.c_uint32 * max(len(plane.exclude) if plane else 0, 1))(*(plane.exclude if plane else ()))
        nex = len(plane.exclude) if plane else 0
        hdr = None if heightfield is None else np.ascontiguousarray(heightfield.header())
        nodes = None if heightfield is None else heightfield.nodes()
        self._keep = (geom, kd, pl, ex, hdr, nodes)
        return geom, kd, pl, ex, nex, hdr, nodes

    def enable_ground_contact_with_plane(self, ground_height: float, friction: float, gains: Sequence,
                                         plane=None, geometry: Optional[np.ndarray] = None) -> int:
        return self.enable_contact_terrain(ground_height, friction, gains, plane, None, geometry)

    def enable_contact_terrain(self, ground_height: float, friction: float, gains: Sequence, plane=None,
                               heightfield=None, geometry: Optional[np.ndarray] = None) -> int:
        geom, kd, pl, ex, nex, hdr, nodes = self._contact_args(gains, plane, heightfield, geometry)
        n = C.c_uint32(0)
        self._check(self._L.phz_enable_contact_terrain(self._h, float(ground_height), float(friction), _dp(kd), _dp(geom),
                                                       _dp(pl), ex, nex, _dp(hdr), _dp(nodes), C.byref(n)))
        return int(n.value)

    def enable_contact_impulse(self, ground_height: float, friction: float, gains: Sequence, plane=None,
                               heightfield=None, solver: Optional[Sequence[float]] = None,
                               geometry: Optional[np.ndarray] = None) -> int:
        geom, kd, pl, ex, nex, hdr, nodes = self._contact_args(gains, plane, heightfield, geometry)
        sp = None if solver is None else np.ascontiguousarray(np.asarray(solver, dtype=np.float64))
        n = C.c_uint32(0)
        self._check(self._L.phz_enable_contact_impulse(self._h, float(ground_height), float(friction), _dp(kd), _dp(geom),
                                                       _dp(pl), ex, nex, _dp(hdr), _dp(nodes), _dp(sp), C.byref(n)))
        return int(n.value)

    def set_heightfield(self, heightfield):
        hdr = np.ascontiguousarray(heightfield.header())
        nodes = heightfield.nodes()
        self._check(self._L.phz_set_heightfield(self._h, _dp(hdr), _dp(nodes)))

    @property
    def contact_sweeps(self) -> int:
        return int(self._L.phz_contact_sweeps(self._h))

    @contact_sweeps.setter
    def contact_sweeps(self, n: int):
        self._check(self._L.phz_set_contact_sweeps(self._h, int(n)))

    def readback_contact_state(self):
        """(cs [nworld][nb][56], ext [nworld][nb][6]): readback rows, warm-start impulses, carried forces."""
        cs = np.zeros((self.nworld, self.nb, 56))
        ext = np.zeros((self.nworld, self.nb, 6))
        self._check(self._L.phz_readback_contact_state(self._h, _dp(cs), _dp(ext)))
        return cs, ext

    def load_contact_state(self, cs, ext=None):
        c = np.ascontiguousarray(np.asarray(cs, dtype=np.float64).reshape(self.nworld, self.nb, 56))
        e = None if ext is None else np.ascontiguousarray(np.asarray(ext, dtype=np.float64).reshape(self.nworld, self.nb, 6))
        self._check(self._L.phz_load_contact_state(self._h, _dp(c), _dp(e)))

    def enable_pd_control(self, dofs: Sequence[PdDof]):
        t = np.ascontiguousarray(pack_pd_dofs(dofs)) if len(dofs) else np.zeros((0, 8))
        self._check(self._L.phz_enable_pd_control(self._h, _dp(t) if len(dofs) else None, len(dofs)))
        self._npd = len(dofs)

    def set_position_targets(self, targets):
        if self._npd == 0:
            self._check(self._L.phz_set_position_targets(self._h, None))
        self._check(self._L.phz_set_position_targets(self._h, _dp(_rows(targets, self.nworld, self._npd, "targets"))))

    def enable_control_noise(self, seed: int, dist: int, a: float, b: float, dofs: Sequence[int]):
        arr = (C.c_uint32 * max(len(dofs), 1))(*dofs)
        self._check(self._L.phz_enable_control_noise(self._h, int(seed), int(dist), float(a), float(b), arr, len(dofs)))

    # ── state I/O ──
    def load_states(self, q, v, ctrl=None):
        qq = _rows(q, self.nworld, self.nq, "q")
        vv = _rows(v, self.nworld, self.nv, "v")
        cc = None if ctrl is None else _rows(ctrl, self.nworld, self.nctrl, "ctrl")
        self._check(self._L.phz_load_states(self._h, _dp(qq), _dp(vv), _dp(cc)))

    def set_controls(self, ctrl):
        self._check(self._L.phz_set_controls(self._h, _dp(_rows(ctrl, self.nworld, self.nctrl, "ctrl"))))

    def readback_states(self):
        q = np.zeros((self.nworld, self.nq))
        v = np.zeros((self.nworld, self.nv))
        self._check(self._L.phz_readback_states(self._h, _dp(q), _dp(v)))
        return q, v

    def readback_states_noalloc(self):
        """readback_states through the library's static per-GPU scratch (no
        device allocation); worlds x max(nq, nv) x 8 bytes at most 32 MiB."""
        q = np.zeros((self.nworld, self.nq))
        v = np.zeros((self.nworld, self.nv))
        self._check(self._L.phz_readback_states_noalloc(self._h, _dp(q), _dp(v)))
        return q, v

    def readback_contacts(self) -> np.ndarray:
        rows = np.zeros((self.nworld, self.nb, 8))
        self._check(self._L.phz_readback_contacts(self._h, _dp(rows)))
        return rows

    def readback_controls(self) -> np.ndarray:
        c = np.zeros((self.nworld, self.nctrl))
        self._check(self._L.phz_readback_controls(self._h, _dp(c)))
        return c

    def readback_qdd(self) -> np.ndarray:
        a = np.zeros((self.nworld, self.nv))
        self._check(self._L.phz_readback_qdd(self._h, _dp(a)))
        return a

    def readback_rng(self) -> np.ndarray:
        r = np.zeros(self.nworld, dtype=np.uint64)
        self._check(self._L.phz_readback_rng(self._h, r.ctypes.data_as(_lib.u64p)))
        return r

    def load_rng(self, states):
        r = np.ascontiguousarray(np.asarray(states, dtype=np.uint64))
        self._check(self._L.phz_load_rng(self._h, r.ctypes.data_as(_lib.u64p)))

    # ── stepping ──
    def step(self):
        self._check(self._L.phz_step(self._h))

    def try_step(self):
        self.step()

    def step_many(self, n: int):
        self._check(self._L.phz_step_many(self._h, int(n)))

    def synchronize(self):
        self._check(self._L.phz_synchronize(self._h))

    def set_graphs_enabled(self, on: bool):
        self._check(self._L.phz_set_graphs_enabled(self._h, 1 if on else 0))

    @property
    def graphs_enabled(self) -> bool:
        return bool(self._L.phz_graphs_enabled(self._h))

    @property
    def collidable_bodies(self) -> int:
        return int(self._L.phz_collidable_bodies(self._h))

    # ── build / measurement ──
    def compile(self):
        self._check(self._L.phz_compile(self._h))

    def kernel_info(self) -> dict:
        info = (C.c_int64 * 6)()
        self._check(self._L.phz_kernel_info(self._h, info))
        keys = ("vgpr", "agpr", "sgpr", "scratch_bytes", "block", "max_steps_per_launch")
        out = dict(zip(keys, [int(x) for x in info]))
        out["lanes_per_world"] = int(self._L.phz_lanes_per_world(self._h))
        return out

    def time_step_many(self, n: int, reps: int) -> np.ndarray:
        ms = np.zeros(reps)
        self._check(self._L.phz_time_step_many(self._h, int(n), int(reps), _dp(ms)))
        return ms

    # ── device-resident control loop (mod.rs:1004-1376) ──
    def enable_kinematics(self):
        self._check(self._L.phz_enable_kinematics(self._h))

    def compute_kinematics(self):
        self._check(self._L.phz_compute_kinematics(self._h))

    def readback_kinematics(self) -> np.ndarray:
        """[nworld][nb][18]: rotation world->body (row-major), origin, omega, v (body frame)."""
        rows = np.zeros((self.nworld, self.nb, XF_STRIDE))
        self._check(self._L.phz_readback_kinematics(self._h, _dp(rows)))
        return rows

    def enable_policy(self, spec: PolicySpec):
        spec.check_lengths()
        table, aux = pack_obs_ops(spec.obs)
        table = np.ascontiguousarray(table)
        aux = np.ascontiguousarray(aux)
        noise = np.ascontiguousarray(np.asarray(spec.input_noise, dtype=np.float64))
        slots = (C.c_uint32 * max(spec.n_out(), 1))(*[int(s) for s in spec.act_slots])
        cs = None if spec.act_clamp_slots is None else np.ascontiguousarray(np.asarray(spec.act_clamp_slots, dtype=np.float64))
        self._check(self._L.phz_enable_policy(self._h, _dp(table) if len(table) else None, spec.n_in(),
                                              _dp(aux) if len(aux) else None, len(aux), int(spec.hidden), slots,
                                              spec.n_out(), float(spec.act_clamp), _dp(cs), float(spec.noise_rho),
                                              _dp(noise) if len(noise) else None, int(spec.history_steps)))
        self._policy = spec

    def set_policy_weights(self, weights):
        w = np.ascontiguousarray(np.asarray(weights, dtype=np.float64).ravel())
        self._check(self._L.phz_set_policy_weights(self._h, _dp(w), w.size))

    def set_policy_std(self, std):
        s = np.ascontiguousarray(np.asarray(std, dtype=np.float64).ravel())
        self._check(self._L.phz_set_policy_std(self._h, _dp(s), s.size))

    def set_policy_base_targets(self, rows):
        self._check(self._L.phz_set_policy_base_targets(self._h, _dp(_rows(rows, self.nworld, self._npd, "base targets"))))

    def seed_policy(self, seed: int):
        self._check(self._L.phz_seed_policy(self._h, int(seed)))

    def run_policy(self, step: int):
        self._check(self._L.phz_run_policy(self._h, int(step)))

    def readback_policy_history(self, start: int, end: int):
        """(obs [n][nworld][n_in], out [n][nworld][n_out + 1]) for control steps [start, end)."""
        spec = self._policy_spec()
        n = max(int(end) - int(start), 0)
        obs = np.zeros((n, self.nworld, spec.n_in()))
        out = np.zeros((n, self.nworld, spec.n_out() + 1))
        self._check(self._L.phz_readback_policy_history(self._h, int(start), int(end), _dp(obs), _dp(out)))
        return obs, out

    def readback_targets(self) -> np.ndarray:
        rows = np.zeros((self.nworld, max(self._npd, 1)))
        self._check(self._L.phz_readback_targets(self._h, _dp(rows)))
        return rows[:, :self._npd]

    def enable_state_history(self, slots: int):
        self._check(self._L.phz_enable_state_history(self._h, int(slots)))

    def record_state(self, slot: int):
        self._check(self._L.phz_record_state(self._h, int(slot)))

    def readback_state_history(self, start: int, end: int):
        """(q [n][nworld][nq], v [n][nworld][nv]) for history slots [start, end)."""
        n = max(int(end) - int(start), 0)
        q = np.zeros((n, self.nworld, self.nq))
        v = np.zeros((n, self.nworld, self.nv))
        self._check(self._L.phz_readback_state_history(self._h, int(start), int(end), _dp(q), _dp(v)))
        return q, v

    def rollout(self, first_step: int, n_control: int, control_every: int, record_states: bool = False):
        self._check(self._L.phz_rollout(self._h, int(first_step), int(n_control), int(control_every),
                                        1 if record_states else 0))

    def time_rollout(self, first_step: int, n_control: int, control_every: int, record_states: bool,
                     reps: int) -> np.ndarray:
        ms = np.zeros(reps)
        self._check(self._L.phz_time_rollout(self._h, int(first_step), int(n_control), int(control_every),
                                             1 if record_states else 0, int(reps), _dp(ms)))
        return ms

    def time_control_kernel(self, which: str, step: int, reps: int) -> np.ndarray:
        ms = np.zeros(reps)
        self._check(self._L.phz_time_control_kernel(self._h, {"obs": 0, "policy": 1}[which], int(step), int(reps), _dp(ms)))
        return ms

    def control_kernel_info(self, which: str) -> dict:
        info = (C.c_int64 * 6)()
        self._check(self._L.phz_control_kernel_info(self._h, {"obs": 0, "policy": 1}[which], info))
        keys = ("vgpr", "agpr", "sgpr", "scratch_bytes", "block", "worlds_per_block")
        return dict(zip(keys, [int(x) for x in info]))

    def _policy_spec(self) -> PolicySpec:
        spec = getattr(self, "_policy", None)
        if spec is None:
            raise PhzError("policy pass not enabled")
        return spec


def from_workload(w, precision: str, nworld: Optional[int] = None, device: int = 0) -> BatchSim:
    """A BatchSim configured for a phyz_amd.workloads.Workload (contact, PD, control noise)."""
    n = w.nworld if nworld is None else nworld
    sim = BatchSim(w.model, n, precision, device)
    if w.contact is not None and w.impulse_sweeps > 0:
        sim.enable_contact_impulse(w.contact.ground_height, w.contact.friction, w.contact_gains(), None, w.heightfield)
        sim.contact_sweeps = w.impulse_sweeps
    elif w.contact is not None and (w.heightfield is not None or w.gains_omega > 0.0):
        sim.enable_contact_terrain(w.contact.ground_height, w.contact.friction, w.contact_gains(), None, w.heightfield)
    elif w.contact is not None:
        sim.enable_ground_contact(w.contact.ground_height, w.contact.stiffness, w.contact.damping, w.contact.friction)
    if w.pd is not None:
        sim.enable_pd_control(w.pd)
    if w.noise is not None:
        sim.enable_control_noise(w.noise.seed, w.noise.dist, w.noise.a, w.noise.b, w.noise.dofs)
    return sim


def from_control_loop(cl, precision: str = "f32", nworld: Optional[int] = None, device: int = 0) -> BatchSim:
    """A BatchSim running a phyz_amd.workloads.ControlLoop: contact, PD servos, the
    policy with its weights, std, base targets and seed, and a state history of
    one slot per control step."""
    n = cl.nworld if nworld is None else nworld
    w = cl.base
    sim = BatchSim(w.model, n, precision, device)
    sim.enable_ground_contact(w.contact.ground_height, w.contact.stiffness, w.contact.damping, w.contact.friction)
    sim.enable_pd_control(cl.pd)
    sim.enable_policy(cl.spec)
    if device >= 0:
        sim.set_policy_weights(cl.weights)
        sim.set_policy_std(cl.std)
        sim.set_policy_base_targets(cl.base_targets(n))
        sim.seed_policy(cl.seed)
    sim.enable_state_history(cl.spec.history_steps)
    return sim

"""CPU restatement of the device-resident control loop — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, and only as the checker. It follows crates/phyz-gpu/src/policy_pipeline.rs:

  kinematics_rows    fk_thread's XF_STRIDE row (phyz_kernels.cu:1423-1456;
                     policy_pipeline.rs:21-29) from the C++ oracle's FK
                     (oracle/phz_oracle.hpp forward_kinematics, kinematics.rs:10-50)
  observe_reference  ObsOp::eval (policy_pipeline.rs:189-249), centre_of_mass (259-273)
  KernelRng          world_seed + xorshift64 + Box–Muller (policy_pipeline.rs:417-456)
  mlp_forward        policy_pipeline.rs:460-481
  policy_reference   policy_pipeline.rs:484-516
  *_batch, BatchRng  the same functions over a leading world axis (numpy arrays,
                     uint64 RNG states), for the control-loop CPU baseline

Everything is f64 (numpy for the MLP, Python integers for the RNG).

How each function is pinned (tests/test_policy_oracle.py):
  kinematics_rows    frame conventions (frame_conventions.rs:17-79) through the
                     FK oracle, and the transpose relation to the oracle's
                     body->world rotation on a known rotation
  observe_reference  closed forms: pitch/roll/yaw of a free body set to a known
                     rotation, yaw-error wrapping, a hand-computed COM, the
                     heading-frame invariance under a pure yaw
                     (cuda_vs_cpu.rs:1455-1651), empty support = 0
  KernelRng          SplitMix64/xorshift64 against an independent 64-bit
                     implementation; Box–Muller against the closed form of its
                     two uniforms; moments
  mlp_forward        known answers with one-hot inputs (a transposed or
                     misplaced weight block changes them), and torch's
                     Linear/Tanh stack on the same weights
  policy_reference   log-prob against scipy.stats.norm.logpdf; AR(1) update
                     and clamps against their definitions on constructed cases
  *_batch, BatchRng  the per-world functions above, world by world, over three
                     control steps with physics between them and every op kind
                     (RNG states bit for bit, the rest to 1e-12)
"""
from __future__ import annotations

import math
from typing import List, Sequence, Tuple

import numpy as np

MASK64 = (1 << 64) - 1
XF_STRIDE = 18


def world_seed(seed: int, world: int) -> int:
    """SplitMix64 of (seed, world), zero mapped to 1 (policy_pipeline.rs:417-424)."""
    z = (seed + 0x9E3779B97F4A7C15 * (world + 1)) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    z = z ^ (z >> 31)
    return max(z, 1)


class KernelRng:
    """KernelRng (policy_pipeline.rs:430-456)."""

    def __init__(self, state: int):
        self.state = state & MASK64

    @classmethod
    def for_world(cls, seed: int, world: int) -> "KernelRng":
        return cls(world_seed(seed, world))

    def next_u64(self) -> int:
        x = self.state
        x ^= (x << 13) & MASK64
        x ^= x >> 7
        x ^= (x << 17) & MASK64
        self.state = x
        return x

    def uniform(self) -> float:
        return float(self.next_u64() >> 11) / float(1 << 53)

    def normal(self) -> float:
        u1 = self.uniform()
        u2 = self.uniform()
        return math.sqrt(-2.0 * math.log(max(u1, 1e-300))) * math.cos(2.0 * math.pi * u2)


def mlp_forward(n_in: int, n_h: int, n_out: int, weights: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Two tanh hidden layers, linear output; W row-major [out][in] (policy_pipeline.rs:460-481)."""
    w = np.asarray(weights, dtype=np.float64)
    o = 0
    W1 = w[o:o + n_h * n_in].reshape(n_h, n_in); o += n_h * n_in
    b1 = w[o:o + n_h]; o += n_h
    W2 = w[o:o + n_h * n_h].reshape(n_h, n_h); o += n_h * n_h
    b2 = w[o:o + n_h]; o += n_h
    W3 = w[o:o + n_out * n_h].reshape(n_out, n_h); o += n_out * n_h
    b3 = w[o:o + n_out]
    h1 = np.tanh(b1 + W1 @ np.asarray(x, dtype=np.float64))
    h2 = np.tanh(b2 + W2 @ h1)
    return b3 + W3 @ h2


def policy_reference(spec, weights, std, rng: KernelRng, obs: np.ndarray, z: np.ndarray, base_targets: np.ndarray,
                     targets: np.ndarray) -> Tuple[np.ndarray, float]:
    """One world's policy step (policy_pipeline.rs:484-516): input noise in place,
    forward, AR(1) Gaussian sample, log-prob, clamped actions onto the base targets.
    `obs`, `z` and `targets` are updated in place."""
    for i in range(len(obs)):
        if spec.input_noise[i] != 0.0:
            obs[i] += spec.input_noise[i] * rng.normal()
    targets[:] = base_targets
    mean = mlp_forward(spec.n_in(), spec.hidden, spec.n_out(), weights, obs)
    rho = spec.noise_rho
    keep = math.sqrt(max(1.0 - rho * rho, 0.0))
    logp = 0.0
    act = np.zeros(spec.n_out())
    for k in range(spec.n_out()):
        z[k] = rho * z[k] + keep * rng.normal()
        a = mean[k] + std[k] * z[k]
        zi = (a - mean[k]) / std[k]
        logp += -0.5 * zi * zi - math.log(std[k]) - 0.5 * math.log(2.0 * math.pi)
        lim = spec.clamp_at(k)
        slot = spec.act_slots[k]
        targets[slot] = base_targets[slot] + min(max(a, -lim), lim)
        act[k] = a
    return act, logp


def kinematics_rows(orc, q, v) -> np.ndarray:
    """[nb][18] readout rows: rotation world->body (row-major), origin, omega, v (body frame)."""
    fk = orc.fk(q, v)
    rows = np.zeros_like(fk)
    rows[:, 0:9] = fk[:, 0:9].reshape(-1, 3, 3).transpose(0, 2, 1).reshape(-1, 9)
    rows[:, 9:18] = fk[:, 9:18]
    return rows


def centre_of_mass(model, rows: np.ndarray) -> np.ndarray:
    """Mass-weighted COM over bodies with positive mass (policy_pipeline.rs:259-273)."""
    num = np.zeros(3)
    den = 0.0
    for i, b in enumerate(model.bodies):
        m = b.inertia.mass
        if m <= 0.0:
            continue
        r = rows[i, 0:9].reshape(3, 3)  # world -> body
        num += (rows[i, 9:12] + r.T @ np.asarray(b.inertia.com, dtype=np.float64)) * m
        den += m
    return num / den if den > 0.0 else np.zeros(3)


def _wrap(e: float) -> float:
    while e > math.pi:
        e -= 2.0 * math.pi
    while e < -math.pi:
        e += 2.0 * math.pi
    return e


def eval_op(model, rows: np.ndarray, q, v, op) -> float:
    """ObsOp::eval (policy_pipeline.rs:189-249) on FK readout rows."""
    k = op.kind
    if k == 0:
        return float(op.c)
    if k == 1:
        return float(q[op.i] - op.c)
    if k == 2:
        return float(v[op.i])
    if k in (3, 4, 5, 6, 7):
        r = rows[op.body, 0:9].reshape(3, 3)
        if k == 3:
            return math.atan2(-r[0, 2], r[2, 2])
        if k == 4:
            return math.atan2(r[1, 2], r[2, 2])
        if k == 5:
            return _wrap(op.cmd - math.atan2(r[0, 1], r[0, 0]))
        if k == 6:
            return float(rows[op.body, 11])
        return float(rows[op.body, 9 + min(op.axis, 2)])
    if k == 8:
        if len(op.support) == 0:
            return 0.0
        tgt = np.zeros(3)
        for b, o in op.support:
            r = rows[b, 0:9].reshape(3, 3)
            tgt += rows[b, 9:12] + r.T @ np.asarray(o, dtype=np.float64)
        e = centre_of_mass(model, rows) - tgt / len(op.support)
        if op.heading_body is None:
            return float(e[op.axis])
        r = rows[op.heading_body, 0:9].reshape(3, 3)
        yaw = math.atan2(r[0, 1], r[0, 0])
        sy, cy = math.sin(yaw), math.cos(yaw)
        if op.axis == 0:
            return cy * e[0] + sy * e[1]
        if op.axis == 1:
            return -sy * e[0] + cy * e[1]
        return float(e[2])
    raise ValueError(f"unknown op kind {k}")


def observe_reference(model, orc, q, v, ops: Sequence) -> List[float]:
    """observe_reference (policy_pipeline.rs:519-523): FK, then the ops."""
    rows = kinematics_rows(orc, q, v)
    return [eval_op(model, rows, q, v, op) for op in ops]


# ── World-batched forms: the same arithmetic over many worlds at once (numpy
# arrays with a leading world axis), for the control-loop CPU baseline. Each
# follows its per-world function above draw for draw and op for op; the matrix
# products and numpy's log/cos may round differently from the per-world
# matrix-vector products and the C library's functions.

class BatchRng:
    """KernelRng with one xorshift64 state per world (policy_pipeline.rs:430-456)."""

    def __init__(self, states):
        self.state = np.array(states, dtype=np.uint64)

    @classmethod
    def for_worlds(cls, seed: int, worlds: Sequence[int]) -> "BatchRng":
        return cls([world_seed(seed, int(w)) for w in worlds])

    def next_u64(self) -> np.ndarray:
        x = self.state
        x ^= x << np.uint64(13)
        x ^= x >> np.uint64(7)
        x ^= x << np.uint64(17)
        return x.copy()

    def uniform(self) -> np.ndarray:
        return (self.next_u64() >> np.uint64(11)).astype(np.float64) / float(1 << 53)

    def normal(self) -> np.ndarray:
        u1 = self.uniform()
        u2 = self.uniform()
        return np.sqrt(-2.0 * np.log(np.maximum(u1, 1e-300))) * np.cos(2.0 * math.pi * u2)


def mlp_forward_batch(n_in: int, n_h: int, n_out: int, weights: np.ndarray, x: np.ndarray) -> np.ndarray:
    """mlp_forward on rows x [nworld][n_in] -> [nworld][n_out]."""
    w = np.asarray(weights, dtype=np.float64)
    o = 0
    W1 = w[o:o + n_h * n_in].reshape(n_h, n_in); o += n_h * n_in
    b1 = w[o:o + n_h]; o += n_h
    W2 = w[o:o + n_h * n_h].reshape(n_h, n_h); o += n_h * n_h
    b2 = w[o:o + n_h]; o += n_h
    W3 = w[o:o + n_out * n_h].reshape(n_out, n_h); o += n_out * n_h
    b3 = w[o:o + n_out]
    h1 = np.tanh(b1 + np.asarray(x, dtype=np.float64) @ W1.T)
    h2 = np.tanh(b2 + h1 @ W2.T)
    return b3 + h2 @ W3.T


def policy_batch(spec, weights, std, rng: BatchRng, obs: np.ndarray, z: np.ndarray, base_targets: np.ndarray,
                 targets: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """policy_reference for every world: obs [nworld][n_in], z [nworld][n_out]
    and targets [nworld][n_pd] updated in place; returns (actions, log-probs)."""
    nw = obs.shape[0]
    for i in range(obs.shape[1]):
        if spec.input_noise[i] != 0.0:
            obs[:, i] += spec.input_noise[i] * rng.normal()
    targets[:] = base_targets
    mean = mlp_forward_batch(spec.n_in(), spec.hidden, spec.n_out(), weights, obs)
    rho = spec.noise_rho
    keep = math.sqrt(max(1.0 - rho * rho, 0.0))
    logp = np.zeros(nw)
    act = np.zeros((nw, spec.n_out()))
    for k in range(spec.n_out()):
        z[:, k] = rho * z[:, k] + keep * rng.normal()
        a = mean[:, k] + std[k] * z[:, k]
        zi = (a - mean[:, k]) / std[k]
        logp += -0.5 * zi * zi - math.log(std[k]) - 0.5 * math.log(2.0 * math.pi)
        lim = spec.clamp_at(k)
        slot = spec.act_slots[k]
        targets[:, slot] = base_targets[:, slot] + np.minimum(np.maximum(a, -lim), lim)
        act[:, k] = a
    return act, logp


def kinematics_rows_batch(orc, q, v, threads: int = 1) -> np.ndarray:
    """kinematics_rows for world-major states: [nworld][nb][18]."""
    fk = orc.fk_batch(q, v, threads)
    nw, nb = fk.shape[0], fk.shape[1]
    rows = fk.copy()
    rows[:, :, 0:9] = fk[:, :, 0:9].reshape(nw, nb, 3, 3).transpose(0, 1, 3, 2).reshape(nw, nb, 9)
    return rows


def _body_point_batch(rows: np.ndarray, b: int, p) -> np.ndarray:
    """World position of body-frame point p on body b, every world: origin + R_wb p."""
    r = rows[:, b, 0:9].reshape(-1, 3, 3)  # world -> body; its transpose maps body -> world
    return rows[:, b, 9:12] + np.einsum("wji,j->wi", r, np.asarray(p, dtype=np.float64))


def centre_of_mass_batch(model, rows: np.ndarray) -> np.ndarray:
    num = np.zeros((rows.shape[0], 3))
    den = 0.0
    for i, b in enumerate(model.bodies):
        m = b.inertia.mass
        if m <= 0.0:
            continue
        num += _body_point_batch(rows, i, b.inertia.com) * m
        den += m
    return num / den if den > 0.0 else np.zeros((rows.shape[0], 3))


def _wrap_batch(e: np.ndarray) -> np.ndarray:
    while (e > math.pi).any():
        e = np.where(e > math.pi, e - 2.0 * math.pi, e)
    while (e < -math.pi).any():
        e = np.where(e < -math.pi, e + 2.0 * math.pi, e)
    return e


def eval_op_batch(model, rows: np.ndarray, q, v, op) -> np.ndarray:
    """eval_op for every world: rows [nworld][nb][18], q/v world-major."""
    k = op.kind
    nw = rows.shape[0]
    if k == 0:
        return np.full(nw, float(op.c))
    if k == 1:
        return q[:, op.i] - op.c
    if k == 2:
        return np.array(v[:, op.i], dtype=np.float64)
    if k in (3, 4, 5, 6, 7):
        r = rows[:, op.body, 0:9]  # row-major world -> body
        if k == 3:
            return np.arctan2(-r[:, 2], r[:, 8])
        if k == 4:
            return np.arctan2(r[:, 5], r[:, 8])
        if k == 5:
            return _wrap_batch(op.cmd - np.arctan2(r[:, 1], r[:, 0]))
        if k == 6:
            return rows[:, op.body, 11].copy()
        return rows[:, op.body, 9 + min(op.axis, 2)].copy()
    if k == 8:
        if len(op.support) == 0:
            return np.zeros(nw)
        tgt = np.zeros((nw, 3))
        for b, o in op.support:
            tgt += _body_point_batch(rows, b, o)
        e = centre_of_mass_batch(model, rows) - tgt / len(op.support)
        if op.heading_body is None:
            return e[:, op.axis].copy()
        r = rows[:, op.heading_body, 0:9]
        yaw = np.arctan2(r[:, 1], r[:, 0])
        sy, cy = np.sin(yaw), np.cos(yaw)
        if op.axis == 0:
            return cy * e[:, 0] + sy * e[:, 1]
        if op.axis == 1:
            return -sy * e[:, 0] + cy * e[:, 1]
        return e[:, 2].copy()
    raise ValueError(f"unknown op kind {k}")


def observe_batch(model, orc, q, v, ops: Sequence, threads: int = 1) -> np.ndarray:
    """observe_reference for world-major states: [nworld][len(ops)]."""
    rows = kinematics_rows_batch(orc, q, v, threads)
    q = np.asarray(q, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    return np.stack([eval_op_batch(model, rows, q, v, op) for op in ops], axis=1)

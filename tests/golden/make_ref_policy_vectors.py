"""Write tests/golden/ref_policy_vectors.npz: input/output vectors of the
reference's own control-loop kernels (phyz_host_fk, phyz_host_obs and
phyz_host_policy of crates/phyz-gpu/cuda/phyz_kernels.cu:1809-1835, compiled
as host C++ by oracle/Makefile into oracle/_ref).

Run in a tree where /root/reference is present (after `make -C oracle`):
    python tests/golden/make_ref_policy_vectors.py

The case is the control-loop ant (phyz_amd.workloads.control_loop: its 29
observation ops, input noise on every feature, AR(1) action noise rho 0.5, 8
clamped action slots) with a 32-wide MLP, on 32 worlds with seeded states
(tilted, yawed torsos, moving joints so the pitch, roll, yaw and COM features
are all non-trivial). Stored: the f32 inputs (q, v, weights, std, base
targets, the per-world xorshift64 seeds) and, per policy pass over three
passes, the reference's FK rows, clean and noisy observation rows, actions
and log-probs, PD targets, AR(1) state and RNG words.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.policy_ref import world_seed  # noqa: E402
from phyz_amd import workloads as W  # noqa: E402
from phyz_amd.model import pack_bodies  # noqa: E402
from tests.ref_host import RefControl, available  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_policy_vectors.npz")
NWORLD = 32
HIDDEN = 32
PASSES = 3
SEED = 0x5EED


def main():
    if not available():
        sys.exit("oracle/_ref/libphyz_ref_host.so missing: run `make -C oracle` with the reference tree present")
    cl = W.control_loop(HIDDEN)
    m = cl.base.model
    rng = np.random.default_rng(17)
    q, v, _, _ = cl.base.initial_state(NWORLD)
    q[:, 0:3] = rng.normal(size=(NWORLD, 3)) * 0.4          # torso rotation vector: pitch, roll and yaw
    q[:, 3:5] = rng.normal(size=(NWORLD, 2)) * 0.3
    q[:, 6:] = rng.uniform(-0.6, 0.6, size=(NWORLD, m.nq - 6))
    v[:] = rng.normal(size=(NWORLD, m.nv)) * 0.7
    q32 = np.ascontiguousarray(q, dtype=np.float32)
    v32 = np.ascontiguousarray(v, dtype=np.float32)
    n_dofs = len(cl.pd)
    base = np.ascontiguousarray(cl.base_targets(NWORLD), dtype=np.float32)
    rc = RefControl(pack_bodies(m), m, cl.spec, cl.weights, cl.std, n_dofs, NWORLD)
    seeds = [world_seed(SEED, w) for w in range(NWORLD)]
    # The state words go in as raw bits (a view, never a float conversion,
    # which would quiet the NaN patterns among them).
    words = np.ascontiguousarray(np.array([[s & 0xFFFFFFFF, s >> 32] for s in seeds],
                                          dtype=np.uint32).reshape(-1).view(np.float32))
    z = np.zeros(NWORLD * cl.spec.n_out(), dtype=np.float32)
    xf = rc.fk(q32, v32)
    out = {"q": q32, "v": v32, "weights": rc.weights, "std": rc.std, "base_targets": base,
           "seeds": np.array(seeds, dtype=np.uint64), "dims": np.array([NWORLD, HIDDEN, PASSES, n_dofs]),
           "xforms": xf.reshape(NWORLD, m.nbodies, 18)}
    for k in range(PASSES):
        clean = rc.obs(q32, v32, xf)
        obs = clean.copy()
        tg, res = rc.policy(obs, words, z, base)
        out[f"pass{k}/obs_clean"] = clean.reshape(NWORLD, -1)
        out[f"pass{k}/obs_noisy"] = obs.reshape(NWORLD, -1)
        out[f"pass{k}/out"] = res
        out[f"pass{k}/targets"] = tg
        out[f"pass{k}/z"] = z.reshape(NWORLD, -1).copy()
        out[f"pass{k}/rng_words"] = words.view(np.uint32).reshape(NWORLD, 2).copy()
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()

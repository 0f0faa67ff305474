"""Writes tests/golden/ppo_ref_vectors.npz: the reference's own PPO update
kernels (crates/phyz-gpu/cuda/phyz_train.cu, compiled as host C++ into
oracle/_ref by oracle/Makefile) driven through TrainPipeline::update's loop
(oracle/ppo_ref.py RefHostPipeline) on the reference parity test's problem
(crates/phyz-gpu/tests/train_parity.rs:29-98). Data only: inputs, shuffles,
settings, and the weights and statistics the reference kernels produce.

    python tests/golden/make_ppo_vectors.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.ppo_ref import Dims, RefHostPipeline, init_flat, make_batch, policy_logp, ref_available, shuffles  # noqa: E402

N, A_IN, C_IN, H, ACT = 512, 12, 20, 16, 4
AD, CD = Dims(A_IN, H, ACT), Dims(C_IN, H, 1)

# name: (iterations, minibatch, rows, target_kl, kl_mode, old log-probs from the initial policy)
CASES = {
    "one": (1, 64, N, 1e9, 1, False),
    "three": (3, 64, N, 1e9, 1, False),
    "brake_k3": (1, 64, N, 1e-4, 1, True),
    "brake_cumulative": (1, 64, N, 5e-4, 0, True),
    "ragged": (1, 100, N - 37, 1e9, 1, False),
}
CLIP, ENTROPY, VDELTA, EPOCHS = 0.2, 0.003, 6.0, 3


def main():
    if not ref_available():
        raise SystemExit("oracle/_ref not built (make -C oracle ref, with the reference tree present)")
    out = {"dims": np.array([A_IN, H, ACT, C_IN, H, 1]), "cfg": np.array([CLIP, ENTROPY, VDELTA, EPOCHS, ACT])}
    base = make_batch(0xC0FFEE, N, A_IN, C_IN, ACT)
    a0, c0 = init_flat(7, AD, ACT, -0.7), init_flat(9, CD)
    out["actor0"], out["critic0"] = a0, c0
    for k, v in base.items():
        out[f"batch_{k}"] = v.astype(np.float32)
    out["batch_logp_policy"] = (policy_logp(a0, AD, base["obs_a"], base["act"]) + 0.01 * base["adv"]).astype(np.float32)
    for name, (iters, mb, rows, target, mode, from_policy) in CASES.items():
        b32 = {k: out[f"batch_{k}"][:rows] for k in base}
        if from_policy:
            b32["logp_old"] = out["batch_logp_policy"][:rows]
        ref = RefHostPipeline(AD, CD, a0, c0, mb)
        stats = []
        for it in range(iters):
            order = shuffles(0x5EED + it, rows, EPOCHS)
            out[f"{name}_order{it}"] = np.stack(order)
            s = ref.update(b32, order, CLIP, ENTROPY, VDELTA, mb, EPOCHS, target, ACT, mode)
            stats.append([s.policy_loss, s.value_loss, s.kl, s.grad_steps, float(s.stopped_early)])
        out[f"{name}_setup"] = np.array([iters, mb, rows, target, mode, float(from_policy)])
        out[f"{name}_stats"] = np.array(stats)
        out[f"{name}_actor"] = ref.actor_params()
        out[f"{name}_critic"] = ref.critic_params()
        print(name, stats[-1])
    path = os.path.join(ROOT, "tests", "golden", "ppo_ref_vectors.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()

"""The PPO update oracle (oracle/ppo_ref.py), pinned without a GPU.

- Against the reference's own update kernels (crates/phyz-gpu/cuda/phyz_train.cu
  compiled as host C++ into oracle/_ref), driven through TrainPipeline::update's
  loop, on the reference parity test's problem (train_parity.rs:29-98): weight
  deltas and losses after one and three updates at the reference's own
  tolerances (train_parity.rs:421-494), and the KL brake stopping on the same
  minibatch.
- By the mathematics: the minibatch gradient against central differences of
  the clipped-surrogate, entropy and squared-error objectives; Adam's first
  step in closed form; the two brake readings on a hand-computed case.
"""
import math

import numpy as np
import pytest

from oracle.ppo_ref import (Adam, CpuPpo, Dims, RefHostPipeline, init_flat, make_batch, mlp_forward, policy_logp,
                            ref_available, shuffles)

N, A_IN, C_IN, H, ACT, MB = 512, 12, 20, 16, 4, 64
AD, CD = Dims(A_IN, H, ACT), Dims(C_IN, H, 1)
need_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref (reference kernels, host build) not built")


def problem(logp_from_policy=False):
    batch = make_batch(0xC0FFEE, N, A_IN, C_IN, ACT)
    a0, c0 = init_flat(7, AD, ACT, -0.7), init_flat(9, CD)
    if logp_from_policy:
        batch["logp_old"] = policy_logp(a0, AD, batch["obs_a"], batch["act"]) + 0.01 * batch["adv"]
    b32 = {k: v.astype(np.float32) for k, v in batch.items()}
    return {k: v.astype(np.float64) for k, v in b32.items()}, b32, a0, c0


def delta_gap(before, cpu, other):
    """train_parity.rs:400-418: largest disagreement of the weight deltas over the largest delta."""
    scale = max(np.abs(cpu - before).max(), 1e-30)
    return np.abs((cpu - before) - (other - before)).max() / scale


def rel(a, b):
    return abs(a - b) / max(abs(b), 1e-12)


def run_both(iters, target_kl, logp_from_policy=False, kl_mode=1, n_rows=N, minibatch=MB):
    b64, b32, a0, c0 = problem(logp_from_policy)
    if n_rows != N:
        b64 = {k: v[:n_rows] for k, v in b64.items()}
        b32 = {k: v[:n_rows] for k, v in b32.items()}
    cpu = CpuPpo(AD, CD, a0, c0)
    ref = RefHostPipeline(AD, CD, a0, c0, minibatch)
    out = []
    for it in range(iters):
        order = shuffles(0x5EED + it, n_rows, 3)
        sc = cpu.update(b64, order, 0.2, 0.003, 6.0, minibatch, 3, target_kl, ACT, kl_mode)
        sr = ref.update(b32, order, 0.2, 0.003, 6.0, minibatch, 3, target_kl, ACT, kl_mode)
        out.append((sc, sr))
    return out, (a0, c0), (cpu.actor, cpu.critic), (ref.actor_params(), ref.critic_params())


@need_ref
def test_one_update_matches_the_reference_kernels():
    out, (a0, c0), (ca, cc), (ra, rc) = run_both(1, 1e9)
    sc, sr = out[0]
    assert sc.grad_steps == sr.grad_steps == 3 * N // MB
    ga, gc = delta_gap(a0, ca, ra), delta_gap(c0, cc, rc)
    print(f"one update: actor delta gap {ga:.3e}, critic {gc:.3e}")
    # The reference holds its host walk to tang at 2e-4 (train_parity.rs:432-433).
    assert ga < 2e-4 and gc < 2e-4
    assert rel(sr.policy_loss, sc.policy_loss) < 1e-4 and rel(sr.value_loss, sc.value_loss) < 1e-4
    assert rel(sr.kl, sc.kl) < 1e-3


@need_ref
def test_three_updates_track_the_reference_kernels():
    out, (a0, c0), (ca, cc), (ra, rc) = run_both(3, 1e9)
    for sc, sr in out:
        assert rel(sr.policy_loss, sc.policy_loss) < 1e-3 and rel(sr.value_loss, sc.value_loss) < 1e-3
    assert delta_gap(a0, ca, ra) < 1e-3 and delta_gap(c0, cc, rc) < 1e-3


@need_ref
@pytest.mark.parametrize("kl_mode", [0, 1])
def test_kl_brake_stops_on_the_same_minibatch(kl_mode):
    # Old log-probs from the initial policy: the reading starts near zero and grows.
    target = 1e-4 if kl_mode == 1 else 5e-4
    out, _, _, _ = run_both(1, target, logp_from_policy=True, kl_mode=kl_mode)
    sc, sr = out[0]
    assert sr.stopped_early and sc.stopped_early
    assert 1 < sr.grad_steps < 3 * N // MB
    assert sc.grad_steps == sr.grad_steps


@need_ref
def test_ragged_last_minibatch_matches_the_reference_kernels():
    out, (a0, c0), (ca, cc), (ra, rc) = run_both(1, 1e9, n_rows=N - 37, minibatch=100)
    sc, sr = out[0]
    assert sc.grad_steps == sr.grad_steps == 3 * math.ceil((N - 37) / 100)
    assert delta_gap(a0, ca, ra) < 2e-4 and delta_gap(c0, cc, rc) < 2e-4


def objectives(cpu: CpuPpo, batch, chunk, clip, entropy_coef):
    """The minibatch objectives whose gradients the update follows, computed
    directly: mean clipped-surrogate loss minus the entropy bonus on log_std,
    and the mean squared value error."""
    ad = cpu.ad
    off = ad.param_count()
    nb = chunk.size
    _, _, mean = mlp_forward(cpu.actor, ad, batch["obs_a"][chunk])
    log_std = cpu.actor[off:off + ad.n_out]
    z = (batch["act"][chunk] - mean) / np.exp(log_std)
    logp = (-0.5 * z * z - log_std - 0.5 * math.log(2 * math.pi)).sum(axis=1)
    ratio = np.exp(logp - batch["logp_old"][chunk])
    adv = batch["adv"][chunk]
    surr = -np.minimum(ratio * adv, np.clip(ratio, 1 - clip, 1 + clip) * adv).sum() / nb
    la = surr - entropy_coef * log_std.sum()
    _, _, v = mlp_forward(cpu.critic, cpu.cd, batch["obs_c"][chunk])
    lc = ((v[:, 0] - batch["ret"][chunk]) ** 2).sum() / nb
    return la, lc


def test_minibatch_gradient_against_central_differences():
    ad, cd = Dims(5, 7, 3), Dims(6, 7, 1)
    batch = make_batch(3, 40, 5, 6, 3)
    a0 = init_flat(1, ad, 3, -0.4)
    batch["logp_old"] = policy_logp(a0, ad, batch["obs_a"], batch["act"]) + 0.3 * np.sin(np.arange(40))
    cpu = CpuPpo(ad, cd, a0, init_flat(2, cd))
    chunk = np.arange(3, 35)
    clip, ent = 0.2, 0.01
    g = cpu.minibatch_grads(batch, chunk, clip, ent, math.inf)
    # Rows at a clip kink would make the objective non-differentiable there.
    lr = policy_logp(cpu.actor, ad, batch["obs_a"][chunk], batch["act"][chunk]) - batch["logp_old"][chunk]
    assert np.min(np.abs(np.exp(lr) - (1 - clip)).tolist() + np.abs(np.exp(lr) - (1 + clip)).tolist()) > 1e-4
    assert 0 < np.sum(np.abs(lr) > math.log(1 + clip)) < chunk.size  # both branches occur
    h = 1e-6
    for which, flat, key in (("actor", cpu.actor, "g_actor"), ("critic", cpu.critic, "g_critic")):
        num = np.zeros_like(flat)
        for k in range(flat.size):
            old = flat[k]
            flat[k] = old + h
            lp = objectives(cpu, batch, chunk, clip, ent)[0 if which == "actor" else 1]
            flat[k] = old - h
            lm = objectives(cpu, batch, chunk, clip, ent)[0 if which == "actor" else 1]
            flat[k] = old
            num[k] = (lp - lm) / (2 * h)
        err = np.abs(num - g[key]).max() / np.abs(num).max()
        print(f"{which}: max gradient error {err:.2e} of {np.abs(num).max():.2e}")
        assert err < 1e-6


def test_huber_clip_caps_the_value_gradient():
    ad, cd = Dims(4, 5, 2), Dims(4, 5, 1)
    batch = make_batch(5, 16, 4, 4, 2)
    batch["ret"] = batch["ret"] * 50.0
    cpu = CpuPpo(ad, cd, init_flat(1, ad, 2), init_flat(2, cd))
    chunk = np.arange(16)
    g_inf = cpu.minibatch_grads(batch, chunk, 0.2, 0.0, math.inf)["g_critic"]
    g_cap = cpu.minibatch_grads(batch, chunk, 0.2, 0.0, 1.0)["g_critic"]
    # The output bias gradient is the mean of 2 * clamp(err): bounded by 2 with the cap.
    assert abs(g_cap[cd.param_count() - 1]) <= 2.0 + 1e-12
    assert abs(g_inf[cd.param_count() - 1]) > 10.0


def test_adam_first_step_closed_form():
    g = np.array([0.5, -2.0, 1e-3, 0.0])
    p = np.ones(4)
    Adam(4, lr=0.01).step(p, g)
    # m_hat = g and v_hat = g^2 after one step: p moves by -lr g / (|g| + eps).
    np.testing.assert_allclose(p, 1.0 - 0.01 * g / (np.abs(g) + 1e-8), rtol=0, atol=1e-15)
    q = np.full(4, 2.0)
    Adam(4, lr=0.01, weight_decay=0.1).step(q, np.zeros(4))
    np.testing.assert_allclose(q, 2.0 * (1 - 0.01 * 0.1), rtol=0, atol=1e-15)


def test_brake_readings_by_hand():
    # One minibatch of two rows whose log-ratios are known: logp_old - logp = (a, b).
    ad, cd = Dims(1, 1, 1), Dims(1, 1, 1)
    actor = np.zeros(ad.param_count() + 1)  # mean 0, log_std 0
    batch = {"obs_a": np.zeros((2, 1)), "obs_c": np.zeros((2, 1)), "act": np.array([[0.0], [1.0]]),
             "adv": np.zeros(2), "ret": np.zeros(2)}
    logp = -0.5 * batch["act"][:, 0] ** 2 - 0.5 * math.log(2 * math.pi)
    d = np.array([0.3, -0.1])
    batch["logp_old"] = logp + d
    for mode, want in ((0, abs(d.mean()) / 2.0), (1, np.mean(np.exp(-d) - 1 + d) / 2.0)):
        cpu = CpuPpo(ad, cd, actor, np.zeros(cd.param_count()))
        s = cpu.update(batch, [np.arange(2)], 0.2, 0.0, 1.0, 2, 1, 1e9, 2.0, mode)
        assert s.kl == pytest.approx(want, rel=1e-12)

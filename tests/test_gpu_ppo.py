"""The PPO update pass on the device (phyz_amd.train over phz_train.hip).

Parity follows the reference's train_parity.rs (crates/phyz-gpu/tests/
train_parity.rs:400-494): the weight delta after one update against the f64
CPU update within 2e-4 of the largest delta, within 1e-3 after three updates,
the policy and value losses within 1e-4 (1e-3 over three updates), the KL
reading within 1e-3, and the brake stopping on the same minibatch. The device
is also held, tighter, to the reference's own kernels on the same inputs
(tests/golden/ppo_ref_vectors.npz, written by tests/golden/make_ppo_vectors.py):
both sides are f32 arithmetic with f64 accumulations and an f64 Adam.
"""
import math
import os

import numpy as np
import pytest

from oracle.ppo_ref import CpuPpo, Dims, init_flat, policy_logp
from phyz_amd.train import (AdamCfg, KlMode, NetDims, PpoUpdateCfg, SampleBatch, TrainError, TrainPipeline)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ppo_ref_vectors.npz")
CASES = ["one", "three", "brake_k3", "brake_cumulative", "ragged"]


def delta_gap(before, want, got):
    scale = max(np.abs(want - before).max(), 1e-30)
    return np.abs((want - before) - (got - before)).max() / scale


def rel(a, b):
    return abs(a - b) / max(abs(b), 1e-12)


def golden():
    return np.load(GOLDEN)


def golden_case(g, name):
    iters, mb, rows, target, mode, from_policy = g[f"{name}_setup"]
    iters, mb, rows, mode = int(iters), int(mb), int(rows), int(mode)
    batch = {k: g[f"batch_{k}"][:rows] for k in ("obs_a", "obs_c", "act", "logp_old", "adv", "ret")}
    if from_policy:
        batch["logp_old"] = g["batch_logp_policy"][:rows]
    clip, ent, vdelta, epochs, kl_scale = g["cfg"]
    cfg = PpoUpdateCfg(clip, ent, vdelta, mb, int(epochs), target, kl_scale, KlMode(mode))
    orders = [g[f"{name}_order{it}"] for it in range(iters)]
    return batch, cfg, orders, rows


def pipeline(g, mb, rows):
    a_in, h, act, c_in, hc, one = (int(x) for x in g["dims"])
    pipe = TrainPipeline(NetDims(a_in, h, act), NetDims(c_in, hc, one), rows, mb)
    pipe.set_adam(AdamCfg(), AdamCfg())
    pipe.set_actor_params(g["actor0"])
    pipe.set_critic_params(g["critic0"])
    return pipe


def upload(pipe, batch, rows):
    pipe.upload_batch(rows, SampleBatch(batch["obs_a"], batch["obs_c"], batch["act"], batch["logp_old"],
                                        batch["adv"], batch["ret"]))


# ── without a device: the constructor's checks come before any device query ──
@pytest.mark.parametrize("actor,critic,msg", [
    ((8, 257, 2), (8, 16, 1), "actor hidden width 257 exceeds TRAIN_MAX_H 256"),
    ((8, 16, 65), (8, 16, 1), "actor output width 65 exceeds TRAIN_MAX_OUT 64"),
    ((8, 16, 2), (8, 300, 1), "critic hidden width 300 exceeds TRAIN_MAX_H 256"),
    ((8, 16, 2), (8, 16, 2), "critic must have one output, got 2"),
])
def test_constructor_rejects_what_the_reference_rejects(actor, critic, msg):
    with pytest.raises(TrainError, match=msg):
        TrainPipeline(NetDims(*actor), NetDims(*critic), 16, 8)


# ── on the device ──
@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_update_matches_the_reference_kernels(name):
    g = golden()
    batch, cfg, orders, rows = golden_case(g, name)
    pipe = pipeline(g, cfg.minibatch, rows)
    upload(pipe, batch, rows)
    stats = [pipe.update(o, cfg) for o in orders]
    want = g[f"{name}_stats"]
    a, c = pipe.actor_params(), pipe.critic_params()
    ga = delta_gap(g["actor0"], g[f"{name}_actor"], a)
    gc = delta_gap(g["critic0"], g[f"{name}_critic"], c)
    print(f"{name}: tile rows {pipe.rows_per_tile}; delta gap vs reference kernels actor {ga:.2e} critic {gc:.2e}; "
          f"stats {stats[-1]}", flush=True)
    for s, w in zip(stats, want):
        assert s.grad_steps == int(w[3]) and s.stopped_early == bool(w[4])
        assert rel(s.policy_loss, w[0]) < 1e-5 and rel(s.value_loss, w[1]) < 1e-5 and rel(s.kl, w[2]) < 1e-4
    tol = 2e-5 if len(orders) == 1 else 1e-4
    assert ga < tol and gc < tol


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["one", "three", "brake_k3"])
def test_update_matches_the_f64_cpu_update(name):
    g = golden()
    batch, cfg, orders, rows = golden_case(g, name)
    pipe = pipeline(g, cfg.minibatch, rows)
    upload(pipe, batch, rows)
    a_in, h, act, c_in, hc, _ = (int(x) for x in g["dims"])
    cpu = CpuPpo(Dims(a_in, h, act), Dims(c_in, hc, 1), g["actor0"], g["critic0"])
    b64 = {k: v.astype(np.float64) for k, v in batch.items()}
    for it, o in enumerate(orders):
        s = pipe.update(o, cfg)
        w = cpu.update(b64, o, cfg.clip, cfg.entropy_coef, cfg.vdelta, cfg.minibatch, cfg.epochs, cfg.target_kl,
                       cfg.kl_scale, int(cfg.kl_mode))
        assert s.grad_steps == w.grad_steps and s.stopped_early == w.stopped_early
        tol = 1e-4 if len(orders) == 1 else 1e-3
        assert rel(s.policy_loss, w.policy_loss) < tol and rel(s.value_loss, w.value_loss) < tol
        assert rel(s.kl, w.kl) < 1e-3
    ga = delta_gap(g["actor0"], cpu.actor, pipe.actor_params())
    gc = delta_gap(g["critic0"], cpu.critic, pipe.critic_params())
    print(f"{name}: delta gap vs f64 CPU update actor {ga:.2e} critic {gc:.2e}", flush=True)
    lim = 2e-4 if len(orders) == 1 else 1e-3
    assert ga < lim and gc < lim


def synthetic(n, ad: Dims, c_in, seed, actor):
    """A batch shaped like the reference's timing batch, with old log-probs
    near the initial policy's so that ratios stay near 1."""
    rng = np.random.default_rng(seed)
    b = {"obs_a": rng.normal(size=(n, ad.n_in)) * 0.5, "obs_c": rng.normal(size=(n, c_in)) * 0.5,
         "act": rng.normal(size=(n, ad.n_out)) * 0.3, "adv": rng.normal(size=n), "ret": rng.normal(size=n) * 2.0}
    b["logp_old"] = policy_logp(actor, ad, b["obs_a"], b["act"]) + 0.05 * rng.normal(size=n)
    return {k: v.astype(np.float32) for k, v in b.items()}


def delta_errors(before, want, got):
    """Per-parameter disagreement of the weight deltas over the largest delta."""
    return np.abs((got - before) - (want - before)) / max(np.abs(want - before).max(), 1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("a_in,c_in,h,act,n,mb", [
    (55, 67, 64, 22, 16384, 4096),   # the reference's timing shape (examples/cuda_train.rs), 4 minibatches
    (55, 67, 64, 22, 10000, 5000),   # 157 tiles per minibatch: Adam's loads past its first 128 tiles
    (40, 40, 256, 8, 1000, 300),     # widest hidden layer, ragged minibatches: weights read from HBM
    (128, 96, 128, 8, 2000, 500),    # too wide to stage every matrix: one layer at a time through LDS
    (2000, 24, 32, 6, 256, 96),      # inputs so wide that a 16-row tile needs more than 64 KiB of LDS
])
def test_shapes_against_the_f64_cpu_update(a_in, c_in, h, act, n, mb):
    """On shapes other than the reference test's, the largest single-parameter
    gap is set by the worst-conditioned gradient (a sum over thousands of rows
    that nearly cancels), and the reference's own kernels exceed 2e-4 on two of
    these three (4e-4 and 3.8e-3). So the check is on the distribution: the
    median, p99 and p99.9 of the per-parameter gaps, where the reference's
    kernels sit at <= 2.2e-7, 2.1e-6 and 6.4e-6 on these shapes (measured on
    their host build, which stays off the GPU box)."""
    ad, cd = Dims(a_in, h, act), Dims(c_in, h, 1)
    a0, c0 = init_flat(11, ad, act, -0.5), init_flat(12, cd)
    batch = synthetic(n, ad, c_in, 3, a0)
    pipe = TrainPipeline(NetDims(a_in, h, act), NetDims(c_in, h, 1), n, mb)
    pipe.set_actor_params(a0)
    pipe.set_critic_params(c0)
    upload(pipe, batch, n)
    order = [np.random.default_rng(5).permutation(n).astype(np.uint32)]
    cfg = PpoUpdateCfg(0.2, 0.003, 6.0, mb, 1, math.inf, act, KlMode.MINIBATCH)
    s = pipe.update(order, cfg)
    cpu = CpuPpo(ad, cd, a0, c0)
    w = cpu.update({k: v.astype(np.float64) for k, v in batch.items()}, order, 0.2, 0.003, 6.0, mb, 1, math.inf,
                   act, 1)
    assert s.grad_steps == w.grad_steps == math.ceil(n / mb)
    assert rel(s.policy_loss, w.policy_loss) < 1e-4 and rel(s.value_loss, w.value_loss) < 1e-4
    for net, x0, xc, xd in (("actor", a0, cpu.actor, pipe.actor_params()),
                            ("critic", c0, cpu.critic, pipe.critic_params())):
        e = delta_errors(x0, xc, xd)
        q = [np.median(e), np.percentile(e, 99), np.percentile(e, 99.9)]
        print(f"{a_in}/{c_in}-{h}-{act} n {n} mb {mb} (tile rows {pipe.rows_per_tile}) {net}: gap median {q[0]:.2e} "
              f"p99 {q[1]:.2e} p99.9 {q[2]:.2e} max {e.max():.2e}", flush=True)
        assert q[0] < 1e-6 and q[1] < 1e-5 and q[2] < 5e-5


@pytest.mark.gpu
def test_update_is_bit_reproducible():
    g = golden()
    batch, cfg, orders, rows = golden_case(g, "three")
    outs = []
    for _ in range(2):
        pipe = pipeline(g, cfg.minibatch, rows)
        upload(pipe, batch, rows)
        st = [pipe.update(o, cfg) for o in orders]
        outs.append((pipe.actor_params(), pipe.critic_params(), st))
    assert np.array_equal(outs[0][0].view(np.uint64), outs[1][0].view(np.uint64))
    assert np.array_equal(outs[0][1].view(np.uint64), outs[1][1].view(np.uint64))
    assert outs[0][2] == outs[1][2]


@pytest.mark.gpu
def test_moments_and_step_counter_persist_across_updates():
    """Two one-epoch updates equal one pipeline run twice, not two fresh ones:
    the second update's first step uses t = (first update's steps) + 1."""
    g = golden()
    batch, cfg, orders, rows = golden_case(g, "three")
    cfg1 = PpoUpdateCfg(cfg.clip, cfg.entropy_coef, cfg.vdelta, cfg.minibatch, 1, cfg.target_kl, cfg.kl_scale,
                        cfg.kl_mode)
    pipe = pipeline(g, cfg.minibatch, rows)
    upload(pipe, batch, rows)
    pipe.update([orders[0][0]], cfg1)
    pipe.update([orders[0][1]], cfg1)
    a_in, h, act, c_in, hc, _ = (int(x) for x in g["dims"])
    cpu = CpuPpo(Dims(a_in, h, act), Dims(c_in, hc, 1), g["actor0"], g["critic0"])
    b64 = {k: v.astype(np.float64) for k, v in batch.items()}
    for e in (0, 1):
        cpu.update(b64, [orders[0][e]], cfg.clip, cfg.entropy_coef, cfg.vdelta, cfg.minibatch, 1, cfg.target_kl,
                   cfg.kl_scale, int(cfg.kl_mode))
    assert cpu.opt_a.t == 2 * math.ceil(rows / cfg.minibatch)
    assert delta_gap(g["actor0"], cpu.actor, pipe.actor_params()) < 2e-4


@pytest.mark.gpu
def test_errors_carry_the_reference_messages():
    g = golden()
    batch, cfg, orders, rows = golden_case(g, "one")
    pipe = pipeline(g, cfg.minibatch, rows)
    # Nothing uploaded: the update is a no-op with default statistics (train.rs:700-702).
    s = pipe.update(orders[0], cfg)
    assert s.grad_steps == 0 and not s.stopped_early
    with pytest.raises(TrainError, match="parameter array is 3 long, network wants"):
        pipe.set_actor_params(np.zeros(3))
    with pytest.raises(TrainError, match=f"{rows + 1} samples into a pipeline built for {rows}"):
        pipe.upload_batch(rows + 1, SampleBatch(*[np.zeros(1, np.float32)] * 6))
    bad = dict(batch)
    bad["adv"] = bad["adv"][:-1]
    with pytest.raises(TrainError, match=f"adv is {rows - 1} long, expected {rows}"):
        upload(pipe, bad, rows)
    upload(pipe, batch, rows)
    big = PpoUpdateCfg(cfg.clip, cfg.entropy_coef, cfg.vdelta, cfg.minibatch + 1, cfg.epochs, cfg.target_kl,
                       cfg.kl_scale, cfg.kl_mode)
    with pytest.raises(TrainError, match=f"minibatch {cfg.minibatch + 1} exceeds the pipeline's {cfg.minibatch}"):
        pipe.update(orders[0], big)
    with pytest.raises(TrainError, match="2 shuffles for 3 epochs"):
        pipe.update(list(orders[0][:2]), cfg)
    with pytest.raises(TrainError, match=f"shuffle is {rows - 1} long, batch is {rows}"):
        pipe.update([o[:-1] for o in orders[0]], cfg)
    stray = [o.copy() for o in orders[0]]
    stray[2][7] = rows
    with pytest.raises(TrainError, match=f"shuffle 2 holds index {rows}, batch is {rows}"):
        pipe.update(stray, cfg)
    # A rejected update changed nothing.
    np.testing.assert_array_equal(pipe.actor_params(), g["actor0"])

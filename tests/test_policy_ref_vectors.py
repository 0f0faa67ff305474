"""The control-loop oracle (oracle/policy_ref.py) held to the reference's own
kernels: vectors that tests/golden/make_ref_policy_vectors.py took from
phyz_host_fk, phyz_host_obs and phyz_host_policy (crates/phyz-gpu/cuda/
phyz_kernels.cu:1423-1715, 1809-1835) compiled as host C++, the reference's
f32 device code. The reference's own device-versus-CPU check replays the RNG
stream exactly (crates/phyz-gpu/tests/cuda_vs_cpu.rs:874-1120); so does this:
the xorshift64 state after every pass must equal the reference's bit for bit,
and the values drawn from it (input noise, AR(1) action noise, log-probs,
clamped targets) must agree to f32 rounding. Planted mistakes in the oracle
(the Box-Muller sine branch, the action draws before the input noise) fail."""
import math
import os

import numpy as np
import pytest

from oracle import policy_ref as PR
from oracle.oracle import Oracle
from phyz_amd import workloads as W

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_policy_vectors.npz")


@pytest.fixture(scope="module")
def vec():
    z = np.load(FIX)
    nworld, hidden, passes, n_dofs = (int(x) for x in z["dims"])
    cl = W.control_loop(hidden)
    return z, cl, nworld, passes


def test_fk_rows_match_reference(vec):
    z, cl, n, _ = vec
    m = cl.base.model
    orc = Oracle(m)
    q, v = z["q"].astype(np.float64), z["v"].astype(np.float64)
    err = max(np.abs(PR.kinematics_rows(orc, q[w], v[w]) - z["xforms"][w]).max() for w in range(n))
    assert err <= 2e-5, err


def _wrapped(a, b):
    d = a - b
    return np.abs((d + math.pi) % (2 * math.pi) - math.pi)


def test_observation_rows_match_reference(vec):
    z, cl, n, _ = vec
    m = cl.base.model
    orc = Oracle(m)
    q, v = z["q"].astype(np.float64), z["v"].astype(np.float64)
    angular = np.array([op.kind in (3, 4, 5) for op in cl.spec.obs])
    for w in range(n):
        got = np.array(PR.observe_reference(m, orc, q[w], v[w], cl.spec.obs))
        want = z["pass0/obs_clean"][w].astype(np.float64)
        d = np.where(angular, _wrapped(got, want), np.abs(got - want))
        assert d.max() <= 5e-5, (w, int(d.argmax()), d.max())
    for k in range(1, 3):  # the same state each pass: the clean rows repeat
        assert np.array_equal(z[f"pass{k}/obs_clean"], z["pass0/obs_clean"])


def replay(z, cl, n, passes, rng_cls=PR.KernelRng, policy=PR.policy_reference):
    """The oracle's policy passes from the reference's clean observation rows,
    world by world. Returns per pass (noisy obs, actions, logp, targets, z,
    rng states)."""
    spec = cl.spec
    weights = z["weights"].astype(np.float64)
    std = z["std"].astype(np.float64)
    base = z["base_targets"].astype(np.float64)
    rngs = [rng_cls(int(s)) for s in z["seeds"]]
    zs = np.zeros((n, spec.n_out()))
    out = []
    for k in range(passes):
        obs = z[f"pass{k}/obs_clean"].astype(np.float64).copy()
        act = np.zeros((n, spec.n_out()))
        logp = np.zeros(n)
        tg = np.zeros_like(base)
        for w in range(n):
            act[w], logp[w] = policy(spec, weights, std, rngs[w], obs[w], zs[w], base[w], tg[w])
        out.append((obs, act, logp, tg, zs.copy(), np.array([r.state for r in rngs], dtype=np.uint64)))
    return out


def mismatch(z, res, n_out):
    """Largest disagreement with the reference over every pass, and whether
    every RNG state matches bit for bit."""
    worst = 0.0
    states_equal = True
    for k, (obs, act, logp, tg, zs, st) in enumerate(res):
        ref_out = z[f"pass{k}/out"].astype(np.float64)
        words = z[f"pass{k}/rng_words"].astype(np.uint64)
        ref_state = (words[:, 1] << np.uint64(32)) | words[:, 0]
        states_equal &= bool(np.array_equal(st, ref_state))
        worst = max(worst,
                    np.abs(obs - z[f"pass{k}/obs_noisy"]).max(),
                    np.abs(act - ref_out[:, :n_out]).max(),
                    np.abs(logp - ref_out[:, n_out]).max() / 10.0,
                    np.abs(tg - z[f"pass{k}/targets"]).max(),
                    np.abs(zs - z[f"pass{k}/z"]).max())
    return worst, states_equal


def test_policy_passes_replay_reference_stream(vec):
    z, cl, n, passes = vec
    res = replay(z, cl, n, passes)
    worst, states_equal = mismatch(z, res, cl.spec.n_out())
    assert states_equal
    assert worst <= 2e-5, worst
    # The vectors exercise the clamp: some actions beyond +-act_clamp.
    acts = np.concatenate([r[1] for r in res])
    assert (np.abs(acts) > cl.spec.act_clamp).any() and (np.abs(acts) < cl.spec.act_clamp).any()


class SineRng(PR.KernelRng):
    """A planted mistake: the Box-Muller sine branch."""

    def normal(self):
        u1 = self.uniform()
        u2 = self.uniform()
        return math.sqrt(-2.0 * math.log(max(u1, 1e-300))) * math.sin(2.0 * math.pi * u2)


def actions_first(spec, weights, std, rng, obs, z, base, targets):
    """A planted mistake: the action draws before the input noise."""
    keep = math.sqrt(max(1.0 - spec.noise_rho ** 2, 0.0))
    draws = [rng.normal() for _ in range(spec.n_out())]
    for i in range(len(obs)):
        if spec.input_noise[i] != 0.0:
            obs[i] += spec.input_noise[i] * rng.normal()
    targets[:] = base
    mean = PR.mlp_forward(spec.n_in(), spec.hidden, spec.n_out(), weights, obs)
    act = np.zeros(spec.n_out())
    logp = 0.0
    for k in range(spec.n_out()):
        z[k] = spec.noise_rho * z[k] + keep * draws[k]
        act[k] = mean[k] + std[k] * z[k]
        logp += -0.5 * z[k] ** 2 - math.log(std[k]) - 0.5 * math.log(2 * math.pi)
        lim = spec.clamp_at(k)
        targets[spec.act_slots[k]] = base[spec.act_slots[k]] + min(max(act[k], -lim), lim)
    return act, logp


@pytest.mark.parametrize("planted", ["sine_branch", "actions_first"])
def test_planted_stream_mistakes_fail(vec, planted):
    z, cl, n, passes = vec
    if planted == "sine_branch":
        res = replay(z, cl, n, passes, rng_cls=SineRng)
    else:
        res = replay(z, cl, n, passes, policy=actions_first)
    worst, _ = mismatch(z, res, cl.spec.n_out())
    assert worst > 1e-2, worst

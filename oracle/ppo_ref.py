"""CPU restatements of the PPO update pass — TEST INFRASTRUCTURE ONLY.

Used by tests/, tests/golden/ scripts and bench.py's cpu_baseline leg; the
product (phyz_amd) never imports this module.

CpuPpo restates, in f64 numpy, the CPU update loop the reference's device pass
is refereed against (crates/phyz-gpu/tests/train_parity.rs:166-296,
`cpu_update`): a three-layer tanh MLP actor with a global learned log_std and
a three-layer tanh MLP critic, as tang's Linear / Tanh modules compute them
(y = x W^T + b, W [out][in]), and tang's ModuleAdam with one step counter per
network. tang (git dependency tang @ 9d28b81, Cargo.toml:26-30, 101-104) is not
vendored in the reference tree; its Adam is restated from the semantics the
reference's kernels encode for it (crates/phyz-gpu/cuda/phyz_train.cu:262-288:
decoupled weight decay, bias corrections 1 - beta^t with t counted from 1).

RefHostPipeline drives the reference's own update kernels, compiled as host
C++ from crates/phyz-gpu/cuda/phyz_train.cu into oracle/_ref (the reference's
`cuda-host` build), through the minibatch loop of TrainPipeline::update and
DeviceNet::backward_and_step (crates/phyz-gpu/src/cuda/train.rs:447-500,
692-791), restated here. It is what the reference's CI runs on machines with
no GPU, and it pins CpuPpo (tests/test_ppo_oracle.py).
"""
from __future__ import annotations

import ctypes as C
import math
import os
from dataclasses import dataclass
from typing import List, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
TRAIN_REF_LIB = os.path.join(HERE, "_ref", "libphyz_train_ref_host.so")

LN_2PI = math.log(2.0 * math.pi)


@dataclass(frozen=True)
class Dims:
    n_in: int
    n_h: int
    n_out: int

    def param_count(self) -> int:
        return self.n_h * self.n_in + self.n_h + self.n_h * self.n_h + self.n_h + self.n_out * self.n_h + self.n_out

    # Offsets of tang's Mlp::to_flat order (phyz_train.cu:62-93).
    def offsets(self):
        o_w1 = 0
        o_b1 = o_w1 + self.n_h * self.n_in
        o_w2 = o_b1 + self.n_h
        o_b2 = o_w2 + self.n_h * self.n_h
        o_w3 = o_b2 + self.n_h
        o_b3 = o_w3 + self.n_out * self.n_h
        return o_w1, o_b1, o_w2, o_b2, o_w3, o_b3


def unpack(flat: np.ndarray, d: Dims):
    o_w1, o_b1, o_w2, o_b2, o_w3, o_b3 = d.offsets()
    W1 = flat[o_w1:o_b1].reshape(d.n_h, d.n_in)
    b1 = flat[o_b1:o_w2]
    W2 = flat[o_w2:o_b2].reshape(d.n_h, d.n_h)
    b2 = flat[o_b2:o_w3]
    W3 = flat[o_w3:o_b3].reshape(d.n_out, d.n_h)
    b3 = flat[o_b3:o_b3 + d.n_out]
    return W1, b1, W2, b2, W3, b3


def mlp_forward(flat: np.ndarray, d: Dims, X: np.ndarray):
    """tang Linear -> Tanh -> Linear -> Tanh -> Linear: (h1, h2, out)."""
    W1, b1, W2, b2, W3, b3 = unpack(flat, d)
    h1 = np.tanh(X @ W1.T + b1)
    h2 = np.tanh(h1 @ W2.T + b2)
    return h1, h2, h2 @ W3.T + b3


def mlp_backward(flat: np.ndarray, d: Dims, X, h1, h2, dout) -> np.ndarray:
    """Parameter gradient (flat, MLP part) of sum(dout * out)."""
    W1, b1, W2, b2, W3, b3 = unpack(flat, d)
    g = np.zeros(d.param_count())
    o_w1, o_b1, o_w2, o_b2, o_w3, o_b3 = d.offsets()
    g[o_w3:o_b3] = (dout.T @ h2).reshape(-1)
    g[o_b3:o_b3 + d.n_out] = dout.sum(axis=0)
    dh2 = (dout @ W3) * (1.0 - h2 * h2)
    g[o_w2:o_b2] = (dh2.T @ h1).reshape(-1)
    g[o_b2:o_w3] = dh2.sum(axis=0)
    dh1 = (dh2 @ W2) * (1.0 - h1 * h1)
    g[o_w1:o_b1] = (dh1.T @ X).reshape(-1)
    g[o_b1:o_w2] = dh1.sum(axis=0)
    return g


class Adam:
    """tang's ModuleAdam over one flat parameter array with one step counter."""

    def __init__(self, n: int, lr=3e-4, beta1=0.9, beta2=0.999, epsilon=1e-8, weight_decay=0.0):
        self.m = np.zeros(n)
        self.v = np.zeros(n)
        self.t = 0
        self.lr, self.beta1, self.beta2, self.eps, self.wd = lr, beta1, beta2, epsilon, weight_decay

    def step(self, p: np.ndarray, g: np.ndarray) -> None:
        self.t += 1
        bc1 = 1.0 - self.beta1 ** self.t
        bc2 = 1.0 - self.beta2 ** self.t
        if self.wd > 0.0:
            p *= 1.0 - self.lr * self.wd
        self.m = self.beta1 * self.m + (1.0 - self.beta1) * g
        self.v = self.beta2 * self.v + (1.0 - self.beta2) * g * g
        p -= self.lr * (self.m / bc1) / (np.sqrt(self.v / bc2) + self.eps)


@dataclass
class Stats:
    policy_loss: float
    value_loss: float
    kl: float
    grad_steps: int
    stopped_early: bool


class CpuPpo:
    """The f64 CPU update (train_parity.rs:166-296), state kept across updates."""

    def __init__(self, actor: Dims, critic: Dims, actor_flat, critic_flat, adam_actor=None, adam_critic=None):
        self.ad, self.cd = actor, critic
        self.actor = np.array(actor_flat, dtype=np.float64)
        self.critic = np.array(critic_flat, dtype=np.float64)
        assert self.actor.size == actor.param_count() + actor.n_out and self.critic.size == critic.param_count()
        self.opt_a = Adam(self.actor.size, **(adam_actor or {}))
        self.opt_c = Adam(self.critic.size, **(adam_critic or {}))

    def minibatch_grads(self, batch: dict, chunk: np.ndarray, clip, entropy_coef, vdelta) -> dict:
        """Gradients of both networks for one minibatch (rows `chunk`), and its
        statistics: the body of the minibatch loop before the Adam steps."""
        ad, cd = self.ad, self.cd
        A = ad.n_out
        off_ls = ad.param_count()
        nb = chunk.size
        xa, xc = batch["obs_a"][chunk], batch["obs_c"][chunk]
        # ── actor: clipped surrogate, gradient through the active branch only ──
        h1, h2, mean = mlp_forward(self.actor, ad, xa)
        std = np.exp(self.actor[off_ls:off_ls + A])
        z = (batch["act"][chunk] - mean) / std
        logp = (-0.5 * z * z - np.log(std) - 0.5 * LN_2PI).sum(axis=1)
        lp_old = batch["logp_old"][chunk]
        log_ratio = logp - lp_old
        ratio = np.exp(log_ratio)
        clipped = np.clip(ratio, 1.0 - clip, 1.0 + clip)
        adv = batch["adv"][chunk]
        uo, co = ratio * adv, clipped * adv
        active = uo <= co + 1e-12
        coef = np.where(active, -adv * ratio / nb, 0.0)[:, None]
        g_a = np.zeros(self.actor.size)
        g_a[:off_ls] = mlp_backward(self.actor, ad, xa, h1, h2, coef * (z / std))
        g_a[off_ls:] = (coef * (z * z - 1.0)).sum(axis=0) - entropy_coef
        # ── critic: squared error, gradient Huber-clipped at vdelta ──
        c1, c2, values = mlp_forward(self.critic, cd, xc)
        err = values[:, 0] - batch["ret"][chunk]
        dv = (2.0 * np.clip(err, -vdelta, vdelta) / nb)[:, None]
        g_c = mlp_backward(self.critic, cd, xc, c1, c2, dv)
        return {"g_actor": g_a, "g_critic": g_c, "ploss": float((-np.minimum(uo, co)).sum()),
                "vloss": float((err * err).sum()), "kl_sum": float((lp_old - logp).sum()),
                "k3_sum": float((ratio - 1.0 - log_ratio).sum()), "rows": nb}

    def update(self, batch: dict, order: Sequence[Sequence[int]], clip, entropy_coef, vdelta, minibatch, epochs,
               target_kl, kl_scale, kl_mode) -> Stats:
        """batch: obs_a [n, a_in], obs_c [n, c_in], act [n, n_out], logp_old, adv, ret [n] (f64).
        kl_mode 0 cumulative, 1 minibatch."""
        policy_acc = value_acc = brake_acc = kl_acc = 0.0
        batches = kl_rows = 0
        stopped = False
        for ep in list(order)[:epochs]:
            ep = np.asarray(ep, dtype=np.int64)
            for s in range(0, ep.size, minibatch):
                mb = self.minibatch_grads(batch, ep[s:s + minibatch], clip, entropy_coef, vdelta)
                nb = mb["rows"]
                self.opt_a.step(self.actor, mb["g_actor"])
                self.opt_c.step(self.critic, mb["g_critic"])
                policy_acc += mb["ploss"] / nb
                value_acc += mb["vloss"] / nb
                kl_acc += mb["kl_sum"]
                kl_rows += nb
                brake = (abs(kl_acc / max(kl_rows, 1)) if kl_mode == 0 else mb["k3_sum"] / nb) / kl_scale
                brake_acc += brake
                batches += 1
                if brake > target_kl:
                    stopped = True
                    break
            if stopped:
                break
        nbm = max(batches, 1)
        return Stats(policy_acc / nbm, value_acc / nbm, brake_acc / nbm, batches, stopped)


# ── the reference's own kernels (host build), driven by the reference loop ──
_u32 = C.c_uint32
_fp = C.POINTER(C.c_float)
_dp = C.POINTER(C.c_double)
_up = C.POINTER(C.c_uint32)


def ref_available() -> bool:
    return os.path.exists(TRAIN_REF_LIB)


def _ref_lib():
    L = C.CDLL(TRAIN_REF_LIB)
    sig = {
        "phyz_train_host_fwd": [_u32, _u32, _u32, _u32, _u32, _fp, _fp, _up, _fp, _fp, _fp],
        "phyz_train_host_ppo_grad": [_u32, _u32, _u32, C.c_float, C.c_float, _fp, _fp, _fp, _fp, _fp, _up, _fp, _fp,
                                     _fp],
        "phyz_train_host_value_grad": [_u32, _u32, C.c_float, _fp, _fp, _up, _fp, _fp],
        "phyz_train_host_bwd_hidden": [_u32, _u32, _u32, _u32, _fp, _fp, _fp, _fp],
        "phyz_train_host_grad_w_idx": [_u32, _u32, _u32, _u32, _fp, _fp, _up, _fp, _u32],
        "phyz_train_host_grad_w": [_u32, _u32, _u32, _u32, _fp, _fp, _fp, _u32],
        "phyz_train_host_grad_b": [_u32, _u32, _u32, _fp, _fp, _u32],
        "phyz_train_host_adam": [_u32, _u32, C.c_double, C.c_double, C.c_double, C.c_double, C.c_double, C.c_double,
                                 C.c_double, _fp, _dp, _dp, _dp, _fp],
        "phyz_train_host_reduce_stats": [_u32, _u32, _fp, _fp],
    }
    for name, args in sig.items():
        f = getattr(L, name)
        f.restype = None
        f.argtypes = args
    return L


def _f(a: np.ndarray, off: int = 0):
    return C.cast(a.ctypes.data + 4 * off, _fp)


def _d(a: np.ndarray):
    return a.ctypes.data_as(_dp)


class _RefNet:
    def __init__(self, d: Dims, extra: int, max_b: int, flat):
        self.d = d
        self.n = d.param_count() + extra
        self.p = np.array(flat, dtype=np.float64)
        self.w = self.p.astype(np.float32)
        self.m = np.zeros(self.n)
        self.v = np.zeros(self.n)
        self.g = np.zeros(self.n, dtype=np.float32)
        self.h1 = np.zeros(max_b * d.n_h, dtype=np.float32)
        self.h2 = np.zeros(max_b * d.n_h, dtype=np.float32)
        self.out = np.zeros(max_b * d.n_out, dtype=np.float32)
        w = max(d.n_h, d.n_out)
        self.dh = np.zeros(max_b * w, dtype=np.float32)
        self.dout = np.zeros(max_b * w, dtype=np.float32)
        self.t = 0


class RefHostPipeline:
    """TrainPipeline::update over the reference's host-compiled kernels."""

    def __init__(self, actor: Dims, critic: Dims, actor_flat, critic_flat, max_b: int, adam=(3e-4, 0.9, 0.999, 1e-8, 0.0)):
        self.L = _ref_lib()
        self.a = _RefNet(actor, actor.n_out, max_b, actor_flat)
        self.c = _RefNet(critic, 0, max_b, critic_flat)
        self.adam = adam
        self.max_b = max_b

    def _backward_and_step(self, net: _RefNet, b: int, x: np.ndarray, idx: np.ndarray):
        L, d = self.L, net.d
        o_w1, o_b1, o_w2, o_b2, o_w3, o_b3 = d.offsets()
        ip = idx.ctypes.data_as(_up)
        L.phyz_train_host_grad_w(d.n_out * d.n_h, b, d.n_out, d.n_h, _f(net.dout), _f(net.h2), _f(net.g), o_w3)
        L.phyz_train_host_grad_b(d.n_out, b, d.n_out, _f(net.dout), _f(net.g), o_b3)
        L.phyz_train_host_bwd_hidden(b * d.n_h, b, d.n_out, d.n_h, _f(net.dout), _f(net.w, o_w3), _f(net.h2),
                                     _f(net.dh))
        net.dh, net.dout = net.dout, net.dh
        L.phyz_train_host_grad_w(d.n_h * d.n_h, b, d.n_h, d.n_h, _f(net.dout), _f(net.h1), _f(net.g), o_w2)
        L.phyz_train_host_grad_b(d.n_h, b, d.n_h, _f(net.dout), _f(net.g), o_b2)
        L.phyz_train_host_bwd_hidden(b * d.n_h, b, d.n_h, d.n_h, _f(net.dout), _f(net.w, o_w2), _f(net.h1),
                                     _f(net.dh))
        net.dh, net.dout = net.dout, net.dh
        L.phyz_train_host_grad_w_idx(d.n_h * d.n_in, b, d.n_h, d.n_in, _f(net.dout), _f(x), ip, _f(net.g), 0)
        L.phyz_train_host_grad_b(d.n_h, b, d.n_h, _f(net.dout), _f(net.g), o_b1)
        net.t += 1
        lr, b1, b2, eps, wd = self.adam
        L.phyz_train_host_adam(net.n, net.n, lr, b1, b2, eps, wd, 1.0 - b1 ** net.t, 1.0 - b2 ** net.t, _f(net.g),
                               _d(net.m), _d(net.v), _d(net.p), _f(net.w))

    def update(self, batch32: dict, order, clip, entropy_coef, vdelta, minibatch, epochs, target_kl, kl_scale,
               kl_mode) -> Stats:
        """batch32: the f32 columns, row-major."""
        L, a, c = self.L, self.a, self.c
        ad, cd = a.d, c.d
        cols = {k: np.ascontiguousarray(v, dtype=np.float32).reshape(-1) for k, v in batch32.items()}
        stats = np.zeros(self.max_b * 4, dtype=np.float32)
        dls = np.zeros(self.max_b * ad.n_out, dtype=np.float32)
        red = np.zeros(4, dtype=np.float32)
        off_ls = ad.param_count()
        policy_acc = value_acc = brake_acc = kl_acc = 0.0
        batches = kl_rows = 0
        stopped = False
        for ep in list(order)[:epochs]:
            ep = np.ascontiguousarray(ep, dtype=np.uint32)
            for s in range(0, ep.size, minibatch):
                idx = np.ascontiguousarray(ep[s:s + minibatch])
                b = idx.size
                ip = idx.ctypes.data_as(_up)
                L.phyz_train_host_fwd(b, b, ad.n_in, ad.n_h, ad.n_out, _f(a.w), _f(cols["obs_a"]), ip, _f(a.h1),
                                      _f(a.h2), _f(a.out))
                L.phyz_train_host_ppo_grad(b, b, ad.n_out, clip, entropy_coef, _f(a.out), _f(a.w, off_ls),
                                           _f(cols["act"]), _f(cols["logp_old"]), _f(cols["adv"]), ip, _f(a.dout),
                                           _f(dls), _f(stats))
                L.phyz_train_host_grad_b(ad.n_out, b, ad.n_out, _f(dls), _f(a.g), off_ls)
                self._backward_and_step(a, b, cols["obs_a"], idx)
                L.phyz_train_host_fwd(b, b, cd.n_in, cd.n_h, cd.n_out, _f(c.w), _f(cols["obs_c"]), ip, _f(c.h1),
                                      _f(c.h2), _f(c.out))
                L.phyz_train_host_value_grad(b, b, vdelta, _f(c.out), _f(cols["ret"]), ip, _f(c.dout), _f(stats))
                self._backward_and_step(c, b, cols["obs_c"], idx)
                L.phyz_train_host_reduce_stats(4, b, _f(stats), _f(red))
                ploss, kl_sum, k3_sum, vloss = (float(x) for x in red)
                policy_acc += ploss / b
                value_acc += vloss / b
                kl_acc += kl_sum
                kl_rows += b
                brake = (abs(kl_acc / max(kl_rows, 1)) if kl_mode == 0 else k3_sum / b) / kl_scale
                brake_acc += brake
                batches += 1
                if brake > target_kl:
                    stopped = True
                    break
            if stopped:
                break
        nbm = max(batches, 1)
        return Stats(policy_acc / nbm, value_acc / nbm, brake_acc / nbm, batches, stopped)

    def actor_params(self) -> np.ndarray:
        return self.a.p.copy()

    def critic_params(self) -> np.ndarray:
        return self.c.p.copy()


# ── the reference test's problem (train_parity.rs:29-94) ───────────────────
class XorShift:
    """Marsaglia xorshift64 (13, 7, 17) with the test's uniform and Box-Muller normal."""

    def __init__(self, seed: int):
        self.s = seed & 0xFFFFFFFFFFFFFFFF

    def next(self) -> int:
        x = self.s
        x ^= (x << 13) & 0xFFFFFFFFFFFFFFFF
        x ^= x >> 7
        x ^= (x << 17) & 0xFFFFFFFFFFFFFFFF
        self.s = x
        return x

    def uniform(self) -> float:
        return (self.next() >> 11) / float(1 << 53)

    def normal(self) -> float:
        u1 = max(self.uniform(), 1e-12)
        u2 = self.uniform()
        return math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2)


def make_batch(seed: int, n: int, a_in: int, c_in: int, act: int, logp_mean: float = -4.0) -> dict:
    """The parity test's synthetic batch (train_parity.rs:64-83), f64."""
    r = XorShift(seed)
    return {
        "obs_a": np.array([r.normal() * 0.5 for _ in range(n * a_in)]).reshape(n, a_in),
        "obs_c": np.array([r.normal() * 0.5 for _ in range(n * c_in)]).reshape(n, c_in),
        "act": np.array([r.normal() * 0.3 for _ in range(n * act)]).reshape(n, act),
        "logp_old": np.array([logp_mean + r.normal() * 0.4 for _ in range(n)]),
        "adv": np.array([r.normal() for _ in range(n)]),
        "ret": np.array([r.normal() * 2.0 for _ in range(n)]),
    }


def shuffles(seed: int, n: int, epochs: int) -> List[np.ndarray]:
    """Fisher-Yates with the test's generator (train_parity.rs:85-98)."""
    r = XorShift(seed)
    out = []
    for _ in range(epochs):
        o = list(range(n))
        for i in range(n - 1, 0, -1):
            j = r.next() % (i + 1)
            o[i], o[j] = o[j], o[i]
        out.append(np.array(o, dtype=np.uint32))
    return out


def init_flat(seed: int, d: Dims, extra: int = 0, extra_value: float = 0.0) -> np.ndarray:
    """Weights uniform in +-1/sqrt(fan_in), biases zero, `extra` trailing entries
    (the actor's log_std) at extra_value."""
    r = XorShift(seed)
    flat = np.zeros(d.param_count() + extra)
    o_w1, o_b1, o_w2, o_b2, o_w3, o_b3 = d.offsets()
    for lo, hi, fan in ((o_w1, o_b1, d.n_in), (o_w2, o_b2, d.n_h), (o_w3, o_b3, d.n_h)):
        k = 1.0 / math.sqrt(fan)
        flat[lo:hi] = [(2.0 * r.uniform() - 1.0) * k for _ in range(hi - lo)]
    flat[d.param_count():] = extra_value
    return flat


def policy_logp(actor_flat, ad: Dims, obs_a: np.ndarray, act: np.ndarray) -> np.ndarray:
    """Log-probability of `act` under the Gaussian policy `actor_flat` (f64)."""
    _, _, mean = mlp_forward(np.asarray(actor_flat, dtype=np.float64), ad, obs_a)
    std = np.exp(np.asarray(actor_flat)[ad.param_count():ad.param_count() + ad.n_out])
    z = (act - mean) / std
    return (-0.5 * z * z - np.log(std) - 0.5 * LN_2PI).sum(axis=1)

"""The PPO update pass on the device: the reference's TrainPipeline
(crates/phyz-gpu/src/cuda/train.rs:523-805) over the C ABI of
phyz_amd/csrc/phz_train.hip.

Same names, argument meanings and error messages as the reference:

    pipe = TrainPipeline(NetDims(55, 64, 22), NetDims(67, 64, 1), capacity, max_b)
    pipe.set_adam(AdamCfg(), AdamCfg())
    pipe.set_actor_params(actor_flat)       # tang's Mlp::to_flat order + log_std
    pipe.set_critic_params(critic_flat)
    pipe.upload_batch(n_rows, SampleBatch(obs_a, obs_c, act, logp_old, adv, ret))
    stats = pipe.update(order, PpoUpdateCfg(...))   # order[e]: epoch e's shuffle
    actor_flat = pipe.actor_params()

Errors raise TrainError with the library's message. There is no host
fallback: the kernels run on a HIP device or not at all.
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import _lib

TRAIN_MAX_H = 256    # train.rs:46
TRAIN_MAX_OUT = 64   # train.rs:50


class TrainError(RuntimeError):
    pass


@dataclass(frozen=True)
class NetDims:
    """A three-layer tanh MLP's shape (train.rs:53-100)."""
    n_in: int
    n_h: int
    n_out: int

    def param_count(self) -> int:
        """W1, b1, W2, b2, W3, b3 — tang's Mlp::to_flat."""
        return self.n_h * self.n_in + self.n_h + self.n_h * self.n_h + self.n_h + self.n_out * self.n_h + self.n_out

    def off_logstd(self) -> int:
        """Offset of the actor's log_std block, after b3."""
        return self.param_count()


@dataclass(frozen=True)
class AdamCfg:
    """tang's ModuleAdam settings (train.rs:102-129)."""
    lr: float = 3e-4
    beta1: float = 0.9
    beta2: float = 0.999
    epsilon: float = 1e-8
    weight_decay: float = 0.0


class KlMode(enum.IntEnum):
    """How the brake reads the divergence (train.rs:150-156)."""
    CUMULATIVE = 0   # |mean of logp_old - logp| over every row so far this update
    MINIBATCH = 1    # Schulman's k3 over the current minibatch


@dataclass(frozen=True)
class PpoUpdateCfg:
    """train.rs:131-148."""
    clip: float
    entropy_coef: float
    vdelta: float
    minibatch: int
    epochs: int
    target_kl: float
    kl_scale: float
    kl_mode: KlMode


@dataclass(frozen=True)
class UpdateStats:
    """train.rs:158-172."""
    policy_loss: float = 0.0
    value_loss: float = 0.0
    kl: float = 0.0
    grad_steps: int = 0
    stopped_early: bool = False


@dataclass
class SampleBatch:
    """One iteration's samples, already GAE'd and normalized (train.rs:509-522).
    Row-major f32: obs_a [n, actor n_in], obs_c [n, critic n_in], act
    [n, actor n_out], logp_old / adv / ret [n]."""
    obs_a: np.ndarray
    obs_c: np.ndarray
    act: np.ndarray
    logp_old: np.ndarray
    adv: np.ndarray
    ret: np.ndarray


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32).reshape(-1))


class TrainPipeline:
    """The device-resident PPO update (train.rs:523-805)."""

    def __init__(self, actor: NetDims, critic: NetDims, capacity: int, max_b: int, device: int = 0):
        self._L = _lib.load()
        self.actor_dims, self.critic_dims = actor, critic
        self.capacity, self.max_b = int(capacity), int(max_b)
        h = C.c_void_p()
        rc = self._L.phz_train_create(_lib.NetDims(actor.n_in, actor.n_h, actor.n_out),
                                      _lib.NetDims(critic.n_in, critic.n_h, critic.n_out),
                                      self.capacity, self.max_b, int(device), C.byref(h))
        if rc != 0:
            raise TrainError(self._L.phz_train_last_error(None).decode())
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._L.phz_train_destroy(h)
            self._h = None

    def _check(self, rc: int):
        if rc != 0:
            raise TrainError(self._L.phz_train_last_error(self._h).decode())

    # ── configuration and weights ──
    def device_name(self) -> str:
        buf = C.create_string_buffer(256)
        self._check(self._L.phz_train_device_name(self._h, buf, len(buf)))
        return buf.value.decode()

    @property
    def rows_per_tile(self) -> int:
        return int(self._L.phz_train_rows_per_tile(self._h))

    def set_adam(self, actor: AdamCfg, critic: AdamCfg):
        a = _lib.AdamCfg(actor.lr, actor.beta1, actor.beta2, actor.epsilon, actor.weight_decay)
        c = _lib.AdamCfg(critic.lr, critic.beta1, critic.beta2, critic.epsilon, critic.weight_decay)
        self._check(self._L.phz_train_set_adam(self._h, C.byref(a), C.byref(c)))

    def _set(self, fn, flat):
        f = np.ascontiguousarray(np.asarray(flat, dtype=np.float64).reshape(-1))
        self._check(fn(self._h, f.ctypes.data_as(_lib.dp), f.size))

    def _get(self, fn, net: int) -> np.ndarray:
        n = int(self._L.phz_train_param_count(self._h, net))
        out = np.zeros(n)
        self._check(fn(self._h, out.ctypes.data_as(_lib.dp), n))
        return out

    def set_actor_params(self, flat):
        """tang's flat Mlp order with log_std appended."""
        self._set(self._L.phz_train_set_actor_params, flat)

    def set_critic_params(self, flat):
        self._set(self._L.phz_train_set_critic_params, flat)

    def actor_params(self) -> np.ndarray:
        return self._get(self._L.phz_train_actor_params, 0)

    def critic_params(self) -> np.ndarray:
        return self._get(self._L.phz_train_critic_params, 1)

    # ── samples and the update ──
    def upload_batch(self, n_rows: int, batch: SampleBatch):
        cols = [_f32(getattr(batch, k)) for k in ("obs_a", "obs_c", "act", "logp_old", "adv", "ret")]
        args = []
        for c in cols:
            args += [c.ctypes.data_as(_lib.fp), c.size]
        self._check(self._L.phz_train_upload_batch(self._h, int(n_rows), *args))

    @staticmethod
    def _args(order, cfg):
        shuffles = [np.ascontiguousarray(np.asarray(o, dtype=np.uint32).reshape(-1)) for o in order]
        n = len(shuffles)
        ptrs = (_lib.u32p * max(n, 1))(*[s.ctypes.data_as(_lib.u32p) for s in shuffles])
        lens = (C.c_uint64 * max(n, 1))(*[s.size for s in shuffles])
        c = _lib.PpoCfg(float(cfg.clip), float(cfg.entropy_coef), float(cfg.vdelta), int(cfg.minibatch),
                        int(cfg.epochs), float(cfg.target_kl), float(cfg.kl_scale), int(cfg.kl_mode))
        return shuffles, ptrs, lens, n, c

    @staticmethod
    def _stats(out) -> UpdateStats:
        return UpdateStats(out.policy_loss, out.value_loss, out.kl, int(out.grad_steps), bool(out.stopped_early))

    def update(self, order: Sequence[Sequence[int]], cfg: PpoUpdateCfg) -> UpdateStats:
        """cfg.epochs passes over the uploaded batch; order[e] is epoch e's shuffle
        of 0..n_rows (the caller owns the PRNG, as in the reference)."""
        keep, ptrs, lens, n, c = self._args(order, cfg)
        out = _lib.UpdateStats()
        self._check(self._L.phz_train_update(self._h, ptrs, lens, n, C.byref(c), C.byref(out)))
        return self._stats(out)

    def time_update(self, order: Sequence[Sequence[int]], cfg: PpoUpdateCfg):
        """An update with hipEvents around every launch: (stats, summed ms of the
        tile kernel and of the Adam + brake kernel, minibatches launched)."""
        keep, ptrs, lens, n, c = self._args(order, cfg)
        out = _lib.UpdateStats()
        ms = np.zeros(2)
        mbs = C.c_uint64()
        self._check(self._L.phz_train_time_update(self._h, ptrs, lens, n, C.byref(c), C.byref(out),
                                                  ms.ctypes.data_as(_lib.dp), C.byref(mbs)))
        return self._stats(out), ms, int(mbs.value)


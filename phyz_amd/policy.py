"""Policy specification for the device-resident control loop.

Mirrors crates/phyz-gpu/src/policy_pipeline.rs: the observation ops (ObsOp,
lines 47-113), their packed table form (ObsOp::pack / aux / pack_obs_ops,
lines 115-151 and 285-297) and PolicySpec (lines 300-355). Validation with the
reference's messages happens in the library (phz_enable_policy); the checks
here are the two the flat C ABI cannot see (vector lengths).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import numpy as np

XF_STRIDE = 18
OBS_OP_STRIDE = 4
POLICY_MAX_IN = 128
POLICY_MAX_H = 256
POLICY_MAX_OUT = 32
SUPPORT_STRIDE = 4


class ObsOp:
    """One observation feature; `row(aux_off)` is its [kind, a, b, c] table row."""

    kind = -1

    def row(self, aux_off: int) -> List[float]:
        raise NotImplementedError

    def aux(self) -> List[float]:
        return []


@dataclass
class Const(ObsOp):
    c: float
    kind = 0

    def row(self, aux_off):
        return [0.0, 0.0, 0.0, float(self.c)]


@dataclass
class QMinus(ObsOp):
    i: int
    c: float
    kind = 1

    def row(self, aux_off):
        return [1.0, float(self.i), 0.0, float(self.c)]


@dataclass
class V(ObsOp):
    i: int
    kind = 2

    def row(self, aux_off):
        return [2.0, float(self.i), 0.0, 0.0]


@dataclass
class BodyPitch(ObsOp):
    body: int
    kind = 3

    def row(self, aux_off):
        return [3.0, float(self.body), 0.0, 0.0]


@dataclass
class BodyRoll(ObsOp):
    body: int
    kind = 4

    def row(self, aux_off):
        return [4.0, float(self.body), 0.0, 0.0]


@dataclass
class BodyYawError(ObsOp):
    body: int
    cmd: float
    kind = 5

    def row(self, aux_off):
        return [5.0, float(self.body), 0.0, float(self.cmd)]


@dataclass
class BodyPosZ(ObsOp):
    body: int
    kind = 6

    def row(self, aux_off):
        return [6.0, float(self.body), 0.0, 0.0]


@dataclass
class BodyPos(ObsOp):
    body: int
    axis: int
    kind = 7

    def row(self, aux_off):
        return [7.0, float(self.body), float(self.axis), 0.0]


@dataclass
class ComOverSupport(ObsOp):
    """Centre of mass minus the mean of body-frame support points, one axis,
    optionally in `heading_body`'s yaw frame (policy_pipeline.rs:81-112)."""
    support: Sequence[Tuple[int, Sequence[float]]]
    heading_body: Optional[int]
    axis: int
    kind = 8

    def row(self, aux_off):
        return [8.0, float(aux_off), float(len(self.support)), float(self.axis)]

    def aux(self):
        a = [1.0 if self.heading_body is not None else 0.0,
             float(self.heading_body if self.heading_body is not None else 0)]
        for b, o in self.support:
            a.append(float(b))
            a.extend(float(x) for x in o)
        return a


def pack_obs_ops(ops: Sequence[ObsOp]) -> Tuple[np.ndarray, np.ndarray]:
    """(table [n_in][4], aux) as pack_obs_ops (policy_pipeline.rs:285-297), in f64."""
    table, aux = [], []
    for op in ops:
        table.append(op.row(len(aux)))
        aux.extend(op.aux())
    return np.asarray(table, dtype=np.float64).reshape(len(ops), OBS_OP_STRIDE), np.asarray(aux, dtype=np.float64)


@dataclass
class PolicySpec:
    """PolicySpec (policy_pipeline.rs:300-355)."""
    obs: List[ObsOp]
    hidden: int
    act_slots: List[int]
    act_clamp: float
    act_clamp_slots: Optional[List[float]] = None
    noise_rho: float = 0.0
    input_noise: List[float] = field(default_factory=list)
    history_steps: int = 1

    def n_in(self) -> int:
        return len(self.obs)

    def n_out(self) -> int:
        return len(self.act_slots)

    def clamp_at(self, k: int) -> float:
        return self.act_clamp_slots[k] if self.act_clamp_slots is not None else self.act_clamp

    def n_weights(self) -> int:
        i, h, o = self.n_in(), self.hidden, self.n_out()
        return i * h + h + h * h + h + h * o + o

    def check_lengths(self) -> None:
        """The two PolicySpec::validate checks on vector lengths (policy_pipeline.rs:383-398)."""
        if self.act_clamp_slots is not None and len(self.act_clamp_slots) != self.n_out():
            raise ValueError(f"act_clamp_slots has {len(self.act_clamp_slots)} entries for {self.n_out()} actions")
        if len(self.input_noise) != self.n_in():
            raise ValueError(f"input_noise has {len(self.input_noise)} entries for {self.n_in()} inputs")

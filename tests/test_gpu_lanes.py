"""Split-lane step kernels (small launches give each world 2 or 4 lanes that
share its revolute joints' sincos) against the one-lane kernel of the same
size (PHZ_LANES=1). The split kernel is forced (PHZ_LANES=2 or 4) so that the
f32 four-lane kernel, which the library itself does not choose, stays covered.
The two compilations may fuse a product into a different fma, so they agree
to rounding, not bit for bit: f64 rollouts within 1e-9, and one step's
accelerations from a late state within 1e-12 (f64) and 1e-5 (f32) relative.
The oracle comparisons of configs 1 and 2 at 200 and 256 worlds
(test_gpu_parity.py, test_gpu_divergence.py) run split-lane kernels in f64
and, for config 1, in f32."""
import os

import numpy as np
import pytest

from phyz_amd import workloads as W
from phyz_amd.sim import from_workload
from tests.helpers import as_precision, rel_err_rows

pytestmark = pytest.mark.gpu


def _sim(w, prec, n, lanes):
    os.environ["PHZ_LANES"] = str(lanes)
    try:
        sim = from_workload(w, prec, nworld=n)
        sim.compile()
    finally:
        os.environ.pop("PHZ_LANES", None)
    return sim


@pytest.mark.parametrize("cfg,n,lanes", [(1, 4096, 2), (1, 100, 2), (2, 1024, 4), (2, 70, 4)])
@pytest.mark.parametrize("prec", ["f64", "f32"])
def test_split_lanes_match_one_lane(cfg, n, lanes, prec):
    w = W.config(cfg)
    steps = 500 if cfg == 1 else 200
    split, one = _sim(w, prec, n, lanes), _sim(w, prec, n, 1)
    assert (split.kernel_info()["lanes_per_world"], one.kernel_info()["lanes_per_world"]) == (lanes, 1)
    q, v, c, tg = w.initial_state(n)
    q, v, c = (as_precision(a, prec) for a in (q, v, c))
    outs = []
    for sim in (split, one):
        sim.load_states(q, v, c)
        if tg is not None:
            sim.set_position_targets(as_precision(tg, prec))
        sim.step_many(steps)
        outs.append(sim.readback_states())
    d = max(np.abs(outs[0][0] - outs[1][0]).max(), np.abs(outs[0][1] - outs[1][1]).max())
    # One step of both kernels from the one-lane kernel's late state.
    ql, vl = (as_precision(a, prec) for a in outs[1])
    qdd = []
    for sim in (split, one):
        sim.load_states(ql, vl, c)
        sim.step()
        qdd.append(sim.readback_qdd())
    e = rel_err_rows(qdd[0], qdd[1]).max()
    print(f"cfg {cfg} {w.name} {prec}, {n} worlds, {lanes} lanes: {steps}-step state difference {d:.3e}, "
          f"late-state qdd rel difference {e:.3e}", flush=True)
    assert e <= (1e-12 if prec == "f64" else 1e-5)
    if prec == "f64":
        assert d <= 1e-9

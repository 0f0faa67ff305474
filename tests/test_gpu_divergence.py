"""500-step f64 state divergence of the device against the oracle, over the
worlds the oracle itself shows to be non-chaotic on that horizon.

Bound: max(|q_gpu - q_cpu|_inf, |v_gpu - v_cpu|_inf) <= 1e-8 after 500 steps,
the maximum over every non-chaotic world. A world is non-chaotic when two
oracle rollouts, one from its state and one with every coordinate of q moved
one ulp, stay within 1e-10 of each other over the same 500 steps: the
reference's one-ulp calibration and its bound for separation that is not a bug
(crates/phyz/src/determinism.rs:333-382, crates/phyz/tests/determinism.rs:
472-531). Both rollouts replay the workload's control stream, so the classifier
sees the same torques the device applied.
"""
import numpy as np
import pytest

from oracle.oracle import one_ulp_divergence
from phyz_amd import workloads as W
from phyz_amd.sim import from_workload
from tests.helpers import abs_err_rows, oracle_for

pytestmark = pytest.mark.gpu

STEPS = 500
NWORLD = 256
CHAOS_LINE = 1e-10  # one-ulp separation beyond which a world counts as chaotic
TOL_STATE = 1e-8


@pytest.mark.parametrize("cfg", [1, 2, 4, 5])
def test_f64_500_step_divergence(cfg):
    w = W.config(cfg)
    orc = oracle_for(w)
    q, v, c, tg = w.initial_state(NWORLD)
    print(f"cfg {cfg} {w.name}: {NWORLD} worlds x {STEPS} steps, f64", flush=True)
    _, d1, q_cpu, v_cpu = one_ulp_divergence(orc, q, v, c, STEPS, targets=tg)
    calm = np.isfinite(d1) & (d1 <= CHAOS_LINE)
    sim = from_workload(w, "f64", nworld=NWORLD)
    sim.load_states(q, v, c)
    if tg is not None:
        sim.set_position_targets(tg)
    sim.step_many(STEPS)
    q_gpu, v_gpu = sim.readback_states()
    err = np.maximum(abs_err_rows(q_gpu, q_cpu), abs_err_rows(v_gpu, v_cpu))
    print(f"  non-chaotic worlds {calm.mean():.3f} (one-ulp separation max {d1[calm].max():.2e}); "
          f"device-oracle divergence over them max {err[calm].max():.3e} median {np.median(err[calm]):.3e}; "
          f"over all worlds max {err.max():.3e}", flush=True)
    assert calm.mean() >= 0.9, "the classifier should leave most of these worlds in"
    assert np.all(np.isfinite(q_gpu[calm])) and np.all(np.isfinite(v_gpu[calm]))
    assert err[calm].max() <= TOL_STATE, f"world {np.flatnonzero(calm)[err[calm].argmax()]}"

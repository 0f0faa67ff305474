"""The oracle's chaos classifier: a rollout against the same rollout with a
one-ulp perturbation, the reference's method (crates/phyz/src/determinism.rs:
164-382, tests crates/phyz/tests/determinism.rs:381-531). The device's 500-step
f64 divergence bound is applied to the worlds this classifies as non-chaotic
(tests/test_gpu_divergence.py).
"""
import numpy as np
import pytest

from oracle.oracle import one_ulp_divergence, state_distance, ulp_offset, ulps_between
from phyz_amd import workloads as W
from tests.helpers import oracle_for

EPS = np.finfo(np.float64).eps


def test_ulp_offset_known_answers():
    """The reference's own doc examples (determinism.rs:175-199), the zero and
    extreme neighbours, and non-finite values left alone."""
    assert ulp_offset(1.0, 1) == 1.0 + EPS
    assert ulp_offset(ulp_offset(1.0, 1), -1) == 1.0
    assert ulp_offset(2.5, 0) == 2.5
    assert ulps_between(1.0, ulp_offset(1.0, 7)) == 7
    assert ulps_between(3.0, 3.0) == 0
    assert ulp_offset(0.0, 1) == 5e-324 and ulp_offset(0.0, -1) == -5e-324
    assert ulp_offset(-0.0, 1) == 5e-324
    assert ulp_offset(-1.0, 1) == -1.0 + EPS / 2  # toward +inf shrinks a negative number
    assert ulp_offset(np.finfo(np.float64).max, 1) == np.finfo(np.float64).max  # clamped to the finite range
    assert np.isnan(ulp_offset(np.nan, 1)) and ulp_offset(np.inf, -3) == np.inf
    assert ulps_between(1.0, np.inf) == (1 << 63) - 1


def test_ulp_offset_is_nextafter():
    """One step equals numpy's nextafter (the C library's) in both directions,
    across signs and magnitudes, and k steps compose."""
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.normal(size=200) * 10.0 ** rng.integers(-300, 300, size=200), [1e-310, -1e-310]])
    for x in xs:
        assert ulp_offset(x, 1) == np.nextafter(x, np.inf)
        assert ulp_offset(x, -1) == np.nextafter(x, -np.inf)
        assert ulp_offset(ulp_offset(x, 5), -2) == ulp_offset(x, 3)
        assert ulps_between(x, ulp_offset(x, -11)) == -11


def test_state_distance():
    a = np.array([[0.0, 3.0]])
    b = np.array([[4.0, 0.0]])
    assert state_distance(a, a, a, a)[0] == 0.0
    assert state_distance(a, np.zeros((1, 1)), b, np.zeros((1, 1)))[0] == 5.0
    assert state_distance(a, a, a * np.nan, a)[0] == np.inf


CASES = [1, 2, 4, 5]


def _inputs(cfg, n):
    w = W.config(cfg)
    q, v, c, tg = w.initial_state(n)
    return w, oracle_for(w), q, v, c, tg


@pytest.mark.parametrize("cfg", CASES)
def test_zero_ulp_perturbation_never_separates(cfg):
    """Identical inputs, identical outputs, bit for bit, through contact, PD and
    the replayed control stream (determinism.rs:424-447)."""
    w, orc, q, v, c, tg = _inputs(cfg, 32)
    d0, d1, _, _ = one_ulp_divergence(orc, q, v, c, 100, targets=tg, ulps=0)
    assert np.all(d0 == 0.0) and np.all(d1 == 0.0)


@pytest.mark.parametrize("cfg", CASES)
def test_one_ulp_perturbation_is_measured(cfg):
    """A one-ulp perturbation starts at the size of an ulp, is not rounded
    away, and stays finite (determinism.rs:381-422)."""
    w, orc, q, v, c, tg = _inputs(cfg, 32)
    d0, d1, qa, _ = one_ulp_divergence(orc, q, v, c, 200, targets=tg)
    assert np.all((d0 > 0.0) & (d0 < 1e-12))
    assert np.all(np.isfinite(d1)) and np.all(d1 > 0.0)


def test_classifier_separates_chaotic_worlds():
    """The offset double pendulum (the reference's fixture,
    crates/phyz-gpu/tests/cuda_vs_cpu.rs:51-63) is chaotic near the top and not
    in small oscillations: over 20 s the classifier puts the two on either side
    of the 1e-10 line the reference quotes for one-ulp chaos
    (determinism.rs:514-523). (The README pendulum of workload 1 hangs both rods
    from one pivot: two independent pendulums, never chaotic.)"""
    from oracle.oracle import Oracle
    from tests.models import double_pendulum_offset
    orc = Oracle(double_pendulum_offset())
    n = 16
    q = np.zeros((n, 2))
    q[:8] = np.array([1.5, 1.5])  # high energy: chaotic
    q[8:] = np.array([0.05, -0.03])  # small oscillations: near-integrable
    q[:, 0] += np.linspace(0.0, 1e-3, n)
    v, c = np.zeros((n, 2)), np.zeros((n, 2))
    _, d1, _, _ = one_ulp_divergence(orc, q, v, c, 20000)
    assert np.all(d1[:8] > 1e-10), d1
    assert np.all(d1[8:] < 1e-12), d1

"""The f64 oracle against the reference's own step kernels.

tests/golden/ref_step_vectors.npz holds inputs and outputs of
crates/phyz-gpu/cuda/phyz_kernels.cu (PD, penalty contact, ABA, integrate),
compiled as host C++ and run in f32 (tests/golden/make_ref_vectors.py). The
reference kernel is the f32 statement of the law this build implements, so the
oracle — f64 — must agree with it to f32 rounding: single steps within
max(2e-4, 4 x the law's own f32 rounding floor) normwise on qdd, short
trajectories within the reference's GPU-vs-CPU tolerance (1e-3,
crates/phyz-gpu/tests/cuda_vs_cpu.rs:246-317).
"""
import os

import numpy as np
import pytest

from oracle.oracle import Oracle
from tests import ref_host
from tests.helpers import rel_err_rows

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_step_vectors.npz")


def _cases():
    z = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


Z, NAMES = _cases()


def _case(name):
    g = {k.split("/")[1]: Z[k] for k in Z.files if k.startswith(name + "/")}
    nb, nq, nv, steps = (int(x) for x in g["dims"])
    contact = None
    if g["geom"].shape[0]:
        contact = (g["geom"], float(g["contact"][0]), float(g["contact"][1]))
    pd = g["pd"] if g["pd"].shape[0] else None
    orc = Oracle(tables=(g["table"], nq, nv, g["gravity"], float(g["dt"][0])), contact=contact, pd=pd)
    return g, orc, steps


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_reference_kernels(name):
    g, orc, steps = _case(name)
    q, v, c = g["q0"].copy(), g["v0"].copy(), g["ctrl0"].copy()
    tg = g["targets"] if g["targets"].shape[1] else None
    want_contacts = g["geom"].shape[0] > 0
    qdd, rows = orc.step_batch(q, v, c, steps, targets=tg, threads=1, want_contacts=want_contacts)
    nworld = q.shape[0]
    if steps == 1:
        # Per-step: qdd against the reference's, tolerance at the f32 floor.
        floor = np.array([rel_err_rows(orc.qdd_f32(g["q0"][k], g["v0"][k], g["ctrl"][k]), qdd[k]) for k in range(nworld)])
        err = rel_err_rows(g["qdd"], qdd)
        tol = np.maximum(2e-4, 4.0 * floor)
        assert np.all(err <= tol), f"{name}: qdd err {err.max():.3e} floor {floor.max():.3e}"
        np.testing.assert_allclose(c, g["ctrl"], rtol=1e-5, atol=1e-5)
        scale = np.maximum(np.abs(g["v"]).max(), 1.0)
        assert np.abs(v - g["v"]).max() <= 4e-4 * scale * max(1.0, np.abs(qdd).max() * float(g["dt"][0]))
    else:
        # Short trajectories: the reference's own GPU-vs-CPU bound.
        assert np.abs(q - g["q"]).max() <= 1e-3
        assert np.abs(v - g["v"]).max() <= 1e-3 * max(1.0, np.abs(g["v"]).max())
    if want_contacts:
        ref_rows = g["rows"]
        touch_ref = ref_rows[:, :, 0] > 0
        touch = rows[:, :, 0] > 0
        # Near-zero penetrations may flip under f32 rounding; everything else agrees.
        deep = ref_rows[:, :, 1] > 1e-5
        assert np.array_equal(touch[deep], touch_ref[deep])
        both = touch & touch_ref
        if both.any():
            f_ref = ref_rows[:, :, 5:8][both]
            f = rows[:, :, 5:8][both]
            ferr = np.abs(f - f_ref).max(axis=-1) / np.maximum(np.abs(f_ref).max(axis=-1), 1.0)
            assert np.median(ferr) <= 1e-4 and ferr.max() <= 5e-2, f"{name}: contact force err {ferr.max():.3e}"
            np.testing.assert_allclose(rows[:, :, 4][both], ref_rows[:, :, 4][both], atol=1e-6)


@pytest.mark.skipif(not ref_host.available(), reason="oracle/_ref not built (reference tree absent)")
def test_reference_host_library_reproduces_fixture():
    """The committed vectors are what oracle/_ref computes now (fixture not stale)."""
    name = "double_pendulum_1"
    g, _, steps = _case(name)
    rs = ref_host.RefStepper(g["table"], int(g["dims"][1]), int(g["dims"][2]), g["gravity"], float(g["dt"][0]),
                             g["q0"].shape[0])
    q32, v32, c32 = (np.ascontiguousarray(g[k], dtype=np.float32) for k in ("q0", "v0", "ctrl0"))
    qdd, _, _ = rs.step(q32, v32, c32)
    np.testing.assert_array_equal(qdd.astype(np.float64), g["qdd"])

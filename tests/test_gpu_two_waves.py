"""The two-waves-per-SIMD build of a step kernel (a one-wave-per-world-group
kernel above 256 registers, in a launch with more waves than SIMDs: the ant
and the MJCF ant at 131072 worlds) runs launches of 16 steps or more; shorter
launches run the one-wave build. Both are the same build of the same source,
so the rebuild only spills registers and changes no arithmetic: a span gives
the same bits however it is split into launches. The ant's pair is its
reassociated build, so it also matches the one-wave kernel alone
(PHZ_TWO_WAVES=0) bit for bit; the MJCF ant's pair is the in-order build,
which PHZ_TWO_WAVES=0 replaces by the reassociated one. From the late state
the two-wave launches reach, one more step meets the f32 oracle bound of 1e-4
on 256 sampled worlds."""
import os

import numpy as np
import pytest

from phyz_amd import workloads as W
from phyz_amd.sim import from_workload
from tests.helpers import late_step_errors

pytestmark = pytest.mark.gpu


def _sim(w, n, one_wave):
    if one_wave:
        os.environ["PHZ_TWO_WAVES"] = "0"
    try:
        sim = from_workload(w, "f32", nworld=n)
        sim.compile()
    finally:
        os.environ.pop("PHZ_TWO_WAVES", None)
    return sim


@pytest.mark.parametrize("cfg,same_as_one_wave", [(3, True), (7, False)])
def test_two_wave_build_same_bits_and_oracle(cfg, same_as_one_wave):
    w = W.config(cfg)
    n, steps = 131072, 320
    print(f"{w.name} f32: {n} worlds, {steps} steps as one launch, as 20 launches of 16 and as 64 of 5", flush=True)
    two, one = _sim(w, n, False), _sim(w, n, True)
    i2, i1 = two.kernel_info(), one.kernel_info()
    assert i2["vgpr"] + max(i2["agpr"], 0) <= 256 and i2["scratch_bytes"] > 0
    assert i1["vgpr"] + i1["agpr"] > 256 and i1["scratch_bytes"] == 0
    q, v, c, _ = w.initial_state(n)
    rng0 = None
    outs = []
    for sim, chunk in ((two, steps), (two, 16), (two, 5), (one, steps)):
        sim.load_states(q, v, c)
        if rng0 is None:
            rng0 = sim.readback_rng()
        sim.load_rng(rng0)
        for _ in range(steps // chunk):
            sim.step_many(chunk)
        qg, vg = sim.readback_states()
        outs.append((qg, vg, sim.readback_rng()))
    for k, name in ((1, "16-step launches"), (2, "5-step launches"), (3, "one-wave kernel")):
        if k == 3 and not same_as_one_wave:
            # Another build (rounding differs): the same random stream, and the worlds stay finite.
            assert np.array_equal(outs[k][2], outs[0][2]), name
            ok = np.isfinite(outs[0][0]).all(axis=1) & np.isfinite(outs[k][0]).all(axis=1)
            assert ok.mean() > 0.99
            continue
        assert np.array_equal(outs[k][0], outs[0][0], equal_nan=True), name
        assert np.array_equal(outs[k][1], outs[0][1], equal_nan=True), name
        assert np.array_equal(outs[k][2], outs[0][2]), name
    qg, vg, _ = outs[0]
    finite = np.flatnonzero(np.isfinite(qg).all(axis=1) & np.isfinite(vg).all(axis=1))
    assert finite.size >= n // 2
    idx = finite[np.linspace(0, finite.size - 1, 256).astype(int)]
    two.load_states(q, v, c)
    two.load_rng(rng0)
    two.step_many(steps)
    e, _ = late_step_errors(w, two, "f32", idx)
    print(f"  scratch {i2['scratch_bytes']} B/lane; spans bit-identical; one more step vs oracle max {e.max():.3e} "
          f"median {np.median(e):.3e}", flush=True)
    assert e.max() <= 1e-4

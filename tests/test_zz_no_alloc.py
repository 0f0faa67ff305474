"""phz_readback_states_noalloc against phz_readback_states, through the C ABI.

The allocation-free entry point stages rows through the library's static
per-GPU scratch array; it must return exactly what the allocating readback
returns, bit for bit, on consecutive calls that reuse the array with a smaller
input the second time (so stale rows from the first call would show), in both
precisions, and refuse sizes beyond the array with a clear error.
"""
import numpy as np
import pytest

from phyz_amd import workloads as W
from phyz_amd.sim import PhzError, from_workload

pytestmark = pytest.mark.gpu


def _stepped(cfg, prec, n, steps):
    w = W.config(cfg)
    sim = from_workload(w, prec, nworld=n)
    q, v, c, tg = w.initial_state(n)
    sim.load_states(q, v, c)
    if tg is not None:
        sim.set_position_targets(tg)
    sim.step_many(steps)
    return sim


@pytest.mark.parametrize("prec", ["f64", "f32"])
def test_noalloc_readback_matches_readback_on_consecutive_calls(prec):
    # The first call fills the scratch with the 14-wide ant rows of 20000
    # worlds; the second, smaller one (7-wide chain rows of 1000 worlds) reads
    # back through the same array.
    for cfg, n in ((3, 20000), (2, 1000)):
        sim = _stepped(cfg, prec, n, 30)
        q0, v0 = sim.readback_states()
        q1, v1 = sim.readback_states_noalloc()
        print(f"cfg {cfg} {prec} {n} worlds: q {q1.shape} v {v1.shape}", flush=True)
        assert q1.shape == q0.shape and v1.shape == v0.shape
        assert np.array_equal(q1.view(np.uint64), q0.view(np.uint64))
        assert np.array_equal(v1.view(np.uint64), v0.view(np.uint64))
        assert np.isfinite(q1).all()
        sim.close()


def test_noalloc_readback_rejects_more_than_its_scratch():
    # 600000 worlds x 7 values x 8 bytes = 33.6 MB > 32 MiB.
    sim = _stepped(2, "f32", 600000, 1)
    with pytest.raises(PhzError, match="above the 33554432-byte scratch"):
        sim.readback_states_noalloc()
    q, _ = sim.readback_states()  # the allocating entry point still works
    assert np.isfinite(q).all()
    sim.close()

"""The static pivot bound (pivots_bounded in phz_host.cpp): where the host
proves from a joint's own inertia, armature and damping that no LDL pivot of
its joint-space inertia can fall below the singular test of aba.rs:210, the
kernel drops the test and the branch around the parent update (Model::piv_ok).
CPU: which joints the bound admits, read from the generated source. GPU: a
chain whose leaf joint is exactly singular (a rod turning about its own axis,
and a massless point) keeps the reference's skip, against the oracle."""
import re

import numpy as np
import pytest

from oracle.oracle import Oracle
from phyz_amd import workloads as W
from phyz_amd.model import ModelBuilder, SpatialInertia, SpatialTransform
from phyz_amd.sim import BatchSim, from_workload
from tests import host_emulation as HE
from tests.helpers import rel_err_rows


def piv_ok(sim):
    src = HE.dump_source(sim)
    m = re.search(r"piv_ok\[\d+\] = \{([^}]*)\}", src)
    return [x.strip() == "true" for x in m.group(1).split(",")]


def singular_chain(leaf: str, armature: float = 0.0):
    b = ModelBuilder().gravity([0.0, 0.0, -9.81]).dt(0.001)
    b.add_revolute_body("a", -1, SpatialTransform.identity(), SpatialInertia.rod(1.0, 0.3), axis=(0.0, 0.0, 1.0))
    b.add_revolute_body("b", 0, SpatialTransform.from_translation([0.0, -0.6, 0.0]), SpatialInertia.rod(0.7, 0.25),
                        axis=(1.0, 0.0, 0.0))
    # The leaf: a rod hanging along -Y turning about Y (its own axis: zero
    # inertia about the joint), or a massless point.
    inertia = SpatialInertia.rod(0.5, 0.2) if leaf == "rod" else SpatialInertia.point_mass(0.0, [0.0, 0.0, 0.0])
    b.add_revolute_body("c", 1, SpatialTransform.from_translation([0.0, -0.5, 0.0]), inertia, axis=(0.0, 1.0, 0.0),
                        armature=armature)
    return b.build()


@pytest.mark.parametrize("prec", ["f32", "f64"])
def test_bound_admits_the_benchmark_chains(prec):
    assert all(piv_ok(from_workload(W.config(2), prec, nworld=64, device=-1)))
    assert all(piv_ok(from_workload(W.config(1), prec, nworld=64, device=-1)))


@pytest.mark.parametrize("leaf", ["rod", "point"])
def test_bound_refuses_a_singular_joint(leaf):
    for prec in ("f32", "f64"):
        assert piv_ok(BatchSim(singular_chain(leaf), 64, prec, device=-1)) == [True, True, False]
        # Armature lifts every pivot of the leaf joint above the test.
        assert piv_ok(BatchSim(singular_chain(leaf, armature=0.01), 64, prec, device=-1)) == [True, True, True]


def test_bound_refuses_a_slide_below_and_multiwave_f64():
    b = ModelBuilder().gravity([0.0, 0.0, -9.81]).dt(0.001)
    b.add_revolute_body("a", -1, SpatialTransform.identity(), SpatialInertia.rod(1.0, 0.3))
    b.add_prismatic_body("s", 0, SpatialTransform.identity(), (1.0, 0.0, 0.0), SpatialInertia.sphere(0.5, 0.1))
    b.add_revolute_body("c", 1, SpatialTransform.identity(), SpatialInertia.rod(0.5, 0.2))
    # A slide joint inside the subtree leaves the reach of its masses unbounded.
    assert piv_ok(BatchSim(b.build(), 64, "f64", device=-1)) == [False, True, True]
    # f64 kernels of several waves keep the test (see the generator's note).
    s = from_workload(W.config(4), "f64", nworld=64, device=-1)
    flags = piv_ok(s)
    assert s.kernel_info()["block"] > 64 and not any(flags)


@pytest.mark.gpu
@pytest.mark.parametrize("prec", ["f32", "f64"])
@pytest.mark.parametrize("leaf", ["rod", "point"])
def test_singular_leaf_matches_oracle(leaf, prec):
    m = singular_chain(leaf)
    n = 64
    rng = np.random.default_rng(5)
    q = rng.uniform(-np.pi, np.pi, size=(n, 3))
    v = rng.normal(size=(n, 3))
    c = rng.normal(size=(n, 3))
    if prec == "f32":
        q, v, c = (a.astype(np.float32).astype(np.float64) for a in (q, v, c))
    s = BatchSim(m, n, prec)
    s.load_states(q, v, c)
    s.step()
    qdd = s.readback_qdd()
    want, _ = Oracle(m).step_batch(q.copy(), v.copy(), c.copy(), 1, threads=8)
    assert np.all(want[:, 2] == 0.0) and np.all(qdd[:, 2] == 0.0)  # the skipped joint
    assert rel_err_rows(qdd, want).max() <= (1e-10 if prec == "f64" else 1e-4)

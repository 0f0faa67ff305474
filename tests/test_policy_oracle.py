"""The control-loop oracle (oracle/policy_ref.py) pinned without the reference:
published SplitMix64 / xorshift64 outputs, closed forms of the observation ops,
torch's own Linear/Tanh stack for the MLP layout, scipy's normal log-density
for the log-prob, and the reference test's hand-computed COM and heading
invariance (crates/phyz-gpu/tests/cuda_vs_cpu.rs:1455-1651)."""
import math

import numpy as np
import pytest
import scipy.stats

from oracle import policy_ref as PR
from oracle.oracle import Oracle, world_seed as c_world_seed
from phyz_amd import policy as P
from tests import models as TM


def test_world_seed_is_splitmix64_published_outputs():
    """world_seed(0, w) is the (w+1)-th output of SplitMix64 seeded with 0; the
    first three published outputs of Vigna's splitmix64.c for seed 0."""
    assert PR.world_seed(0, 0) == 0xE220A8397B1DCDAF
    assert PR.world_seed(0, 1) == 0x6E789E6AA1B965F4
    assert PR.world_seed(0, 2) == 0x06C45D188009454F
    rng = np.random.default_rng(3)
    for _ in range(50):
        s, w = int(rng.integers(0, 2**63)), int(rng.integers(0, 1 << 20))
        assert PR.world_seed(s, w) == c_world_seed(s, w)


def test_xorshift64_matches_marsaglia():
    """xorshift64 with shifts (13, 7, 17) from Marsaglia's seed 88172645463325252
    (Xorshift RNGs, J. Stat. Softw. 2003): first outputs."""
    r = PR.KernelRng(88172645463325252)
    assert [r.next_u64() for _ in range(3)] == [8748534153485358512, 3040900993826735515, 3453997556048239312]


def test_normal_draws_are_standard_normal():
    r = PR.KernelRng.for_world(99, 0)
    x = np.array([r.normal() for _ in range(40000)])
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1.0) < 0.02
    assert scipy.stats.kstest(x, "norm").pvalue > 1e-3
    u = PR.KernelRng(12345)
    vals = [u.uniform() for _ in range(1000)]
    assert min(vals) >= 0.0 and max(vals) < 1.0


def test_mlp_forward_known_answer_one_hot():
    """W1 = 0.1 * [[1,2,3],[4,5,6],[7,8,9]] ([out][in]); input e0 selects its first
    COLUMN (0.1, 0.4, 0.7); a transposed layout would select (0.1, 0.2, 0.3)."""
    W1 = 0.1 * np.arange(1, 10, dtype=float)
    b1 = np.array([0.0, 0.5, -0.5])
    W2 = np.diag([1.0, 2.0, 3.0]).ravel()
    b2 = np.zeros(3)
    W3 = np.array([[1.0, 0.0, 0.0], [0.0, 0.0, 1.0]]).ravel()
    b3 = np.array([0.0, 1.0])
    w = np.concatenate([W1, b1, W2, b2, W3, b3])
    out = PR.mlp_forward(3, 3, 2, w, np.array([1.0, 0.0, 0.0]))
    h1 = np.tanh([0.1, 0.4 + 0.5, 0.7 - 0.5])
    assert out[0] == pytest.approx(math.tanh(1.0 * h1[0]), abs=1e-15)
    assert out[1] == pytest.approx(math.tanh(3.0 * h1[2]) + 1.0, abs=1e-15)


def test_mlp_forward_matches_torch_linear_stack():
    """The flat order is PyTorch's parameter order of Linear-Tanh-Linear-Tanh-Linear
    (weight [out][in], then bias, per layer). torch is imported here, not at
    module level: collecting this file for a device run would otherwise load
    torch's bundled HIP runtime and hiprtc (same sonames as the system ROCm's)
    before the library, and its kernels would be compiled by that hiprtc."""
    import torch
    torch.manual_seed(0)
    n_in, n_h, n_out = 7, 11, 3
    net = torch.nn.Sequential(torch.nn.Linear(n_in, n_h), torch.nn.Tanh(), torch.nn.Linear(n_h, n_h), torch.nn.Tanh(),
                              torch.nn.Linear(n_h, n_out)).double()
    flat = torch.nn.utils.parameters_to_vector(net.parameters()).detach().numpy()
    assert flat.size == P.PolicySpec(obs=[P.Const(0)] * n_in, hidden=n_h, act_slots=[0] * n_out, act_clamp=1).n_weights()
    x = np.random.default_rng(1).normal(size=n_in)
    want = net(torch.from_numpy(x)).detach().numpy()
    np.testing.assert_allclose(PR.mlp_forward(n_in, n_h, n_out, flat, x), want, rtol=0, atol=1e-14)


def _spec(**kw):
    base = dict(obs=[P.Const(1.0), P.Const(-0.5), P.Const(0.25)], hidden=4, act_slots=[2, 0], act_clamp=0.3,
                noise_rho=0.0, input_noise=[0.0, 0.1, 0.0], history_steps=1)
    base.update(kw)
    return P.PolicySpec(**base)


def test_policy_reference_logprob_and_targets():
    spec = _spec(act_clamp_slots=[0.05, 2.0])
    w = np.random.default_rng(2).normal(size=spec.n_weights())
    std = np.array([0.2, 0.7])
    rng = PR.KernelRng.for_world(5, 3)
    obs = np.array([1.0, -0.5, 0.25])
    z = np.zeros(2)
    base = np.array([0.1, 0.2, 0.3])
    tg = np.zeros(3)
    act, logp = PR.policy_reference(spec, w, std, rng, obs, z, base, tg)
    # obs[1] carries the recorded input noise; the others are untouched.
    assert obs[0] == 1.0 and obs[2] == 0.25 and obs[1] != -0.5
    mean = PR.mlp_forward(3, 4, 2, w, obs)
    np.testing.assert_allclose(act, mean + std * z, atol=1e-15)
    assert logp == pytest.approx(scipy.stats.norm.logpdf(act, mean, std).sum(), abs=1e-12)
    assert tg[1] == 0.2  # not actioned: base
    assert tg[2] == pytest.approx(0.3 + np.clip(act[0], -0.05, 0.05), abs=1e-15)
    assert tg[0] == pytest.approx(0.1 + np.clip(act[1], -2.0, 2.0), abs=1e-15)


def test_policy_reference_ar1_noise():
    """rho = 1 keeps z frozen (keep = 0); rho = 0.9 has a stationary unit variance."""
    spec = _spec(noise_rho=1.0, input_noise=[0.0, 0.0, 0.0])
    w = np.zeros(spec.n_weights())
    z = np.array([0.3, -1.2])
    r = PR.KernelRng(77)
    for _ in range(3):
        PR.policy_reference(spec, w, np.ones(2), r, np.ones(3), z, np.zeros(3), np.zeros(3))
    assert list(z) == [0.3, -1.2]
    spec = _spec(noise_rho=0.9, input_noise=[0.0, 0.0, 0.0])
    z = np.zeros(2)
    zs = []
    for _ in range(20000):
        PR.policy_reference(spec, w, np.ones(2), r, np.ones(3), z, np.zeros(3), np.zeros(3))
        zs.append(z[0])
    assert abs(np.var(zs[100:]) - 1.0) < 0.1


def _free_body_rows(q0_rot, pos=(0.0, 0.0, 1.0)):
    m = TM.free_base_with_limb()
    q = np.zeros(m.nq)
    q[0:3] = q0_rot
    q[3:6] = pos
    return m, PR.kinematics_rows(Oracle(m), q, np.zeros(m.nv)), q


@pytest.mark.parametrize("theta", [0.3, -1.1, 2.5])
def test_pitch_roll_yaw_of_axis_rotations(theta):
    """A free body turned by theta about world y / x / z reads pitch / roll / yaw = theta."""
    for axis, op in ((1, P.BodyPitch(0)), (0, P.BodyRoll(0)), (2, P.BodyYawError(0, 0.0))):
        w = np.zeros(3)
        w[axis] = theta
        m, rows, q = _free_body_rows(w)
        val = PR.eval_op(m, rows, q, np.zeros(m.nv), op)
        want = -theta if isinstance(op, P.BodyYawError) else theta
        assert val == pytest.approx(want, abs=1e-12)


def test_readout_rotation_is_world_to_body():
    m, rows, q = _free_body_rows([0.0, 0.0, 0.4], pos=(1.0, 2.0, 3.0))
    r = rows[0, 0:9].reshape(3, 3)
    # A world point maps into the body frame by r (p_world - origin).
    p_body = r @ (np.array([1.0 + math.cos(0.4), 2.0 + math.sin(0.4), 3.0]) - rows[0, 9:12])
    np.testing.assert_allclose(p_body, [1.0, 0.0, 0.0], atol=1e-12)
    np.testing.assert_allclose(rows[1, 9:12], [1.0 + 0.2 * math.cos(0.4), 2.0 + 0.2 * math.sin(0.4), 3.0], atol=1e-12)


def test_yaw_error_wraps_into_pi():
    m, rows, q = _free_body_rows([0.0, 0.0, 3.0])
    e = PR.eval_op(m, rows, q, np.zeros(m.nv), P.BodyYawError(0, -3.0))
    assert e == pytest.approx(-6.0 + 2 * math.pi, abs=1e-12)


def test_centre_of_mass_literal():
    """Trunk at (0, 0, 1), feet at zero angle: COM = (0.16, 0.015, 10.34) / 11."""
    m = TM.trunk_and_two_feet()
    q = np.zeros(m.nq)
    q[5] = 1.0
    rows = PR.kinematics_rows(Oracle(m), q, np.zeros(m.nv))
    np.testing.assert_allclose(PR.centre_of_mass(m, rows), [0.16 / 11, 0.015 / 11, 10.34 / 11], atol=1e-14)
    sup = [(1, [0.01, 0.0, -0.04]), (2, [0.01, 0.0, -0.04])]
    # Support mean: feet origins (0, +-0.12, 0.4) + (0.01, 0, -0.04).
    e = [PR.eval_op(m, rows, q, np.zeros(m.nv), P.ComOverSupport(sup, None, a)) for a in range(3)]
    np.testing.assert_allclose(e, [0.16 / 11 - 0.01, 0.015 / 11, 10.34 / 11 - 0.36], atol=1e-14)
    assert PR.eval_op(m, rows, q, np.zeros(m.nv), P.ComOverSupport([], 0, 0)) == 0.0


def test_heading_frame_is_yaw_invariant():
    """cuda_vs_cpu.rs:1590-1628: heading-relative COM-over-support entries do not
    move under a pure yaw of the whole rig; the world-frame entry does."""
    m = TM.trunk_and_two_feet()
    sup = [(1, [0.01, 0.0, -0.04]), (2, [0.01, 0.0, -0.04])]
    ops = [P.ComOverSupport(sup, 0, a) for a in range(3)] + [P.ComOverSupport(sup, None, 0)]
    q0 = np.zeros(m.nq)
    q0[5] = 1.0
    q0[6], q0[7] = 0.2, -0.1
    q1 = q0.copy()
    q1[2] = math.pi / 2
    orc = Oracle(m)
    r0 = PR.observe_reference(m, orc, q0, np.zeros(m.nv), ops)
    r1 = PR.observe_reference(m, orc, q1, np.zeros(m.nv), ops)
    np.testing.assert_allclose(r0[:3], r1[:3], atol=1e-12)
    assert abs(r0[3] - r1[3]) > 1e-6


def test_batched_forms_follow_the_per_world_functions():
    """The world-batched observation, RNG and policy (the control-loop CPU
    baseline's forms) against the per-world functions, world by world, over
    three control steps of the ant control workload with its PD physics in
    between: RNG states bit for bit, everything else to 1e-12 (the batched
    products and numpy's log/cos round differently)."""
    from phyz_amd import workloads as W
    from phyz_amd.model import pack_geometries, pack_pd_dofs
    cl = W.control_loop(hidden=32)
    m = cl.base.model
    g, _ = pack_geometries(m, cl.base.contact.stiffness, cl.base.contact.damping)
    orc = Oracle(m, contact=(g, cl.base.contact.ground_height, cl.base.contact.friction), pd=pack_pd_dofs(cl.pd))
    nw = 12
    q, v, c, _ = cl.base.initial_state(nw)
    rng = np.random.default_rng(5)
    q[:, 6:] += rng.uniform(-0.3, 0.3, size=(nw, m.nq - 6))
    v += rng.uniform(-0.5, 0.5, size=v.shape)
    base = cl.base_targets(nw)
    # Every op kind, including the world-frame COM entry, a constant and an empty support.
    feet = [(2 + 2 * k, [0.0, 0.0, 0.0]) for k in range(4)]
    extra = [P.Const(0.25), P.BodyPos(0, 2), P.BodyPos(3, 1), P.ComOverSupport(feet, None, 2),
             P.ComOverSupport(feet, 0, 2), P.ComOverSupport([], 0, 0), P.BodyYawError(0, 3.0)]
    ops = list(cl.spec.obs) + extra
    rows_b = PR.kinematics_rows_batch(orc, q, v, threads=3)
    ob = PR.observe_batch(m, orc, q, v, ops, threads=2)
    for w in range(nw):
        np.testing.assert_array_equal(rows_b[w], PR.kinematics_rows(orc, q[w], v[w]))
        np.testing.assert_allclose(ob[w], PR.observe_reference(m, orc, q[w], v[w], ops), rtol=0, atol=1e-12)
    rngs = [PR.KernelRng.for_world(cl.seed, w) for w in range(nw)]
    brng = PR.BatchRng.for_worlds(cl.seed, range(nw))
    z1, zb = np.zeros((nw, cl.spec.n_out())), np.zeros((nw, cl.spec.n_out()))
    t1, tb = np.zeros((nw, len(cl.pd))), np.zeros((nw, len(cl.pd)))
    qb, vb, cb = q.copy(), v.copy(), c.copy()
    for step in range(3):
        obs_b = PR.observe_batch(m, orc, qb, vb, cl.spec.obs, threads=2)
        act_b, lp_b = PR.policy_batch(cl.spec, cl.weights, cl.std, brng, obs_b, zb, base, tb)
        for w in range(nw):
            o = np.array(PR.observe_reference(m, orc, q[w], v[w], cl.spec.obs))
            a, lp = PR.policy_reference(cl.spec, cl.weights, cl.std, rngs[w], o, z1[w], base[w], t1[w])
            assert int(brng.state[w]) == rngs[w].state, (step, w)
            np.testing.assert_allclose(obs_b[w], o, rtol=0, atol=1e-12)
            np.testing.assert_allclose(act_b[w], a, rtol=0, atol=1e-12)
            assert lp_b[w] == pytest.approx(lp, abs=1e-11)
        np.testing.assert_allclose(zb, z1, rtol=0, atol=1e-12)
        np.testing.assert_allclose(tb, t1, rtol=0, atol=1e-12)
        orc.step_batch(q, v, c, cl.control_every, targets=t1, threads=1)
        orc.step_batch(qb, vb, cb, cl.control_every, targets=tb, threads=4)
        np.testing.assert_allclose(qb, q, rtol=0, atol=1e-9)
    # The states really moved and the policy acted on them.
    assert np.abs(t1 - base).max() > 1e-3


def test_batch_rng_draws_match_kernel_rng():
    """BatchRng's u64 words, uniforms and normals against KernelRng per world."""
    worlds = [0, 1, 7, 1000, 123456]
    b = PR.BatchRng.for_worlds(42, worlds)
    ks = [PR.KernelRng.for_world(42, w) for w in worlds]
    for _ in range(5):
        assert [int(x) for x in b.next_u64()] == [k.next_u64() for k in ks]
        np.testing.assert_array_equal(b.uniform(), [k.uniform() for k in ks])
        np.testing.assert_allclose(b.normal(), [k.normal() for k in ks], rtol=1e-15, atol=1e-15)

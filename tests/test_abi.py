"""C ABI and host logic, without a GPU.

The library loads, exports every symbol include/phyz_amd.h declares, rejects
the inputs the reference rejects with the reference's messages
(crates/phyz-gpu/src/cuda/mod.rs:498-510, 573-597, 765-796, 988-997;
crates/phyz-gpu/src/layout.rs:281-311), and compiles model-specialised kernels
on a host-only sim (device ordinal -1). Packing follows layout.rs slot for slot.
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

from phyz_amd import _lib
from phyz_amd import workloads as W
from phyz_amd.model import (BODY_STRIDE, FREE, Geometry, Joint, ModelBuilder, PdDof, SpatialInertia,
                            SpatialTransform, pack_bodies, pack_geometries, pack_pd_dofs, rotation_axis_angle)
from phyz_amd.sim import BatchSim, PhzError
from tests import models as TM

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "phyz_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(phz_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = C.CDLL(_lib.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 25
    for s in syms:
        assert hasattr(L, s), f"{s} declared in include/phyz_amd.h but not exported"
    assert set(syms) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def host_sim(model, n=8, prec="f32"):
    return BatchSim(model, n, prec, device=-1)


def test_rejects_oversized_and_malformed_models():
    b = ModelBuilder()
    for i in range(33):
        b.add_revolute_body(f"l{i}", i - 1, SpatialTransform.identity(), SpatialInertia.sphere(1.0, 0.1))
    with pytest.raises(PhzError, match="33 bodies but the kernels hold at most 32"):
        host_sim(b.build())
    m = TM.double_pendulum_offset()
    t = pack_bodies(m)
    L = _lib.load()
    g = np.asarray(m.gravity, dtype=np.float64)
    h = C.c_void_p()
    assert L.phz_sim_create(t.ctypes.data_as(_lib.dp), 2, 2, 3, g.ctypes.data_as(_lib.dp), 0.001, 4, 0, -1, C.byref(h)) != 0
    assert "nq == nv" in L.phz_last_error(None).decode()
    bad = t.copy()
    bad[1, 0] = 1.0  # body 1 its own parent
    assert L.phz_sim_create(bad.ctypes.data_as(_lib.dp), 2, 2, 2, g.ctypes.data_as(_lib.dp), 0.001, 4, 0, -1, C.byref(h)) != 0
    assert "topological" in L.phz_last_error(None).decode()
    bad = t.copy()
    bad[0, 4] = np.nan
    assert L.phz_sim_create(bad.ctypes.data_as(_lib.dp), 2, 2, 2, g.ctypes.data_as(_lib.dp), 0.001, 4, 0, -1, C.byref(h)) != 0
    bad = t.copy()
    bad[1, 2] = 5.0  # q offset past nq
    assert L.phz_sim_create(bad.ctypes.data_as(_lib.dp), 2, 2, 2, g.ctypes.data_as(_lib.dp), 0.001, 4, 0, -1, C.byref(h)) != 0


def test_error_paths_match_reference():
    s = host_sim(TM.double_pendulum_offset())
    with pytest.raises(PhzError, match="no body has GPU-collidable geometry"):
        s.enable_ground_contact(0.0, 1.0, 1.0, 0.5)
    with pytest.raises(PhzError, match="ground contact not enabled"):
        s.readback_contacts()
    with pytest.raises(PhzError, match="PD control not enabled"):
        s.set_position_targets(np.zeros((8, 1)))
    with pytest.raises(PhzError, match="PD pipeline needs at least one servoed DOF"):
        s.enable_pd_control([])
    with pytest.raises(PhzError, match="PD DOF out of range"):
        s.enable_pd_control([PdDof(5, 0, 1.0, 0.1, 1.0)])
    with pytest.raises(PhzError, match="shape changed"):
        s.set_model(TM.arm_6dof())
    with pytest.raises(PhzError, match="host-only"):
        s.step()
    with pytest.raises(PhzError, match="out of range"):
        s.enable_control_noise(1, 0, 0.0, 1.0, [7])


def test_step_span_preconditions_shared_by_timing():
    """step_many and time_step_many check the same preconditions before any
    launch: impulse mode needs a sweep, zero steps or worlds launch nothing
    (step_many succeeds, the timer refuses), a host-only sim never launches."""
    s = host_sim(TM.shapes()["sphere"])
    s.step_many(0)  # nothing to launch: a no-op even without a device
    with pytest.raises(PhzError, match="at least one step"):
        s.time_step_many(0, 1)
    with pytest.raises(PhzError, match="host-only"):
        s.time_step_many(5, 1)
    s.enable_contact_impulse(0.0, 0.5, [(1e4, 100.0)])
    s.contact_sweeps = 0
    for call in (lambda: s.step_many(3), lambda: s.time_step_many(3, 2)):
        with pytest.raises(PhzError, match="at least one contact sweep"):
            call()
    s.contact_sweeps = 4
    with pytest.raises(PhzError, match="host-only"):
        s.step_many(3)
    empty = host_sim(TM.shapes()["sphere"], n=0)
    empty.step_many(3)  # zero worlds: nothing to launch
    with pytest.raises(PhzError, match="at least one world"):
        empty.time_step_many(3, 1)


def test_set_model_same_shape_and_collidable_count():
    m = TM.shapes()["sphere"]
    s = host_sim(m)
    assert s.enable_ground_contact(0.0, 1e4, 100.0, 0.5) == 1
    assert s.collidable_bodies == 1
    m2 = TM.shapes()["box"]
    s.set_model(m2)  # same shape: accepted, kernel recompiled lazily
    s.compile()


def test_host_only_sim_compiles_workload_kernels():
    """hiprtc compiles the gfx950 step kernel for every workload without a GPU."""
    for idx in W.ALL:
        w = W.config(idx)
        from phyz_amd.sim import from_workload
        s = from_workload(w, w.precisions[0], nworld=64, device=-1)
        s.compile()
        info = s.kernel_info()
        assert info["vgpr"] > 0 and info["block"] % 64 == 0 and info["scratch_bytes"] == 0


def test_pack_bodies_slots():
    """layout.rs:19-38 slot meanings."""
    rot = rotation_axis_angle([0, 0, 1], 0.3)
    m = (ModelBuilder()
         .add_body("a", -1, Joint(FREE, SpatialTransform.new(rot, [1, 2, 3]), np.zeros(3)),
                   SpatialInertia.new(2.0, [0.1, 0.2, 0.3], [[1, 0.1, 0.2], [0.1, 2, 0.3], [0.2, 0.3, 3]]))
         .add_revolute_body("b", 0, SpatialTransform.from_translation([0, 0, -1]), SpatialInertia.sphere(1, 0.1),
                            axis=(0, 1, 0), damping=0.5, stiffness=2.0, spring_ref=0.1, armature=0.01)
         .build())
    t = pack_bodies(m)
    assert t.shape == (2, BODY_STRIDE)
    assert list(t[0, :5]) == [-1, 4, 0, 0, 2.0] and list(t[1, :4]) == [0, 0, 6, 6]
    np.testing.assert_array_equal(t[0, 5:8], [0.1, 0.2, 0.3])
    np.testing.assert_array_equal(t[0, 8:14], [1, 2, 3, 0.1, 0.2, 0.3])
    np.testing.assert_array_equal(t[0, 14:23], rot.reshape(9))
    np.testing.assert_array_equal(t[0, 23:26], [1, 2, 3])
    np.testing.assert_array_equal(t[1, 26:33], [0, 1, 0, 0.5, 2.0, 0.1, 0.01])
    g, n = pack_geometries(m, 10.0, 2.0)
    assert n == 0 and g[0, 13] == 1 and g[0, 17] == 1 and g[0, 21] == 1 and g[0, 8] == 10.0 and g[0, 9] == 2.0
    pd = pack_pd_dofs([PdDof(6, 6, 30.0, 2.0, 25.0)])
    np.testing.assert_array_equal(pd[0, :5], [6, 6, 30.0, 2.0, 25.0])


@pytest.mark.parametrize("idx,nb,nv", [(1, 2, 2), (2, 7, 7), (3, 9, 14), (4, 22, 27), (5, 25, 24)])
def test_workload_shapes(idx, nb, nv):
    """Body counts and widths of the five workloads."""
    w = W.config(idx)
    assert w.model.nbodies == nb and w.model.nv == nv and w.model.nq == nv
    q, v, c, tg = w.initial_state(16)
    assert q.shape == (16, nv) and np.isfinite(q).all()
    if idx == 3:
        assert sum(1 for b in w.model.bodies if b.geometry is not None) == 4
    if idx == 4:
        assert sum(1 for b in w.model.bodies if b.geometry is not None) == 10
        assert sum(1 for b in w.model.bodies if b.joint.jtype == 0) == 21
    if idx == 5:
        assert tg.shape == (16, 24) and len(w.pd) == 24


def _limb_spec(**kw):
    from phyz_amd import policy as P
    base = dict(obs=[P.V(0)], hidden=8, act_slots=[0], act_clamp=0.5, input_noise=[0.0], history_steps=2)
    base.update(kw)
    return P.PolicySpec(**base)


def test_policy_errors_match_reference():
    """PolicySpec::validate / ObsOp::check (policy_pipeline.rs:153-183, 357-416) and
    the BatchSim guards (mod.rs:1004-1376), through the C ABI."""
    from phyz_amd import policy as P
    m = TM.free_base_with_limb()
    s = host_sim(m)
    with pytest.raises(PhzError, match="policy pass needs PD control"):
        s.enable_policy(_limb_spec())
    with pytest.raises(PhzError, match="policy pass not enabled"):
        s.set_policy_weights([0.0])
    with pytest.raises(PhzError, match="kinematics not enabled"):
        s.compute_kinematics()
    s.enable_pd_control([PdDof(6, 6, 20.0, 1.0, 10.0)])
    cases = [
        (dict(obs=[], input_noise=[]), "policy input width 0 not in 1..=128"),
        (dict(hidden=0), "policy hidden width 0 not in 1..=256"),
        (dict(hidden=257), "policy hidden width 257 not in 1..=256"),
        (dict(act_slots=[]), "policy output width 0 not in 1..=32"),
        (dict(history_steps=0), "policy history_steps must be at least 1"),
        (dict(obs=[P.QMinus(7, 0.0)]), r"observation op QMinus\(7, 0\) out of range \(nq 7, nv 7, nbodies 2\)"),
        (dict(obs=[P.V(7)]), r"observation op V\(7\) out of range"),
        (dict(obs=[P.BodyPitch(2)]), r"observation op BodyPitch\(2\) out of range"),
        (dict(obs=[P.BodyPos(1, 3)]), r"observation op BodyPos \{ body: 1, axis: 3 \} out of range"),
        (dict(obs=[P.ComOverSupport([(5, [0, 0, 0])], None, 0)]), "observation op ComOverSupport.* out of range"),
        (dict(obs=[P.ComOverSupport([(1, [0, 0, 0])], 2, 0)]), r"heading_body: Some\(2\).* out of range"),
        (dict(act_slots=[1]), "action slot 1 exceeds the 1 registered PD servos"),
    ]
    for kw, msg in cases:
        with pytest.raises(PhzError, match=msg):
            s.enable_policy(_limb_spec(**kw))
    with pytest.raises(ValueError, match="input_noise has 2 entries for 1 inputs"):
        s.enable_policy(_limb_spec(input_noise=[0.0, 0.0]))
    s.enable_policy(_limb_spec())
    with pytest.raises(PhzError, match="policy expects 97 weights, got 3"):
        s.set_policy_weights([0.0, 0.0, 0.0])
    with pytest.raises(PhzError, match="policy has 1 actions, got 2 stds"):
        s.set_policy_std([1.0, 1.0])
    with pytest.raises(PhzError, match="host-only"):
        s.run_policy(0)
    with pytest.raises(PhzError, match="state history needs at least one slot"):
        s.enable_state_history(0)
    with pytest.raises(PhzError, match="state history not enabled"):
        s.record_state(0)
    s.enable_state_history(2)
    with pytest.raises(PhzError, match="history slot 2 exceeds 2 slots"):
        s.record_state(2)


def test_host_only_sim_compiles_control_kernels():
    """The FK/observation and MFMA policy kernels compile for gfx950 without
    scratch at the largest widths the reference accepts (128 in, 256 hidden, 32 out)."""
    from phyz_amd import policy as P
    w = W.config(4)
    s = BatchSim(w.model, 64, "f32", device=-1)
    s.enable_pd_control([PdDof(6 + k, 6 + k, 20.0, 1.0, 10.0) for k in range(21)])
    obs = [P.V(i % 27) for i in range(120)] + [P.BodyPitch(0), P.BodyRoll(0), P.BodyYawError(0, 0.0), P.BodyPosZ(3),
                                                P.BodyPos(5, 1), P.QMinus(7, 0.1), P.Const(1.0),
                                                P.ComOverSupport([(9, [0, 0, -0.1]), (12, [0, 0, -0.1])], 0, 1)]
    s.enable_policy(P.PolicySpec(obs=obs, hidden=256, act_slots=[k % 21 for k in range(32)], act_clamp=0.4,
                                 input_noise=[0.01] * len(obs), history_steps=1))
    s.compile()
    for k in ("obs", "policy"):
        info = s.control_kernel_info(k)
        assert info["vgpr"] > 0 and info["scratch_bytes"] == 0, (k, info)
    assert s.control_kernel_info("policy")["worlds_per_block"] == 32

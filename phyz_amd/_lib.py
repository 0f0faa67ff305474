"""ctypes binding of libphyz_amd.so (the C ABI in include/phyz_amd.h).

The library must be built in-tree (python -m phyz_amd.build); loading fails
loudly when it is missing — there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libphyz_amd.so")

_lib = None

dp = C.POINTER(C.c_double)
u32p = C.POINTER(C.c_uint32)
u64p = C.POINTER(C.c_uint64)
i64p = C.POINTER(C.c_int64)
SIM = C.c_void_p

TRAIN = C.c_void_p


class NetDims(C.Structure):
    _fields_ = [("n_in", C.c_uint64), ("n_h", C.c_uint64), ("n_out", C.c_uint64)]


class AdamCfg(C.Structure):
    _fields_ = [("lr", C.c_double), ("beta1", C.c_double), ("beta2", C.c_double), ("epsilon", C.c_double),
                ("weight_decay", C.c_double)]


class PpoCfg(C.Structure):
    _fields_ = [("clip", C.c_double), ("entropy_coef", C.c_double), ("vdelta", C.c_double), ("minibatch", C.c_uint64),
                ("epochs", C.c_uint64), ("target_kl", C.c_double), ("kl_scale", C.c_double), ("kl_mode", C.c_int32)]


class UpdateStats(C.Structure):
    _fields_ = [("policy_loss", C.c_double), ("value_loss", C.c_double), ("kl", C.c_double),
                ("grad_steps", C.c_uint64), ("stopped_early", C.c_int32)]


fp = C.POINTER(C.c_float)

# name -> (restype, argtypes); every symbol declared in include/phyz_amd.h.
SIGNATURES = {
    "phz_sim_create": (C.c_int, [dp, C.c_uint32, C.c_uint32, C.c_uint32, dp, C.c_double, C.c_uint32, C.c_int, C.c_int,
                                 C.POINTER(C.c_void_p)]),
    "phz_sim_destroy": (None, [SIM]),
    "phz_last_error": (C.c_char_p, [SIM]),
    "phz_set_model": (C.c_int, [SIM, dp, C.c_uint32, C.c_uint32, C.c_uint32, dp, C.c_double]),
    "phz_enable_ground_contact": (C.c_int, [SIM, C.c_double, C.c_double, C.c_double, C.c_double, dp, u32p]),
    "phz_enable_ground_contact_per_body": (C.c_int, [SIM, C.c_double, C.c_double, dp, dp, u32p]),
    "phz_enable_pd_control": (C.c_int, [SIM, dp, C.c_uint32]),
    "phz_set_position_targets": (C.c_int, [SIM, dp]),
    "phz_enable_control_noise": (C.c_int, [SIM, C.c_uint64, C.c_int, C.c_double, C.c_double, u32p, C.c_uint32]),
    "phz_set_joint_terms": (C.c_int, [SIM, dp]),
    "phz_set_actuators": (C.c_int, [SIM, dp, C.c_uint32]),
    "phz_nctrl": (C.c_int, [SIM]),
    "phz_load_states": (C.c_int, [SIM, dp, dp, dp]),
    "phz_set_controls": (C.c_int, [SIM, dp]),
    "phz_step": (C.c_int, [SIM]),
    "phz_step_many": (C.c_int, [SIM, C.c_uint32]),
    "phz_set_graphs_enabled": (C.c_int, [SIM, C.c_int]),
    "phz_graphs_enabled": (C.c_int, [SIM]),
    "phz_synchronize": (C.c_int, [SIM]),
    "phz_readback_states": (C.c_int, [SIM, dp, dp]),
    "phz_readback_states_noalloc": (C.c_int, [SIM, dp, dp]),
    "phz_readback_contacts": (C.c_int, [SIM, dp]),
    "phz_readback_controls": (C.c_int, [SIM, dp]),
    "phz_readback_qdd": (C.c_int, [SIM, dp]),
    "phz_readback_rng": (C.c_int, [SIM, u64p]),
    "phz_load_rng": (C.c_int, [SIM, u64p]),
    "phz_collidable_bodies": (C.c_int, [SIM]),
    "phz_compile": (C.c_int, [SIM]),
    "phz_time_step_many": (C.c_int, [SIM, C.c_uint32, C.c_uint32, dp]),
    "phz_kernel_info": (C.c_int, [SIM, i64p]),
    "phz_lanes_per_world": (C.c_int, [SIM]),
    "phz_enable_contact_terrain": (C.c_int, [SIM, C.c_double, C.c_double, dp, dp, dp, u32p, C.c_uint32, dp, dp, u32p]),
    "phz_enable_contact_impulse": (C.c_int, [SIM, C.c_double, C.c_double, dp, dp, dp, u32p, C.c_uint32, dp, dp, dp,
                                             u32p]),
    "phz_set_heightfield": (C.c_int, [SIM, dp, dp]),
    "phz_set_contact_sweeps": (C.c_int, [SIM, C.c_uint32]),
    "phz_contact_sweeps": (C.c_int, [SIM]),
    "phz_readback_contact_state": (C.c_int, [SIM, dp, dp]),
    "phz_load_contact_state": (C.c_int, [SIM, dp, dp]),
    "phz_enable_kinematics": (C.c_int, [SIM]),
    "phz_compute_kinematics": (C.c_int, [SIM]),
    "phz_readback_kinematics": (C.c_int, [SIM, dp]),
    "phz_enable_policy": (C.c_int, [SIM, dp, C.c_uint32, dp, C.c_uint32, C.c_uint32, u32p, C.c_uint32, C.c_double, dp,
                                    C.c_double, dp, C.c_uint32]),
    "phz_set_policy_weights": (C.c_int, [SIM, dp, C.c_uint64]),
    "phz_set_policy_std": (C.c_int, [SIM, dp, C.c_uint32]),
    "phz_set_policy_base_targets": (C.c_int, [SIM, dp]),
    "phz_seed_policy": (C.c_int, [SIM, C.c_uint64]),
    "phz_run_policy": (C.c_int, [SIM, C.c_uint32]),
    "phz_readback_policy_history": (C.c_int, [SIM, C.c_uint32, C.c_uint32, dp, dp]),
    "phz_readback_targets": (C.c_int, [SIM, dp]),
    "phz_enable_state_history": (C.c_int, [SIM, C.c_uint32]),
    "phz_record_state": (C.c_int, [SIM, C.c_uint32]),
    "phz_readback_state_history": (C.c_int, [SIM, C.c_uint32, C.c_uint32, dp, dp]),
    "phz_rollout": (C.c_int, [SIM, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int]),
    "phz_time_rollout": (C.c_int, [SIM, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int, C.c_uint32, dp]),
    "phz_time_control_kernel": (C.c_int, [SIM, C.c_int, C.c_uint32, C.c_uint32, dp]),
    "phz_control_kernel_info": (C.c_int, [SIM, C.c_int, i64p]),
    "phz_train_create": (C.c_int, [NetDims, NetDims, C.c_uint64, C.c_uint64, C.c_int, C.POINTER(C.c_void_p)]),
    "phz_train_destroy": (None, [TRAIN]),
    "phz_train_last_error": (C.c_char_p, [TRAIN]),
    "phz_train_device_name": (C.c_int, [TRAIN, C.c_char_p, C.c_uint64]),
    "phz_train_param_count": (C.c_uint64, [TRAIN, C.c_int]),
    "phz_train_rows_per_tile": (C.c_uint32, [TRAIN]),
    "phz_train_set_adam": (C.c_int, [TRAIN, C.POINTER(AdamCfg), C.POINTER(AdamCfg)]),
    "phz_train_set_actor_params": (C.c_int, [TRAIN, dp, C.c_uint64]),
    "phz_train_set_critic_params": (C.c_int, [TRAIN, dp, C.c_uint64]),
    "phz_train_actor_params": (C.c_int, [TRAIN, dp, C.c_uint64]),
    "phz_train_critic_params": (C.c_int, [TRAIN, dp, C.c_uint64]),
    "phz_train_upload_batch": (C.c_int, [TRAIN, C.c_uint64, fp, C.c_uint64, fp, C.c_uint64, fp, C.c_uint64, fp,
                                         C.c_uint64, fp, C.c_uint64, fp, C.c_uint64]),
    "phz_train_update": (C.c_int, [TRAIN, C.POINTER(u32p), u64p, C.c_uint64, C.POINTER(PpoCfg),
                                   C.POINTER(UpdateStats)]),
    "phz_train_time_update": (C.c_int, [TRAIN, C.POINTER(u32p), u64p, C.c_uint64, C.POINTER(PpoCfg),
                                        C.POINTER(UpdateStats), dp, u64p]),
}


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run `python -m phyz_amd.build` (hipcc, gfx950)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib

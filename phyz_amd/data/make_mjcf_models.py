"""Write phyz_amd/data/mjcf_models.npz: the reference's benchmark MJCF models
(models/ant.xml, humanoid.xml, shadow_hand.xml, half_cheetah.xml,
simple_arm.xml under the reference tree) as loaded by phyz_amd.mjcf, in the
packed tables the C ABI takes. The model files themselves stay in the
reference; this is the data they describe, package data that the benchmark
workloads (phyz_amd.workloads.mjcf_model) and the GPU tests load where the
reference tree is absent. tests/test_mjcf.py checks that the loader still
produces exactly these tables.

    python phyz_amd/data/make_mjcf_models.py [reference root]
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from phyz_amd.mjcf import MjcfLoader  # noqa: E402
from phyz_amd.model import pack_actuators, pack_bodies, pack_geometries, pack_joint_terms  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mjcf_models.npz")
MODELS = ("ant", "humanoid", "shadow_hand", "half_cheetah", "simple_arm")


def tables(model):
    return {
        "body": pack_bodies(model),
        "geom": pack_geometries(model)[0],
        "joint_terms": pack_joint_terms(model),
        "actuators": pack_actuators(model),
        "gravity": np.asarray(model.gravity, dtype=np.float64),
        "dims": np.array([model.nq, model.nv, model.dt], dtype=np.float64),
        "body_names": np.array([b.name for b in model.bodies], dtype=np.str_),
        "joint_names": np.array([b.joint.name for b in model.bodies], dtype=np.str_),
        "actuator_names": np.array([a.name for a in model.actuators] or [""], dtype=np.str_),
    }


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    out = {}
    for name in MODELS:
        m = MjcfLoader.from_file(os.path.join(ref, "models", f"{name}.xml")).build_model()
        for k, v in tables(m).items():
            out[f"{name}/{k}"] = v
        print(name, m.nbodies, m.nq, m.nv, m.nu())
    np.savez_compressed(OUT, **out)
    print("wrote", OUT)


if __name__ == "__main__":
    main()

"""Build libphyz_amd.so in-tree (hipcc, gfx950).

    python -m phyz_amd.build

1. Embed csrc/phz_device.h and csrc/phz_control.h as raw strings
   (csrc/phz_device_src.inc, csrc/phz_control_src.inc) so the library can hand
   them to hiprtc with each model's constants.
2. Compile the host library (csrc/phz_host.cpp), the ahead-of-time layout
   kernels (csrc/phz_io.hip) and the PPO update pass (csrc/phz_train.hip) for
   gfx950 and link them with hiprtc.

Packed FP32 instructions are disabled in every device compile.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libphyz_amd.so")
ARCH = "gfx950"
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm 7 expected under /opt/rocm)")


def _embed(header: str, inc: str, delim: str) -> str:
    src = open(os.path.join(CSRC, header)).read()
    assert f"){delim}\"" not in src
    out = os.path.join(CSRC, inc)
    text = f'R"{delim}({src}){delim}"\n'
    if not os.path.exists(out) or open(out).read() != text:
        with open(out, "w") as f:
            f.write(text)
    return out


def embed_device_source() -> None:
    _embed("phz_device.h", "phz_device_src.inc", "PHZ_DEVICE_SRC")
    _embed("phz_control.h", "phz_control_src.inc", "PHZ_CONTROL_SRC")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}):\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build(verbose: bool = False) -> str:
    embed_device_source()
    cc = hipcc()
    bdir = os.path.join(HERE, "_build")
    os.makedirs(bdir, exist_ok=True)
    io_obj = os.path.join(bdir, "phz_io.o")
    host_obj = os.path.join(bdir, "phz_host.o")
    train_obj = os.path.join(bdir, "phz_train.o")
    _run([cc, "-x", "hip", f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", *NO_PACKED_FP32, "-c",
          os.path.join(CSRC, "phz_io.hip"), "-o", io_obj], verbose)
    _run([cc, "-x", "hip", f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", *NO_PACKED_FP32, "-c",
          os.path.join(CSRC, "phz_train.hip"), "-o", train_obj], verbose)
    _run([cc, "-x", "c++", "-O2", "-fPIC", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-c",
          os.path.join(CSRC, "phz_host.cpp"), "-o", host_obj], verbose)
    tmp = LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", io_obj, train_obj, host_obj, "-o", tmp,
          "-L/opt/rocm/lib", "-lhiprtc", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

"""The step kernel run on the CPU: a workgroup emulation of the generated
multi-wave source — TEST INFRASTRUCTURE ONLY.

The library generates a model-specialised HIP source for each sim and
compiles it with hiprtc for gfx950. This module takes that same source
(PHZ_DUMP_SOURCE), rewrites the few device-only constructs for the host, and
compiles it with clang++ together with a driver that runs one workgroup of G
waves as G host threads:

  - each thread is one wave and runs the kernel for one lane at a time (the
    lanes of a partitioned kernel never exchange data: a lane's LDS slots are
    its own column, lds[slot * 64 + lane]);
  - __syncthreads() is a pthread barrier over the G threads;
  - the workgroup's LDS is one heap array of exactly the kernel's size, so
    AddressSanitizer bounds every slot access (the f64 sine and log tables,
    namespace-scope __shared__ arrays that wave 0 fills before a barrier, one
    entry pair per lane, are plain globals that the emulated lane fills
    whole);
  - the AMDGPU builtins become their host meanings (v_sin_f32 / v_cos_f32
    take turns, v_rcp / v_rsq are reciprocals, v_cvt_i32 saturates and maps
    NaN to 0).

build_device_ir runs, through the same driver, the device compiler's own
optimised IR of the source (compiled for gfx950, rewritten for x86-64): the
IR that reaches the AMDGPU back end, checked against the oracle.

Builds: "asan" (AddressSanitizer + UndefinedBehaviorSanitizer, every
automatic variable initialised to a NaN pattern so that a read before a
write poisons the result, and the FP traps for invalid operations and
division by zero armed), "tsan" (ThreadSanitizer: the waves' LDS exchange
checked as the multi-threaded protocol it is), and "finite" (-O3 under the
device kernels' own floating-point flags). Plans that the planner refuses on
a device (a merged f64 plan, a three-wave plan) are generated on a host-only
sim with PHZ_HOST_LIFT_GUARDS=1.
"""
from __future__ import annotations

import hashlib
import os
import re
import subprocess
import tempfile
from typing import Dict, Optional

import numpy as np

CLANG = "/opt/rocm/lib/llvm/bin/clang++"
HERE = os.path.dirname(os.path.abspath(__file__))
CACHE = os.path.join(tempfile.gettempdir(), "phz_host_emulation")

PRELUDE = r"""
#include <cmath>
#include <cstdint>
#include <cstring>
#define __HIPCC_RTC__ 1
#define __device__
#define __global__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__
struct EmuDim3 { unsigned x = 0, y = 0, z = 0; };
thread_local EmuDim3 threadIdx, blockIdx;
extern "C" void emu_syncthreads();
#define __syncthreads() emu_syncthreads()
extern void* emu_lds_base;
static inline float emu_amdgcn_rcpf(float x) { return 1.0f / x; }
static inline double emu_amdgcn_rcp(double x) { return 1.0 / x; }
static inline float emu_amdgcn_rsqf(float x) { return 1.0f / std::sqrt(x); }
static inline double emu_amdgcn_rsq(double x) { return 1.0 / std::sqrt(x); }
static inline float emu_amdgcn_sqrtf(float x) { return std::sqrt(x); }
static inline float emu_amdgcn_sinf(float t) { return (float)std::sin(6.283185307179586 * (double)t); }
static inline float emu_amdgcn_cosf(float t) { return (float)std::cos(6.283185307179586 * (double)t); }
static inline float emu_amdgcn_logf(float x) { return std::log2(x); }
static inline double emu_amdgcn_frexp_mant(double x) { int e; return std::frexp(x, &e); }
static inline int emu_amdgcn_frexp_exp(double x) { int e; std::frexp(x, &e); return e; }
static inline int emu_amdgcn_readfirstlane(int x) { return x; }
static inline int emu_amdgcn_mov_dpp(int x, int, int, int, bool) { return x; }
template <class F> static inline int emu_cvt_sat(F x) {
  if (!(x == x)) return 0;
  if (x >= (F)2147483647.0) return 2147483647;
  if (x <= (F)-2147483648.0) return (-2147483647 - 1);
  return (int)x;
}
"""

DRIVER = r"""
#include <pthread.h>
#include <cfenv>
#include <cstdio>
#include <cstdlib>
#include <vector>

void* emu_lds_base = nullptr;
static pthread_barrier_t emu_bar;
extern "C" void emu_syncthreads() { pthread_barrier_wait(&emu_bar); }

struct EmuJob { phz::StepArgs a; int g, lane, block; };
static void* emu_wave(void* p) {
  EmuJob* j = (EmuJob*)p;
  threadIdx.x = (unsigned)(j->g * 64 + j->lane);
  blockIdx.x = (unsigned)j->block;
  phz_step(j->a);
  return nullptr;
}

template <class T> static std::vector<T> slurp(FILE* f, size_t n) {
  std::vector<T> v(n ? n : 1);
  if (n && fread(v.data(), sizeof(T), n, f) != n) { fprintf(stderr, "short read\n"); exit(3); }
  return v;
}

int main(int argc, char** argv) {
  // argv: input file, output file, waves per workgroup, trap flag
  FILE* f = fopen(argv[1], "rb");
  long hdr[10];
  if (fread(hdr, sizeof(long), 10, f) != 10) return 3;
  const int nworld = (int)hdr[0], stride = (int)hdr[1], nsteps = (int)hdr[2], nq = (int)hdr[3], nv = (int)hdr[4];
  const int nctrl = (int)hdr[5], nb = (int)hdr[6], npd = (int)hdr[7], launches = (int)hdr[8];
  const int G = atoi(argv[3]);
  typedef EMU_T T;
  std::vector<T> q = slurp<T>(f, (size_t)nq * stride), v = slurp<T>(f, (size_t)nv * stride);
  std::vector<T> ctrl = slurp<T>(f, (size_t)nctrl * stride), tg = slurp<T>(f, (size_t)npd * stride);
  std::vector<unsigned long long> rng = slurp<unsigned long long>(f, (size_t)stride);
  const int hf_nx = (int)hdr[9] & 0xffff, hf_ny = (int)(hdr[9] >> 16);
  std::vector<double> hf_hdr = slurp<double>(f, 4);  // origin x, y, z, cell
  std::vector<double> hf = slurp<double>(f, (size_t)hf_nx * hf_ny);
  fclose(f);
  std::vector<T> qdd((size_t)nv * stride), rows((size_t)nb * 8 * stride), ext((size_t)nb * 6 * stride);
  std::vector<T> imp((size_t)nb * 48 * stride);
  if (atoi(argv[4])) feenableexcept(FE_INVALID | FE_DIVBYZERO);
  const int nblocks = stride / 64;
  const size_t lds_n = (size_t)(Model::NSLOT > 0 ? Model::NSLOT : 1) * 64;
  for (int l = 0; l < launches; l++) {
    for (int b = 0; b < nblocks; b++) {
      // Every slot starts as a signalling NaN: with the FP traps armed, a
      // slot read before any wave wrote it traps at its first use.
      T* lds = new T[lds_n];
      {
        const unsigned long long s64 = 0x7FF4000000000000ull;
        const unsigned s32 = 0x7FA00000u;
        for (size_t k = 0; k < lds_n; k++) {
          if (sizeof(T) == 8) memcpy(&lds[k], &s64, 8);
          else memcpy(&lds[k], &s32, 4);
        }
      }
      emu_lds_base = lds;
      for (int lane = 0; lane < 64; lane++) {
        pthread_barrier_init(&emu_bar, nullptr, (unsigned)G);
        std::vector<pthread_t> th(G);
        std::vector<EmuJob> jobs(G);
        for (int g = 0; g < G; g++) {
          phz::StepArgs a{};
          a.q = q.data(); a.v = v.data(); a.ctrl = ctrl.data(); a.qdd = qdd.data(); a.targets = tg.data();
          a.rng = rng.data(); a.contact_rows = rows.data(); a.ext = ext.data(); a.imp = imp.data(); a.hf = hf.data();
          a.hf_ox = hf_hdr[0]; a.hf_oy = hf_hdr[1]; a.hf_oz = hf_hdr[2]; a.hf_cell = hf_hdr[3];
          a.hf_nx = hf_nx; a.hf_ny = hf_ny;
          a.nworld = nworld; a.stride = stride; a.nsteps = nsteps; a.write_contacts = 1;
          jobs[g] = EmuJob{a, g, lane, b};
          pthread_create(&th[g], nullptr, emu_wave, &jobs[g]);
        }
        for (int g = 0; g < G; g++) pthread_join(th[g], nullptr);
        pthread_barrier_destroy(&emu_bar);
      }
      delete[] lds;
    }
  }
  FILE* o = fopen(argv[2], "wb");
  fwrite(q.data(), sizeof(T), (size_t)nq * stride, o);
  fwrite(v.data(), sizeof(T), (size_t)nv * stride, o);
  fwrite(qdd.data(), sizeof(T), (size_t)nv * stride, o);
  fwrite(rng.data(), 8, (size_t)stride, o);
  fclose(o);
  return 0;
}
"""

FLAGS = {
    "asan": ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
             "-ftrivial-auto-var-init=pattern"],
    "tsan": ["-O1", "-g", "-fsanitize=thread"],
    # The device kernels' own floating-point contract (finite values only,
    # signed zeros ignored, the spatial algebra reassociable): a source that
    # breaks the contract (an inf or NaN on any path) can compute wrong
    # values here too, while the builds above trap where it happens.
    "finite": ["-O3", "-ffinite-math-only", "-fno-signed-zeros", "-DPHZ_REASSOC=1"],
}


def host_device_code(s: str) -> str:
    """Device source with its AMDGPU builtins and inline asm given host meanings."""
    s = s.replace("#pragma once", "")
    s = s.replace("__builtin_amdgcn_", "emu_amdgcn_")
    s = s.replace('asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(x));', "r = emu_cvt_sat(x);")
    s = s.replace('asm("v_cvt_i32_f64 %0, %1" : "=v"(r) : "v"(x));', "r = emu_cvt_sat(x);")
    return s.replace('"+s"', '"+r"').replace('"+v"', '"+x"')


def host_source(device_src: str, prec: str) -> str:
    """The generated kernel source, rewritten for the host."""
    s = host_device_code(device_src)
    t = "double" if prec == "f64" else "float"
    s, n = re.subn(r"__shared__\s+" + t + r"\s+lds\[[^;]*\];", f"{t}* lds = ({t}*)emu_lds_base;", s)
    assert n == 1, "the kernel's LDS declaration was not found"
    # One emulated lane at a time: the filling lane writes the whole table.
    fill = ("phz_sc_tab[lane] = k[lane];\n  phz_sc_tab[64 + lane] = k[64 + lane];\n"
            "  phz_log_tab[lane] = lg[lane];\n  phz_log_tab[64 + lane] = lg[64 + lane];")
    assert fill in s, "the f64 tables' fill was not found"
    s = s.replace(fill, "for (int e = 0; e < 128; e++) { phz_sc_tab[e] = k[e]; phz_log_tab[e] = lg[e]; }")
    assert "asm(" not in s, "an unhandled inline asm block is left in the source"
    return PRELUDE + s + "\n#define EMU_T " + t + "\n" + DRIVER


def build(device_src: str, prec: str, mode: str) -> str:
    """Compile (cached by content) and return the executable's path."""
    src = host_source(device_src, prec)
    key = hashlib.sha1((src + mode + " ".join(FLAGS[mode])).encode()).hexdigest()[:16]
    os.makedirs(CACHE, exist_ok=True)
    exe = os.path.join(CACHE, f"emu_{key}_{mode}")
    if not os.path.exists(exe):
        cpp = exe + ".cpp"
        with open(cpp, "w") as f:
            f.write(src)
        r = subprocess.run([CLANG, "-x", "c++", "-std=c++17", *FLAGS[mode], cpp, "-o", exe + ".tmp", "-lpthread"],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"host build failed:\n{r.stderr[-4000:]}")
        os.replace(exe + ".tmp", exe)
    return exe


def dump_source(sim) -> str:
    """The source the library generates for `sim` (a host-only sim)."""
    path = os.path.join(tempfile.mkdtemp(prefix="phz_src_"), "step.hip")
    os.environ["PHZ_DUMP_SOURCE"] = path
    try:
        sim.compile()
    finally:
        os.environ.pop("PHZ_DUMP_SOURCE", None)
    return open(path).read()


def run(exe: str, prec: str, waves: int, q: np.ndarray, v: np.ndarray, ctrl: np.ndarray, rng: np.ndarray,
        nsteps: int, launches: int = 1, nb: int = 1, targets: Optional[np.ndarray] = None, trap: bool = True,
        env: Optional[Dict[str, str]] = None, heightfield=None):
    """Run `launches` launches of `nsteps` steps for world-major (q, v, ctrl)
    and the per-world RNG states (heightfield: a phyz_amd.model.Heightfield
    the model's contact was enabled with). Returns (q, v, qdd, rng, stderr)."""
    dt = np.float64 if prec == "f64" else np.float32
    nworld = q.shape[0]
    stride = (nworld + 63) // 64 * 64

    def soa(a, width):
        out = np.zeros((width, stride), dtype=dt)
        if width:
            out[:, :nworld] = np.asarray(a, dtype=np.float64).T
        return out

    nq, nv, nctrl = q.shape[1], v.shape[1], ctrl.shape[1]
    npd = 0 if targets is None else targets.shape[1]
    r = np.zeros(stride, dtype=np.uint64)
    r[:nworld] = rng
    with tempfile.TemporaryDirectory() as d:
        inp, out = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
        hf = heightfield
        hfw = 0 if hf is None else (hf.nx | (hf.ny << 16))
        with open(inp, "wb") as f:
            f.write(np.array([nworld, stride, nsteps, nq, nv, nctrl, nb, npd, launches, hfw], dtype=np.int64).tobytes())
            for a, w in ((q, nq), (v, nv), (ctrl, nctrl), (targets, npd)):
                f.write(soa(a, w).tobytes() if w else b"")
            f.write(r.tobytes())
            f.write(np.array([0.0, 0.0, 0.0, 1.0] if hf is None else [*hf.origin, hf.cell], dtype=np.float64).tobytes())
            if hf is not None:
                f.write(hf.nodes().tobytes())
        e = dict(os.environ)
        e.update(env or {})
        p = subprocess.run([exe, inp, out, str(waves), "1" if trap else "0"], capture_output=True, text=True, env=e)
        if p.returncode != 0:
            raise RuntimeError(f"host emulation failed ({p.returncode}):\n{p.stderr[-6000:]}")
        raw = open(out, "rb").read()
    n1, n2 = nq * stride, nv * stride
    arr = np.frombuffer(raw[: (n1 + 2 * n2) * np.dtype(dt).itemsize], dtype=dt)
    qo = arr[:n1].reshape(nq, stride)[:, :nworld].T.astype(np.float64)
    vo = arr[n1:n1 + n2].reshape(nv, stride)[:, :nworld].T.astype(np.float64)
    qddo = arr[n1 + n2:].reshape(nv, stride)[:, :nworld].T.astype(np.float64)
    ro = np.frombuffer(raw[(n1 + 2 * n2) * np.dtype(dt).itemsize:], dtype=np.uint64)[:nworld]
    return qo, vo, qddo, ro, p.stderr


# ── The device compiler's own optimised IR, run on the host ─────────────────
# The step source compiled for gfx950 to LLVM IR (the optimisation pipeline's
# output under the library's flags, before the AMDGPU back end), rewritten for
# x86-64 and linked into the driver above. It tells whether a device failure
# is already in the IR the AMDGPU pipeline produced: if this run matches the
# oracle, every IR pass (SROA, instcombine, the target-aware ones) kept the
# source's meaning, and the difference arises in the back end or on the device.
# The rewrite: address spaces dropped (every pointer is a plain host pointer;
# the kernel argument block is passed by pointer), the f64 tables made plain
# globals that the driver fills, and the few AMDGPU intrinsics and inline asm
# statements of the step kernel given host meanings (work-item ids, uniform
# reads, the barrier, v_rcp/v_rsq as exact reciprocals, the saturating
# conversions; the empty asm statements that pin a value in a register stay
# empty asm statements on x86 registers).
X86_LAYOUT = 'e-m:e-p270:32:32-p271:32:32-p272:64:64-i64:64-i128:128-f80:128-n8:16:32:64-S128'
DEVICE_IR_FLAGS = {
    "finite": ["-O3", "-ffinite-math-only", "-fno-signed-zeros"],
    "reassoc": ["-O3", "-ffinite-math-only", "-fno-signed-zeros", "-DPHZ_REASSOC=1"],
    "ieee": ["-O3", "-fno-signed-zeros"],
}
IR_INTRINSICS = (("llvm.amdgcn.workitem.id.x", "irx_tid"), ("llvm.amdgcn.workgroup.id.x", "irx_bid"),
                 ("llvm.amdgcn.readfirstlane.i32", "irx_rfl"), ("llvm.amdgcn.s.barrier", "irx_barrier"),
                 ("llvm.amdgcn.rcp.f64", "irx_rcp"), ("llvm.amdgcn.rsq.f64", "irx_rsq"))
IR_SHIMS = r"""
extern "C" void phz_step_ir(const void*);
extern "C" double irx_sc_tab[128], irx_log_tab[128];
extern "C" unsigned irx_tid() { return threadIdx.x; }
extern "C" unsigned irx_bid() { return blockIdx.x; }
extern "C" int irx_rfl(int x) { return x; }
extern "C" void irx_barrier() { emu_syncthreads(); }
extern "C" double irx_rcp(double x) { return 1.0 / x; }
extern "C" double irx_rsq(double x) { return 1.0 / std::sqrt(x); }
extern "C" int irx_cvt_f64(double x) { return emu_cvt_sat(x); }
extern "C" int irx_cvt_f32(float x) { return emu_cvt_sat(x); }
"""


def device_ir_for_host(ir: str) -> str:
    """gfx950 IR of the step kernel rewritten for x86-64 (see above)."""
    out = []
    for line in ir.split("\n"):
        if line.startswith("target datalayout"):
            line = f'target datalayout = "{X86_LAYOUT}"'
        elif line.startswith("target triple"):
            line = 'target triple = "x86_64-unknown-linux-gnu"'
        elif line.startswith(("@__hip_cuid", "@llvm.compiler.used", "!llvm.module.flags")):
            continue
        elif line.startswith("attributes #"):
            line = re.sub(r"= \{.*\}", "= { nounwind }", line)
        out.append(line)
    ir = "\n".join(out)
    ir = re.sub(r" addrspace\(\d\)", "", ir)
    ir = re.sub(r"(%[\w.]+) = addrspacecast ptr (%[\w.]+) to ptr", r"\1 = getelementptr i8, ptr \2, i64 0", ir)
    assert "addrspacecast" not in ir, "an address-space cast the rewrite does not handle"
    ir = ir.replace("amdgpu_kernel ", "")
    ir = re.sub(r"byref\([^)]*\) ", "", ir)
    ir = re.sub(r'syncscope\("[a-z-]*"\) ', "", ir)
    ir = ir.replace("@phz_step(", "@phz_step_ir(")
    for name, host in (("_ZN3phz10phz_sc_tabE", "irx_sc_tab"), ("_ZN3phz11phz_log_tabE", "irx_log_tab")):
        ir = re.sub(rf"@{name} = [^\n]*global \[128 x double\] undef", f"@{host} = global [128 x double] zeroinitializer", ir)
        ir = ir.replace("@" + name, "@" + host)
    for dev, host in IR_INTRINSICS:
        ir = ir.replace("@" + dev + "(", "@" + host + "(")
    left = set(re.findall(r"@llvm\.amdgcn\.[\w.]+", ir))
    assert not left, f"AMDGPU intrinsics without a host meaning: {left}"
    ir = re.sub(r"!amdgpu\.[\w.]+ !\d+", "", ir)
    ir = ir.replace('asm "v_cvt_i32_f64 $0, $1", "=v,v"(', "@irx_cvt_f64(")
    ir = ir.replace('asm "v_cvt_i32_f32 $0, $1", "=v,v"(', "@irx_cvt_f32(")
    ir = re.sub(r'(double|float) asm sideeffect "", "=v,0"', r'\1 asm sideeffect "", "=x,0"', ir)
    ir = re.sub(r'(i32|i64) asm sideeffect "", "=v,0"', r'\1 asm sideeffect "", "=r,0"', ir)
    ir = ir.replace('asm sideeffect "", "=s,=s,0,1"', 'asm sideeffect "", "=r,=r,0,1"')
    ir = ir.replace('asm sideeffect "", "=s,=s,=s,0,1,2"', 'asm sideeffect "", "=r,=r,=r,0,1,2"')
    assert not re.search(r'"=[vs]', ir), "an inline asm statement the rewrite does not handle"
    return ir + "\ndeclare i32 @irx_cvt_f64(double)\ndeclare i32 @irx_cvt_f32(float)\n"


def build_device_ir(device_src: str, prec: str, build: str) -> str:
    """Compile `device_src` for gfx950 to optimised IR under the library's
    `build` flags (finite, reassoc, ieee), run it on the host through the
    driver; returns the executable's path (cached by content)."""
    key = hashlib.sha1((device_src + prec + build + " ".join(DEVICE_IR_FLAGS[build])).encode()).hexdigest()[:16]
    os.makedirs(CACHE, exist_ok=True)
    base = os.path.join(CACHE, f"ir_{key}_{build}")
    exe = base + ".exe"
    if os.path.exists(exe):
        return exe
    with open(base + ".hip", "w") as f:
        f.write(device_src)
    r = subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "--offload-arch=gfx950", "-std=c++17", *DEVICE_IR_FLAGS[build],
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
                        "-emit-llvm", base + ".hip", "-o", base + ".ll"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"device IR build failed:\n{r.stderr[-4000:]}")
    with open(base + "_x86.ll", "w") as f:
        f.write(device_ir_for_host(open(base + ".ll").read()))
    r = subprocess.run([CLANG, "-O0", "-c", base + "_x86.ll", "-o", base + ".o"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host codegen of the device IR failed:\n{r.stderr[-4000:]}")
    drv = host_source(device_src, prec)
    drv = drv.replace("  phz_step(j->a);", "  phz_step_ir(&j->a);")
    drv = drv.replace("struct EmuJob {", IR_SHIMS + "struct EmuJob {")
    drv = drv.replace("int main(int argc, char** argv) {", "int main(int argc, char** argv) {\n"
                      "  phz::fill_tables(0);\n"
                      "  memcpy(irx_sc_tab, phz::phz_sc_tab, sizeof(irx_sc_tab));\n"
                      "  memcpy(irx_log_tab, phz::phz_log_tab, sizeof(irx_log_tab));")
    with open(base + "_drv.cpp", "w") as f:
        f.write(drv)
    r = subprocess.run([CLANG, "-x", "c++", "-std=c++17", "-O1", base + "_drv.cpp", "-x", "none", base + ".o",
                        "-o", exe + ".tmp", "-lpthread"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"driver build failed:\n{r.stderr[-4000:]}")
    os.replace(exe + ".tmp", exe)
    return exe

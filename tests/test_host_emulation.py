"""The step kernel's generated source, run on the CPU by the workgroup
emulation of tests/host_emulation.py, for the plans whose device builds gave
wrong or launch-varying results (the planner refuses them on a device):

  - the MJCF humanoid in f64 with control noise, subtrees merged into two
    waves (on gfx950: every world NaN within a 50-step launch) and into three
    (values of order 1e67 from the first step);
  - the MJCF hand in f64 merged into two waves (one world's NaN bits changed
    between repeats);
  - the f64 terrain + impulse ant under the finite-math flags (qdd wrong by
    1e5 on gfx950, so that kernel is built IEEE).

On the host each runs the same source 50 steps (the impulse case one step
from a settled contact state) under AddressSanitizer and
UndefinedBehaviorSanitizer with every automatic variable and every LDS slot
initialised to NaN and the FP traps armed, under ThreadSanitizer (the waves'
LDS exchange as a multi-threaded protocol), and at -O3 under the device
kernels' finite-math flags; each must match the f64 oracle. They do, to
1e-14: the source holds no out-of-bounds access, read before write, data
race or finite-math violation that these tools see, so the device failures
lie in how the source is compiled for gfx950 or run there, and the plans stay
refused on the device.
"""
import os
import re

import numpy as np
import pytest

from oracle.oracle import Oracle
from phyz_amd import workloads as W
from phyz_amd.model import pack_geometries, uniform_frequency_gains
from phyz_amd.sim import BatchSim, from_workload
from tests import host_emulation as HE
from tests.helpers import oracle_for

pytestmark = pytest.mark.skipif(not os.path.exists(HE.CLANG), reason="clang++ (ROCm LLVM) not present")

NOISE = (0xA55, 1, -0.03, 0.03)  # as tests/test_gpu_mjcf.py


def mjcf_case(name, groups, prec="f64", n=64, lift_pivot=False):
    m = W.mjcf_model(name)
    gains = uniform_frequency_gains(m, 50.0, 1.0)
    geom, _ = pack_geometries(m, gains=gains)
    os.environ["PHZ_HOST_LIFT_GUARDS"] = "1"
    os.environ["PHZ_MAX_GROUPS"] = str(groups)
    if lift_pivot:
        os.environ["PHZ_HOST_LIFT_PIVOT"] = "1"
    try:
        s = BatchSim(m, n, prec, device=-1)
        s.enable_ground_contact_per_body(0.0, 1.0, gains)
        s.enable_control_noise(*NOISE, list(range(m.nctrl())))
        src = HE.dump_source(s)
        block = s.kernel_info()["block"]
    finally:
        os.environ.pop("PHZ_HOST_LIFT_GUARDS", None)
        os.environ.pop("PHZ_MAX_GROUPS", None)
        os.environ.pop("PHZ_HOST_LIFT_PIVOT", None)
    orc = Oracle(m, contact=(geom, 0.0, 1.0), noise=(*NOISE, list(range(m.nctrl()))))
    rng = np.random.default_rng(13)
    q = np.zeros((n, m.nq))
    v = rng.normal(size=(n, m.nv)) * 0.1
    for i, b in enumerate(m.bodies):
        j, o = b.joint, m.q_offsets[i]
        if j.ndof() == 1:
            lo, hi = j.limits if j.limits is not None else (-1.0, 1.0)
            q[:, o] = rng.uniform(lo + 0.05, hi - 0.05, size=n)
        elif j.ndof() == 6:
            q[:, o:o + 3] = rng.normal(size=(n, 3)) * 0.2
            q[:, o + 3:o + 6] = rng.normal(size=(n, 3)) * 0.05
    c = rng.uniform(-0.05, 0.05, size=(n, m.nctrl()))
    return m, src, block, orc, q, v, c


def finite_rows(q, v):
    return np.isfinite(q).all(axis=1) & np.isfinite(v).all(axis=1) & (np.abs(v).max(axis=1) < 1e4)


@pytest.mark.parametrize("name,groups,mode", [
    ("humanoid", 2, "asan"), ("humanoid", 2, "tsan"), ("humanoid", 2, "finite"),
    ("humanoid", 3, "asan"), ("humanoid", 3, "finite"),
    ("shadow_hand", 2, "asan"), ("shadow_hand", 2, "tsan"),
])
def test_refused_f64_plans_are_correct_on_the_host(name, groups, mode):
    n, steps = 64, 50
    m, src, block, orc, q, v, c = mjcf_case(name, groups)
    assert block == 64 * groups  # the guarded plan itself, subtrees merged
    exe = HE.build(src, "f64", mode)
    # The hand's explicit limit law lets a few worlds run away in the oracle
    # too, legitimately producing inf and NaN: traps only where none do.
    trap = mode == "asan" and name == "humanoid"
    qe, ve, _, re, err = HE.run(exe, "f64", groups, q, v, c, orc.rng_states(n), steps, nb=m.nbodies, trap=trap)
    assert "WARNING: ThreadSanitizer" not in err and "runtime error" not in err, err[-3000:]
    qo, vo, co = q.copy(), v.copy(), c.copy()
    rng = orc.rng_states(n)
    orc.step_batch(qo, vo, co, steps, rng=rng, threads=8)
    fo, fe = finite_rows(qo, vo), finite_rows(qe, ve)
    assert np.array_equal(fo, fe) and fo.mean() >= 0.9
    assert np.array_equal(re[fo], rng[fo])  # the control stream advanced exactly as the oracle's
    assert np.abs(qe[fo] - qo[fo]).max() <= 1e-12
    assert np.abs(ve[fo] - vo[fo]).max() <= 1e-12 * max(1.0, np.abs(vo[fo]).max())


@pytest.mark.parametrize("mode", ["asan", "finite"])
def test_f64_impulse_terrain_kernel_is_correct_on_the_host(mode):
    w = W.config(6)
    n = 64
    s = from_workload(w, "f64", nworld=n, device=-1)
    src = HE.dump_source(s)
    q, v, c, _ = w.initial_state(n)
    orc = oracle_for(w)
    nb = w.model.nbodies
    e0, s0 = np.zeros((n, nb, 6)), np.zeros((n, nb, 56))
    orc.step_batch(q, v, c, 300, rng=orc.rng_states(n), threads=8, ext_state=e0, cs_state=s0)  # feet on the terrain
    exe = HE.build(src, "f64", mode)
    qe, ve, qdde, _, err = HE.run(exe, "f64", 1, q, v, c, orc.rng_states(n), 1, nb=nb, trap=mode == "asan",
                                  heightfield=w.heightfield)
    assert "runtime error" not in err, err[-3000:]
    e1, s1 = np.zeros((n, nb, 6)), np.zeros((n, nb, 56))
    want, rows = orc.step_batch(q.copy(), v.copy(), c.copy(), 1, rng=orc.rng_states(n), threads=8, ext_state=e1,
                                cs_state=s1, want_contacts=True)
    assert (rows[:, :, 0] > 0).any()  # contacts active in the compared step
    rel = np.abs(qdde - want).max(axis=1) / np.maximum(np.abs(want).max(axis=1), 1e-12)
    assert rel.max() <= 1e-12


@pytest.mark.parametrize("build", ["finite", "reassoc"])
def test_f64_impulse_device_ir_is_correct_on_the_host(build):
    """The device compiler's own optimised IR of the f64 terrain + impulse
    kernel under the finite-math flags (the build whose accelerations were
    wrong by 1e5 on gfx950; the library builds this kernel IEEE), run on the
    host from settled contact states: it matches the oracle, so the IR passes
    kept the source's meaning."""
    w = W.config(6)
    n = 64
    s = from_workload(w, "f64", nworld=n, device=-1)
    src = HE.dump_source(s)
    q, v, c, _ = w.initial_state(n)
    orc = oracle_for(w)
    nb = w.model.nbodies
    e0, s0 = np.zeros((n, nb, 6)), np.zeros((n, nb, 56))
    orc.step_batch(q, v, c, 300, rng=orc.rng_states(n), threads=8, ext_state=e0, cs_state=s0)
    exe = HE.build_device_ir(src, "f64", build)
    _, _, qdde, _, err = HE.run(exe, "f64", 1, q, v, c, orc.rng_states(n), 1, nb=nb, trap=False,
                                heightfield=w.heightfield)
    e1, s1 = np.zeros((n, nb, 6)), np.zeros((n, nb, 56))
    want, rows = orc.step_batch(q.copy(), v.copy(), c.copy(), 1, rng=orc.rng_states(n), threads=8, ext_state=e1,
                                cs_state=s1, want_contacts=True)
    assert (rows[:, :, 0] > 0).any()
    rel = np.abs(qdde - want).max(axis=1) / np.maximum(np.abs(want).max(axis=1), 1e-12)
    assert rel.max() <= 1e-12, err[-2000:]


@pytest.mark.parametrize("name,groups,build", [("humanoid", 2, "finite"), ("humanoid", 2, "reassoc"),
                                               ("humanoid", 3, "reassoc"), ("humanoid", 4, "reassoc"),
                                               ("humanoid", 4, "finite")])
def test_refused_f64_plans_device_ir_on_the_host(name, groups, build):
    """The refused f64 kernels from the device compiler's own optimised IR, run
    on the host: the MJCF humanoid merged into 2 and 3 waves (NaN or
    launch-varying values from multi-step launches on gfx950) and its 4-wave
    plan with the static pivot bound (non-finite worlds on gfx950), 50 steps
    each against the oracle: the same finite worlds, the same control stream,
    states within 1e-12. What went wrong on the device is not in this IR."""
    n, steps = 64, 50
    m, src, block, orc, q, v, c = mjcf_case(name, groups, lift_pivot=groups == 4)
    assert block == 64 * groups
    if groups == 4:
        assert re.search(r"piv_ok\[\d+\] = \{true(, true)*\}", src)  # the bound's kernel, every body bounded
    exe = HE.build_device_ir(src, "f64", build)
    qe, ve, _, re_, err = HE.run(exe, "f64", groups, q, v, c, orc.rng_states(n), steps, nb=m.nbodies, trap=False)
    qo, vo, co = q.copy(), v.copy(), c.copy()
    rng = orc.rng_states(n)
    orc.step_batch(qo, vo, co, steps, rng=rng, threads=8)
    fo, fe = finite_rows(qo, vo), finite_rows(qe, ve)
    assert np.array_equal(fo, fe) and fo.mean() >= 0.9, err[-2000:]
    assert np.array_equal(re_[fo], rng[fo])
    assert np.abs(qe[fo] - qo[fo]).max() <= 1e-12
    assert np.abs(ve[fo] - vo[fo]).max() <= 1e-12 * max(1.0, np.abs(vo[fo]).max())


def device_math(call: str, words: np.ndarray, nout: int) -> np.ndarray:
    """Run a device-header function on the host: `call` is a C++ statement
    that reads in[i] (a double x = X(i) or a 64-bit word W(i)) and writes
    o[nout * i + j]; the tables filled as a wave fills them."""
    import subprocess
    hdr = open(os.path.join(os.path.dirname(HE.HERE), "phyz_amd", "csrc", "phz_device.h")).read()
    main = r'''
#include <cstdio>
#include <vector>
void* emu_lds_base = nullptr;
extern "C" void emu_syncthreads() {}
int main(int argc, char** argv) {
  for (int lane = 0; lane < 64; lane++) phz::fill_tables(lane);
  FILE* f = fopen(argv[1], "rb");
  long n = 0;
  if (fread(&n, 8, 1, f) != 1) return 3;
  std::vector<unsigned long long> in(n);
  std::vector<double> o(NOUT * n);
  if (fread(in.data(), 8, n, f) != (size_t)n) return 3;
  fclose(f);
  for (long i = 0; i < n; i++) { CALL; }
  f = fopen(argv[2], "wb");
  fwrite(o.data(), 8, NOUT * n, f);
  fclose(f);
  return 0;
}
'''.replace("NOUT", str(nout)).replace("CALL", call)
    prelude = HE.PRELUDE + "#define X(i) __builtin_bit_cast(double, in[i])\n#define W(i) in[i]\n"
    os.makedirs(HE.CACHE, exist_ok=True)
    exe = os.path.join(HE.CACHE, f"device_math_{os.getpid()}")
    with open(exe + ".cpp", "w") as f:
        f.write(prelude + HE.host_device_code(hdr) + main)
    fin, fout = exe + ".in", exe + ".out"
    try:
        r = subprocess.run([HE.CLANG, "-x", "c++", "-std=c++20", "-O2", "-ffp-contract=off", exe + ".cpp", "-o", exe],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-3000:]
        with open(fin, "wb") as f:
            np.array([len(words)], np.int64).tofile(f)
            np.ascontiguousarray(words).view(np.uint64).tofile(f)
        subprocess.run([exe, fin, fout], check=True)
        return np.fromfile(fout).reshape(-1, nout)
    finally:
        for q in (exe, exe + ".cpp", fin, fout):
            if os.path.exists(q):
                os.remove(q)


def test_f64_table_sincos_accuracy():
    """tab_sincos, the f64 kernels' sine and cosine of a revolute joint angle
    and of the Box-Muller angle, compiled from the device header for the host,
    against mpmath at 40 digits: within 2 ulp on joint-angle ranges (4 ulp up
    to |x| = 3e6, where the reduction's two-part 2 pi / 64 loses a little),
    exact where the angle is below pi / 128 (the sine is then r itself), and
    at the table's own nodes and the midpoints between them."""
    import mpmath
    rng = np.random.default_rng(1)
    nodes = np.arange(-320, 321) * (2 * np.pi / 64)
    near = np.concatenate([rng.uniform(-60, 60, 3000), nodes, np.nextafter(nodes, np.inf),
                           np.nextafter(nodes, -np.inf), nodes + np.pi / 64, [np.pi, -np.pi, np.pi / 2, 2 * np.pi]])
    tiny = np.concatenate([np.logspace(-300, np.log10(np.pi / 128) - 1e-9, 300), [0.0]])
    tiny = np.concatenate([tiny, -tiny])
    far = rng.uniform(-3e6, 3e6, 500)
    xs = np.concatenate([near, tiny, far])
    o = device_math("phz::tab_sincos(X(i), &o[2 * i], &o[2 * i + 1])", xs, 2)
    mpmath.mp.dps = 40
    ref = np.array([[float(mpmath.sin(mpmath.mpf(x))), float(mpmath.cos(mpmath.mpf(x)))] for x in xs])
    err, ulp = np.abs(o - ref), np.spacing(np.abs(ref))
    a, b = len(near), len(near) + len(tiny)
    assert (err[:a] <= 2 * ulp[:a] + 2.0 ** -60).all()
    assert (err[a:b, 0] == 0).all() and (err[a:b, 1] <= ulp[a:b, 1]).all()
    assert (err[b:] <= 4 * ulp[b:] + 2.0 ** -60).all()


def test_f64_table_log_sqrt_and_box_muller_accuracy():
    """The f64 Box-Muller pieces compiled from the device header for the host,
    against mpmath at 40 digits: tab_log within 1 ulp over 1 - u for uniform u,
    x just below 1 (1 - k 2^-53), the powers of two the radius meets, the
    table's interval boundaries and their neighbours, and normal x from 1e-300
    to 1e300, exactly 0 at 1; nr_sqrt (with the host's exact reciprocal square
    root for the hardware estimate, so this pins the refinement, not the
    estimate) correctly rounded on [0, 80] and over the normal range; and
    box_muller(double) from 64-bit states: the state advanced by exactly two
    xorshift64 draws, the radius within 1 ulp of sqrt(-2 ln(1 - u1)) and the
    sine and cosine within 2 ulp of those of 2 pi u2."""
    import struct

    import mpmath
    mpmath.mp.dps = 40
    rng = np.random.default_rng(3)
    bounds = []
    for i in range(65):
        b = struct.unpack("<d", struct.pack("<Q", (0x3FE62000 + i * 2 ** 14) << 32))[0]
        bounds += [b, np.nextafter(b, 0), np.nextafter(b, 2)]
    xs = np.concatenate([1 - rng.random(2000), 1 - np.arange(0, 200) * 2.0 ** -53, 2.0 ** -np.arange(0, 54), bounds,
                         np.exp(rng.uniform(-690, 690, 1000)), [1e-300]])
    got = device_math("o[i] = phz::tab_log(X(i))", xs, 1)[:, 0]
    ref = np.array([float(mpmath.log(mpmath.mpf(x))) for x in xs])
    assert got[xs == 1.0].tolist() == [0.0] * int((xs == 1.0).sum())
    nz = ref != 0
    assert (np.abs(got - ref)[nz] <= np.spacing(np.abs(ref))[nz]).all()

    ys = np.concatenate([rng.uniform(0, 80, 2000), [0.0, 2.0 ** -52, 2.0 ** -1000, 1.0, 2.0, 4.0],
                         np.exp(rng.uniform(-690, 690, 1000))])
    assert np.array_equal(device_math("o[i] = phz::nr_sqrt(X(i))", ys, 1)[:, 0], np.sqrt(ys))

    st = rng.integers(1, 2 ** 63, 1500, dtype=np.int64).astype(np.uint64)
    got = device_math("{ unsigned long long s = W(i); phz::box_muller(s, &o[4 * i], &o[4 * i + 1], &o[4 * i + 2]);"
                      " o[4 * i + 3] = __builtin_bit_cast(double, s); }", st, 4)
    mask = (1 << 64) - 1

    def xorshift(x):
        x ^= (x << 13) & mask
        x ^= x >> 7
        return x ^ ((x << 17) & mask)

    ref, nxt = [], []
    for s0 in st:
        x1 = xorshift(int(s0))
        x2 = xorshift(x1)
        u1, u2 = mpmath.mpf(x1 >> 11) / 2 ** 53, mpmath.mpf(x2 >> 11) / 2 ** 53
        ref.append([float(mpmath.sqrt(-2 * mpmath.log(1 - u1))), float(mpmath.sin(2 * mpmath.pi * u2)),
                    float(mpmath.cos(2 * mpmath.pi * u2))])
        nxt.append(x2)
    ref = np.array(ref)
    assert np.array_equal(got[:, 3].view(np.uint64), np.array(nxt, dtype=np.uint64))
    err, ulp = np.abs(got[:, :3] - ref), np.spacing(np.abs(ref))
    assert (err[:, 0] <= ulp[:, 0]).all() and (err[:, 1:] <= 2 * ulp[:, 1:]).all()

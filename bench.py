"""Benchmark: world-steps/s of the fused step kernel on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload 2] [--no-cpu]

A "step" is one physics step (control noise, PD, contact, ABA, integrate) of
every world of the workload. The headline `value` is the 7-link chain, 65536
worlds, f32: W warmup steps run untimed, then spans of exactly K steps are
timed by the host clock with the device synchronized on both sides (the median
of --reps spans, each from the workload's seeded initial state, reloaded
untimed); the kernel's own time comes from hipEvents on the sim's stream that
the span's first and last launch stamp with their own start and end
(hipExtModuleLaunchKernel), so it is the kernels' execution time, without the
dispatch around them. Before the warmup the device runs the same span
untimed for --settle-ms, so a short span is not timed at the idle clock. State
stays resident in HBM for the whole measurement.

configs (unless --no-configs): every benchmark configuration (the double
pendulum, chain7, ant, humanoid and hand) at its own worlds x rollout length,
in each precision it names, each with its roofline, its CPU baseline and the
device's parity at the rollout's late state.

roofline: algorithmic FLOPs per launch (tests/golden/flops_per_world_step.json,
counted on the oracle's structure-exploiting formulation x worlds x steps per
launch) over the kernel-stamped launch duration, against MI355X's vector peak
(FP64 78.6 TFLOP/s; FP32 157.3 TFLOP/s published). `traffic` is the kernel's
measured HBM bytes per launch (profiles/hbm_traffic.json, rocprofv3 --pmc
FETCH_SIZE and WRITE_SIZE scaled by a plain copy's readings): one state round
trip per launch, whatever its step count.

cpu_baseline: the f64 CPU oracle (a restatement of the reference's CPU step),
threaded over worlds on the host's cores (the CPUs this process may use,
capped by the cgroup quota), timed on a bounded sample of the same workload.
parity: one more device step from the timed rollout's late state against the
oracle on 64 sampled worlds, with the bound (qdd normwise relative error 1e-10
f64, 1e-4 f32), pass or fail, and the share of worlds within it.

terrain_impulse (unless --no-impulse): the same measurement of workload 6, the
ant on a rolling heightfield with impulse-mode contact (16 sweeps per step),
131072 worlds x 1000 steps, f32, with its own roofline, CPU baseline and parity.
mjcf (unless --no-mjcf): workloads 7-9, the reference's MJCF ant, humanoid and
hand driven by their own actuators, f32, at a 1 ms step (the reference's
explicit joint-limit law runs light links away at the files' own steps).
`value` counts the worlds still finite at the end of the timed span (every
world, at 1 ms), and `all_worlds_value` every world.
world_sweep (unless --no-sweep; --sweep-only runs just this): chain7 in f32
and f64 at 1024 to 262144 worlds, 100-step spans: kernel and wall
world-steps/s, and with each span's load and readback.
io (every configuration): load_states, readback_states and its
allocation-free variant timed apart from the resident spans, and the
reference's repetition (load, span, readback) with the readback's share.
control_loop (unless --no-control): the ant driven by the on-device policy.
ppo_update (unless --no-ppo; --ppo-only runs just this): the PPO update pass at
the reference's timing shape (a million samples, actor 55-64-64-22, critic
67-64-64-1, minibatch 4096, one epoch) with the batch resident: samples/s of
whole updates, the tile kernel's roofline from kernel-stamped hipEvents, and, with the CPU
leg, the f64 CPU update on 128 minibatches plus the device's update of that
sample against it.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "world-steps/sec (ABA+contact+integrate) on 1 MI355X; % of HBM/FP64 roofline"
PEAK_TFLOPS = {"f64": 78.6, "f32": 157.3}
HBM_PEAK_GBS = 8000.0
FLOPS_JSON = os.path.join(ROOT, "tests", "golden", "flops_per_world_step.json")
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "hbm_traffic.json")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def host_threads():
    """Threads for the CPU baseline: the CPUs this process may run on, capped by
    the cgroup's CPU quota where one is set. Returns (threads, details)."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = max(1, int(q) // int(period))
    except (OSError, ValueError):
        pass
    threads = min(aff, quota) if quota else aff
    return threads, {"os_cpu_count": os.cpu_count(), "affinity_cpus": aff, "cgroup_quota_cpus": quota}


def cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def run_gpu(w, prec, steps, warmup, reps, settle_ms=0.0):
    """W = warmup untimed steps (whole spans of the timed length), then `reps`
    wall-clock spans of exactly `steps` steps, each from the workload's seeded
    initial state (reloaded untimed) and bracketed by a device synchronization
    on both sides, plus the same number of spans run back to back from the
    initial state, each timed by hipEvents its own launches stamp with their
    start and end on the sim's stream. settle_ms: untimed spans run first until the device has been
    busy that long, so that a short timed span does not run at the idle clock."""
    from phyz_amd.sim import from_workload
    sim = from_workload(w, prec, nworld=w.nworld, device=0)
    q, v, c, tg = w.initial_state()

    def reload():
        sim.load_states(q, v, c)
        if tg is not None:
            sim.set_position_targets(tg)

    reload()
    sim.compile()
    settle = {"spans": 0, "ms": 0.0}
    if settle_ms > 0:
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < settle_ms:
            sim.step_many(steps)
            sim.synchronize()
            settle["spans"] += 1
        settle["ms"] = round((time.perf_counter() - t0) * 1e3, 2)
        reload()
    done = 0
    while done < warmup:  # captures the span's graph, so the timed spans replay it
        sim.step_many(steps)
        done += steps
    walls = []
    for _ in range(reps):
        reload()
        sim.synchronize()
        t0 = time.perf_counter()
        sim.step_many(steps)
        sim.synchronize()
        walls.append(time.perf_counter() - t0)
    # Kernel time: `reps` spans back to back (the clock stays up between them),
    # each timed by the events its own launches stamp.
    reload()
    ev = list(sim.time_step_many(steps, reps))
    io = time_io(sim, reload, steps)
    reload()
    sim.step_many(steps)
    info = sim.kernel_info()
    return sim, np.array(walls), np.array(ev), info, done, settle, io


def _median_ms(fn, reps):
    t = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        t.append(time.perf_counter() - t0)
    return round(float(np.median(t)) * 1e3, 4)


def time_io(sim, reload, steps, reps=5):
    """Upload and readback, timed apart from the resident spans (the
    reference's batch bench, crates/phyz-bench/src/suites/gpu_batch.rs:231-246):
    load_states (world-major f64 rows to the device's SoA layout, with the PD
    targets where the workload has them), readback_states and its
    allocation-free variant, and the reference's own repetition, load + span +
    readback, with the readback's share of it."""
    out = {"load_states_ms": _median_ms(reload, reps)}
    sim.step_many(steps)
    sim.synchronize()
    out["readback_states_ms"] = _median_ms(sim.readback_states, reps)
    width = max(sim.model.nq, sim.model.nv)
    if sim.nworld * width * 8 <= 32 << 20:
        out["readback_states_noalloc_ms"] = _median_ms(sim.readback_states_noalloc, reps)

    def rep():
        reload()
        sim.step_many(steps)
        sim.readback_states()

    out["load_span_readback_ms"] = _median_ms(rep, reps)
    out["readback_share"] = round(out["readback_states_ms"] / out["load_span_readback_ms"], 4)
    out["steps"] = steps
    return out


def launches_per_span(steps, info):
    per = max(1, int(info["max_steps_per_launch"]))
    return (steps + per - 1) // per


def traffic_for(traffic_tab, name, prec, steps_per_launch):
    """Measured HBM bytes per launch of this kernel. The step kernels load the
    state once and store it once per launch whatever its step count, so a
    figure measured at another span length applies; the entry for the exact
    span is used where one was measured."""
    if not traffic_tab:
        return None, None
    exact = traffic_tab.get(f"{name}_{prec}_{int(steps_per_launch)}")
    if exact:
        return exact["hbm_bytes_per_launch"], exact["steps_per_launch"]
    for k in sorted(traffic_tab):
        e = traffic_tab[k]
        if k.startswith(f"{name}_{prec}_") and "steps_per_launch" in e:
            return e["hbm_bytes_per_launch"], e["steps_per_launch"]
    return None, None


def roofline(w, prec, steps, ev_ms, info, flops_tab, traffic_tab):
    f = flops_tab[w.name]
    nl = launches_per_span(steps, info)
    steps_per_launch = steps / nl
    flops_per_launch = f["flops_per_world_step"] * w.nworld * steps_per_launch
    launch_s = float(np.median(ev_ms)) / 1e3 / nl
    achieved = flops_per_launch / launch_s / 1e12
    traffic, measured_at = traffic_for(traffic_tab, w.name, prec, steps_per_launch)
    algo_bytes = f["bytes_per_world_step"][prec] * w.nworld  # one state round trip per launch
    return {
        "bound": "valu",
        "achieved": round(achieved, 4),
        "peak": PEAK_TFLOPS[prec],
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_TFLOPS[prec], 5),
        "traffic": traffic,
        "traffic_measured_steps_per_launch": measured_at,
        "algorithmic_bytes_per_launch": int(algo_bytes),
        "flops_per_world_step": f["flops_per_world_step"],
        "launch_ms": round(launch_s * 1e3, 4),
        "steps_per_launch": int(steps_per_launch),
        "hbm_frac": round(algo_bytes / launch_s / 1e9 / HBM_PEAK_GBS, 6),
    }


# Per-step qdd bounds, normwise relative to max|qdd| of the f64 oracle, in
# every contact mode.
QDD_BOUND = {"f64": 1e-10, "f32": 1e-4}


def device_step_parity(w, sim, prec):
    """One more device step from the benchmark's late states against the oracle,
    on 64 sampled finite worlds (tests.helpers.late_step_errors). Reports the
    largest error, the bound, pass or fail, and the share of worlds within the
    bound."""
    from tests.helpers import late_step_errors
    qg, vg = sim.readback_states()
    finite = np.flatnonzero(np.isfinite(qg).all(axis=1) & np.isfinite(vg).all(axis=1))
    if finite.size == 0:
        return {"worlds_checked": 0, "pass": False, "note": "no finite world left after the timed spans"}
    idx = finite[np.linspace(0, len(finite) - 1, 64).astype(int)]
    e, extra = late_step_errors(w, sim, prec, idx)
    bound = QDD_BOUND[prec]
    return {"worlds_checked": len(idx), "qdd_rel_err_max": float(e.max()), "qdd_rel_err_median": float(np.median(e)),
            "bound": bound, "pass": bool(e.max() <= bound), "share_within_bound": round(float(np.mean(e <= bound)), 4),
            **extra}


def cpu_baseline(w, budget_s=8.0):
    """The f64 oracle (a restatement of the reference's CPU step) threaded over
    worlds on the host's cores, on a bounded sample of the same workload (its
    seeded initial states, replayed control stream): `budget_s` seconds of
    multi-threaded work, plus a single-thread rate on a smaller sample."""
    from tests.helpers import oracle_for
    threads, host = host_threads()
    orc = oracle_for(w)
    imp = w.impulse_sweeps > 0
    nb = w.model.nbodies

    def carried(n):
        return (np.zeros((n, nb, 6)), np.zeros((n, nb, 56))) if imp else (None, None)

    def run(n, steps, nthreads):
        q, v, c, tg = w.initial_state(n)
        e, cs = carried(n)
        t0 = time.perf_counter()
        orc.step_batch(q, v, c, steps, targets=tg, rng=orc.rng_states(n), threads=nthreads, ext_state=e, cs_state=cs)
        return time.perf_counter() - t0

    n = min(w.nworld, max(1024, 256 * threads))
    probe = run(n, 2, threads)
    s = max(2, int(budget_s * 2 / max(probe, 1e-6)))
    dt = run(n, s, threads)
    n1 = min(n, 256)
    s1 = max(2, int(0.1 * budget_s * n * s / dt / n1 / max(threads, 1)))
    dt1 = run(n1, s1, 1)
    return {
        "value": round(n * s / dt, 1),
        "unit": "world-steps/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{w.name}: first {n} worlds x {s} steps, f64 oracle, {threads} threads ({dt:.1f} s)",
        "single_thread_value": round(n1 * s1 / dt1, 1),
        "host": {**host, "cpu": cpu_model_name()},
    }


def measure(w, precs, steps, warmup, reps, with_cpu, cpu_budget_s=8.0, settle_ms=0.0):
    """Wall-clock and event-timed spans of `steps` steps per precision, the
    roofline of the step kernel, the device's parity at the late state, and
    (with_cpu) the oracle's CPU rate."""
    flops_tab = json.load(open(FLOPS_JSON))
    traffic_tab = json.load(open(TRAFFIC_JSON)) if os.path.exists(TRAFFIC_JSON) else None
    results = {}
    for prec in precs:
        log(f"[bench] {w.name} {prec}: {w.nworld} worlds, warmup {warmup}, timed {steps} steps x {reps}")
        sim, walls, ev, info, warm_done, settle, io = run_gpu(w, prec, steps, warmup, reps, settle_ms)
        wall = float(np.median(walls))
        med = float(np.median(ev))
        spread = (max(ev) - min(ev)) / med if med > 0 else 0.0
        qf, vf = sim.readback_states()
        finite = float(np.mean(np.isfinite(qf).all(axis=1) & np.isfinite(vf).all(axis=1)))
        r = {
            "value": round(w.nworld * steps / wall, 1),
            "unit": "world-steps/s",
            "ms_per_step": round(wall * 1e3 / steps, 6),
            "wall_ms_per_span": {"median": round(wall * 1e3, 4), "min": round(float(walls.min()) * 1e3, 4),
                                 "max": round(float(walls.max()) * 1e3, 4), "reps": len(walls)},
            "event_ms_per_span": {"median": round(med, 4), "min": round(float(min(ev)), 4),
                                  "max": round(float(max(ev)), 4), "reps": len(ev), "noisy": bool(spread > 0.25)},
            "world_steps_per_s_event_median": round(w.nworld * steps / (med / 1e3), 1),
            "finite_worlds": round(finite, 4),
            "roofline": roofline(w, prec, steps, ev, info, flops_tab, traffic_tab),
            "kernel": info,
            "warmup_steps_run": warm_done,
            "io": io,
        }
        if settle["spans"]:
            r["clock_settle"] = settle
        if with_cpu:
            r["parity"] = device_step_parity(w, sim, prec)
        sim.close()
        results[prec] = r
        log(f"[bench] {w.name} {prec}: {r['value']:.4g} world-steps/s, {r['roofline']['achieved']:.3f} TFLOP/s "
            f"({100 * r['roofline']['frac']:.2f}% of peak)"
            + (f"; parity qdd {r['parity']['qdd_rel_err_max']:.2e} ({'pass' if r['parity']['pass'] else 'FAIL'})"
               if with_cpu else ""))
    cpu = None
    if with_cpu:
        log(f"[bench] {w.name}: cpu_baseline")
        cpu = cpu_baseline(w, cpu_budget_s)
    return {"results": results, "cpu": cpu}


SWEEP_WORLDS = (1024, 2048, 4096, 8192, 16384, 32768, 65536, 131072, 262144)


def run_world_sweep(idx=2, sizes=SWEEP_WORLDS, precs=("f32", "f64"), steps=100, reps=5):
    """Throughput against the number of worlds (the reference sweeps batch
    sizes the same way, BENCHMARKS.md:318-338): the workload's kernel at each
    size, spans of `steps` steps from its seeded states; kernel time from the
    launches' own hipEvents, wall time with the device synchronized on both
    sides, and the reference's repetition (load, span, readback). 8192 worlds
    is one GPU's share of the 65536-world chain over eight GPUs."""
    from phyz_amd import workloads as W
    from phyz_amd.sim import from_workload
    w = W.config(idx)
    flops = json.load(open(FLOPS_JSON))[w.name]["flops_per_world_step"]
    out = []
    for prec in precs:
        for n in sizes:
            sim = from_workload(w, prec, nworld=n, device=0)
            q, v, c, tg = w.initial_state(n)

            def reload():
                sim.load_states(q, v, c)
                if tg is not None:
                    sim.set_position_targets(tg)

            reload()
            sim.compile()
            for _ in range(3):
                sim.step_many(steps)
            sim.synchronize()
            ev = float(np.median(sim.time_step_many(steps, reps)))
            reload()
            wall = []
            for _ in range(reps):
                sim.synchronize()
                t0 = time.perf_counter()
                sim.step_many(steps)
                sim.synchronize()
                wall.append(time.perf_counter() - t0)
            wall_ms = float(np.median(wall)) * 1e3

            def rep():
                reload()
                sim.step_many(steps)
                sim.readback_states()

            rep_ms = _median_ms(rep, 3)
            info = sim.kernel_info()
            out.append({"workload": w.name, "dtype": prec, "nworld": n, "steps": steps,
                        "lanes_per_world": info["lanes_per_world"], "block": info["block"],
                        "event_ms_per_span": round(ev, 4), "wall_ms_per_span": round(wall_ms, 4),
                        "world_steps_per_s_event": round(n * steps / (ev / 1e3), 1),
                        "world_steps_per_s_wall": round(n * steps / (wall_ms / 1e3), 1),
                        "tflops_event": round(flops * n * steps / (ev / 1e3) / 1e12, 3),
                        "frac_of_peak_event": round(flops * n * steps / (ev / 1e3) / 1e12 / PEAK_TFLOPS[prec], 4),
                        "load_span_readback_ms": rep_ms,
                        "world_steps_per_s_with_io": round(n * steps / (rep_ms / 1e3), 1)})
            sim.close()
            r = out[-1]
            log(f"[bench] sweep {w.name} {prec} {n:>6} worlds: {r['world_steps_per_s_event']:.3g} world-steps/s "
                f"(kernel), {r['world_steps_per_s_wall']:.3g} (wall), {100 * r['frac_of_peak_event']:.1f}% of peak; "
                f"with load + readback {r['world_steps_per_s_with_io']:.3g}")
    return out


def run_control_loop(prec: str, reps: int, with_cpu: bool):
    """The ant driven by the on-device policy (phyz_amd.workloads.control_loop):
    a rollout of n_control control steps, each FK + observation, the MLP policy,
    control_every physics steps and a state snapshot, as one captured graph."""
    from phyz_amd import workloads as W
    from phyz_amd.sim import from_control_loop
    cl = W.control_loop()
    n, nc, every = cl.nworld, cl.n_control, cl.control_every
    log(f"[bench] control loop {cl.name}: {n} worlds, {nc} control steps x {every} physics steps, "
        f"MLP {cl.spec.n_in()}-{cl.spec.hidden}-{cl.spec.hidden}-{cl.spec.n_out()}")
    sim = from_control_loop(cl, prec)
    q, v, _, _ = cl.base.initial_state()
    sim.load_states(q, v)
    sim.compile()
    sim.rollout(0, nc, every, True)  # builds the kernels and captures the rollout graph
    sim.synchronize()
    ev = []
    for _ in range(reps):
        sim.load_states(q, v)
        sim.seed_policy(cl.seed)
        ev.extend(sim.time_rollout(0, nc, every, True, 1))
    t_roll = float(np.median(ev))
    t_obs = float(np.median(sim.time_control_kernel("obs", 0, 20)))
    t_pol = float(np.median(sim.time_control_kernel("policy", 0, 20)))
    t_phys = float(np.median(sim.time_step_many(nc * every, 3)))
    m = cl.base.model
    obs_bytes = n * 4 * ((m.nq + m.nv) + 18 * m.nbodies + cl.spec.n_in())
    pol_flops = cl.flops_per_world() * n
    out = {
        "workload": cl.name, "nworld": n, "n_control": nc, "control_every": every, "dtype": prec,
        "mlp": [cl.spec.n_in(), cl.spec.hidden, cl.spec.hidden, cl.spec.n_out()],
        "rollout_ms": {"median": round(t_roll, 4), "min": round(float(min(ev)), 4), "max": round(float(max(ev)), 4)},
        "world_steps_per_s": round(n * nc * every / (t_roll / 1e3), 1),
        "control_steps_per_s": round(n * nc / (t_roll / 1e3), 1),
        "physics_only_ms": round(t_phys, 4),
        "policy_roofline": {"bound": "mfma", "achieved": round(pol_flops / (t_pol / 1e3) / 1e12, 3), "peak": 157.3,
                            "unit": "TFLOP/s", "frac": round(pol_flops / (t_pol / 1e3) / 1e12 / 157.3, 4),
                            "launch_ms": round(t_pol, 5), "flops_per_world": cl.flops_per_world(),
                            "kernel": sim.control_kernel_info("policy")},
        "obs_roofline": {"bound": "hbm", "achieved": round(obs_bytes / (t_obs / 1e3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(obs_bytes / (t_obs / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                         "launch_ms": round(t_obs, 5), "bytes_per_world": obs_bytes // n},
    }
    log(f"[bench] control loop: {out['world_steps_per_s']:.4g} world-steps/s, rollout {t_roll:.3f} ms "
        f"(physics alone {t_phys:.3f} ms), policy {t_pol:.4f} ms = {out['policy_roofline']['achieved']} TFLOP/s, "
        f"obs {t_obs:.4f} ms = {out['obs_roofline']['achieved']} GB/s")
    if with_cpu:
        out["parity"], orc = control_parity(cl, sim, q, v)
        out["cpu_baseline"] = control_cpu_baseline(cl, orc)
    return out


def control_parity(cl, sim, q, v):
    """Part of the CPU-baseline leg: one control step of sampled worlds against
    the oracle, exact stream replay."""
    from oracle import policy_ref as PR
    from oracle.oracle import Oracle
    from phyz_amd.model import pack_geometries, pack_pd_dofs
    m, n = cl.base.model, cl.nworld
    sim.load_states(q, v)
    sim.seed_policy(cl.seed)
    sim.run_policy(0)
    dq, dv = sim.readback_states()
    obs_h, out_h = sim.readback_policy_history(0, 1)
    tgt = sim.readback_targets()
    g, _ = pack_geometries(m, cl.base.contact.stiffness, cl.base.contact.damping)
    orc = Oracle(m, contact=(g, cl.base.contact.ground_height, cl.base.contact.friction), pd=pack_pd_dofs(cl.pd))
    idx = np.linspace(0, n - 1, 32).astype(int)
    base = cl.base_targets(n)
    err = {"obs": 0.0, "act": 0.0, "logp": 0.0, "targets": 0.0}
    for k in idx:
        o = np.array(PR.observe_reference(m, orc, dq[k], dv[k], cl.spec.obs))
        z = np.zeros(cl.spec.n_out())
        t = np.zeros(len(cl.pd))
        a, lp = PR.policy_reference(cl.spec, cl.weights, cl.std, PR.KernelRng.for_world(cl.seed, int(k)), o, z, base[k], t)
        err["obs"] = max(err["obs"], float(np.abs(obs_h[0, k] - o).max()))
        err["act"] = max(err["act"], float(np.abs(out_h[0, k, :-1] - a).max()))
        err["logp"] = max(err["logp"], abs(float(out_h[0, k, -1]) - lp))
        err["targets"] = max(err["targets"], float(np.abs(tgt[k] - t).max()))
    return {"worlds_checked": len(idx), **{k: float(f"{e:.3g}") for k, e in err.items()}}, orc


def control_cpu_baseline(cl, orc, nworld: int = 8192, n_control: int = 32):
    """The oracle's rollout on a bounded sample: per control step the f64 FK on
    all host threads, the observation ops and the policy batched over worlds in
    numpy (oracle/policy_ref.py's batched forms), then the f64 physics steps
    threaded over worlds."""
    from oracle import policy_ref as PR
    threads, _ = host_threads()
    m = cl.base.model
    q, v, c, _ = cl.base.initial_state(nworld)
    base = cl.base_targets(nworld)
    rng = PR.BatchRng.for_worlds(cl.seed, range(nworld))
    z = np.zeros((nworld, cl.spec.n_out()))
    tg = np.zeros((nworld, len(cl.pd)))
    t_pol = 0.0
    t0 = time.perf_counter()
    for _ in range(n_control):
        ta = time.perf_counter()
        obs = PR.observe_batch(m, orc, q, v, cl.spec.obs, threads)
        PR.policy_batch(cl.spec, cl.weights, cl.std, rng, obs, z, base, tg)
        t_pol += time.perf_counter() - ta
        orc.step_batch(q, v, c, cl.control_every, targets=tg, threads=threads)
    dt = time.perf_counter() - t0
    return {"value": round(nworld * n_control * cl.control_every / dt, 1), "unit": "world-steps/s", "cores": threads,
            "kind": "port", "sample": f"{nworld} worlds x {n_control} control steps x {cl.control_every} physics steps, "
                                      f"f64 oracle (FK and physics in C++ on {threads} threads, observation and policy "
                                      f"batched over worlds in numpy), {dt:.1f} s of which observe+policy "
                                      f"{t_pol:.1f} s",
            "control_steps_per_s": round(nworld * n_control / dt, 1)}


# The reference's PPO timing shape (crates/phyz-gpu/examples/cuda_train.rs:46-66):
# a million samples, actor obs 55 -> 64 -> 64 -> 22, critic obs 67 -> 64 -> 64 -> 1,
# minibatch 4096, one epoch (245 minibatches), no KL brake.
PPO_SHAPE = {"samples": 1_000_000, "actor_in": 55, "critic_in": 67, "hidden": 64, "act": 22, "minibatch": 4096}
# Its published times (docs/design/cuda-backend.md:291-299): one update on an
# RTX PRO 6000 Blackwell, and tang's f64 CPU update.
PPO_REFERENCE_S = {"device": 3.57, "device_hardware": "RTX PRO 6000 Blackwell", "tang_f64_cpu": 35.26}


def ppo_flops(b, nets):
    """Algorithmic FLOPs of one minibatch of b rows: per network the forward
    (3 layers), the weight and bias gradients (same size) and the two hidden
    backprops, 2 FLOPs per multiply-add."""
    f = 0
    for n_in, n_h, n_out in nets:
        layers = n_in * n_h + n_h * n_h + n_h * n_out
        f += 2 * b * (2 * layers + n_out * n_h + n_h * n_h)
    return f


def ppo_traffic():
    """HBM bytes per tile-kernel launch from the committed FETCH_SIZE / WRITE_SIZE
    counters (profiles/ppo_update_kernel_stats.txt), or None."""
    if not os.path.exists(TRAFFIC_JSON):
        return None
    entry = json.load(open(TRAFFIC_JSON)).get("ppo_tiles")
    return entry["hbm_bytes_per_launch"] if entry else None


def run_ppo_update(reps: int, with_cpu: bool):
    """The PPO update pass (phyz_amd.train) at the reference's timing shape:
    wall time per update with the batch resident, and the tile kernel's
    hipEvent time for its roofline."""
    from phyz_amd.train import AdamCfg, KlMode, NetDims, PpoUpdateCfg, SampleBatch, TrainPipeline
    P = PPO_SHAPE
    n, a_in, c_in, h, act, mb = P["samples"], P["actor_in"], P["critic_in"], P["hidden"], P["act"], P["minibatch"]
    ad, cd = NetDims(a_in, h, act), NetDims(c_in, h, 1)
    log(f"[bench] ppo update: {n} samples, actor {a_in}-{h}-{h}-{act}, critic {c_in}-{h}-{h}-1, minibatch {mb}")
    rng = np.random.default_rng(0xC0FFEE)
    f32 = lambda a: a.astype(np.float32)  # noqa: E731
    batch = SampleBatch(f32(rng.normal(size=(n, a_in)) * 0.5), f32(rng.normal(size=(n, c_in)) * 0.5),
                        f32(rng.normal(size=(n, act)) * 0.3), f32(-20.0 + rng.normal(size=n) * 0.4),
                        f32(rng.normal(size=n)), f32(rng.normal(size=n) * 2.0))
    a0 = rng.normal(size=ad.param_count() + act) * 0.1
    c0 = rng.normal(size=cd.param_count()) * 0.1
    cfg = PpoUpdateCfg(0.2, 0.003, 6.0, mb, 1, float("inf"), float(act), KlMode.MINIBATCH)
    pipe = TrainPipeline(ad, cd, n, mb)
    pipe.set_adam(AdamCfg(), AdamCfg())
    pipe.set_actor_params(a0)
    pipe.set_critic_params(c0)
    t0 = time.perf_counter()
    pipe.upload_batch(n, batch)
    upload_s = time.perf_counter() - t0
    orders = [rng.permutation(n).astype(np.uint32) for _ in range(reps + 2)]
    pipe.update([orders[0]], cfg)  # warmup
    wall = []
    for r in range(reps):
        t0 = time.perf_counter()
        st = pipe.update([orders[1 + r]], cfg)
        wall.append(time.perf_counter() - t0)
    _, ms, nmb = pipe.time_update([orders[-1]], cfg)
    med = float(np.median(wall))
    nets = [(a_in, h, act), (c_in, h, 1)]
    full, last = divmod(n, mb)
    flops = full * ppo_flops(mb, nets) + (ppo_flops(last, nets) if last else 0)
    tiles_ms = float(ms[0])
    out = {
        "value": round(n / med, 1), "unit": "samples/s", "dtype": "f32 (f64 Adam and gradient sums)",
        "seconds_per_update": round(med, 6), "ms_per_minibatch": round(med * 1e3 / st.grad_steps, 5),
        "minibatches": st.grad_steps, "upload_s": round(upload_s, 4),
        "wall_s": {"median": round(med, 6), "min": round(min(wall), 6), "max": round(max(wall), 6), "reps": reps},
        "config": {"workload": "ppo_update", **P, "epochs": 1, "tile_rows": pipe.rows_per_tile},
        "kernel_ms_per_launch": {"ppo_tiles": round(ms[0] / nmb, 5), "ppo_adam": round(ms[1] / nmb, 5)},
        "roofline": {"bound": "valu", "kernel": "ppo_tiles",
                     "achieved": round(flops / (tiles_ms / 1e3) / 1e12, 3), "peak": 157.3, "unit": "TFLOP/s",
                     "frac": round(flops / (tiles_ms / 1e3) / 1e12 / 157.3, 4), "flops_per_update": flops,
                     "launch_ms": round(tiles_ms / nmb, 5), "traffic": ppo_traffic()},
        "reference_published": {**PPO_REFERENCE_S, "speedup_vs_published_device": round(PPO_REFERENCE_S["device"] / med, 1)},
    }
    log(f"[bench] ppo update: {med * 1e3:.3f} ms per update ({out['ms_per_minibatch'] * 1e3:.1f} us per minibatch), "
        f"tiles {out['kernel_ms_per_launch']['ppo_tiles'] * 1e3:.1f} us / adam+brake "
        f"{out['kernel_ms_per_launch']['ppo_adam'] * 1e3:.1f} us per launch; "
        f"{out['roofline']['achieved']} TFLOP/s in the tile kernel")
    if with_cpu:
        out["cpu_baseline"], out["parity"] = ppo_cpu_baseline(batch, a0, c0, ad, cd, cfg)
    return out


def ppo_cpu_baseline(batch, a0, c0, ad, cd, cfg, n_mb: int = 128):
    """The f64 CPU update (the oracle's restatement of tang's) on the first
    n_mb minibatches of the same batch, BLAS on the host's cores, as samples/s; and
    the device's update of that sample against it (per-parameter weight-delta
    gaps over the largest delta)."""
    from threadpoolctl import threadpool_limits
    from oracle.ppo_ref import CpuPpo, Dims
    from phyz_amd.train import SampleBatch, TrainPipeline
    rows = n_mb * cfg.minibatch
    cols = {k: getattr(batch, k)[:rows] for k in ("obs_a", "obs_c", "act", "logp_old", "adv", "ret")}
    order = [np.random.default_rng(7).permutation(rows).astype(np.uint32)]
    cpu = CpuPpo(Dims(ad.n_in, ad.n_h, ad.n_out), Dims(cd.n_in, cd.n_h, 1), a0, c0)
    threads, _ = host_threads()
    with threadpool_limits(threads):
        t0 = time.perf_counter()
        cpu.update({k: v.astype(np.float64) for k, v in cols.items()}, order, cfg.clip, cfg.entropy_coef, cfg.vdelta,
                   cfg.minibatch, 1, cfg.target_kl, cfg.kl_scale, int(cfg.kl_mode))
        dt = time.perf_counter() - t0
    pipe = TrainPipeline(ad, cd, rows, cfg.minibatch)
    pipe.set_actor_params(a0)
    pipe.set_critic_params(c0)
    pipe.upload_batch(rows, SampleBatch(**cols))
    pipe.update(order, cfg)
    gaps = {}
    for net, x0, xc, xd in (("actor", a0, cpu.actor, pipe.actor_params()), ("critic", c0, cpu.critic, pipe.critic_params())):
        e = np.abs((xd - x0) - (xc - x0)) / np.abs(xc - x0).max()
        gaps[net] = {"median": float(f"{np.median(e):.3g}"), "p99": float(f"{np.percentile(e, 99):.3g}"),
                     "max": float(f"{e.max():.3g}")}
    base = {"value": round(rows / dt, 1), "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": f"{n_mb} minibatches x {cfg.minibatch} rows, f64 numpy update (tang's arithmetic), "
                      f"{threads} BLAS threads ({dt:.2f} s)",
            "seconds_per_update_extrapolated": round(dt * PPO_SHAPE["samples"] / rows, 2)}
    return base, {"rows": rows, "weight_delta_gap": gaps}


def config_of(w, r):
    from phyz_amd import workloads as W
    c = {"workload": w.name, "config_index": w.index, "nworld": w.nworld, "bodies": w.model.nbodies,
         "nv": w.model.nv, "dt": w.model.dt, "steps_per_launch": r["roofline"]["steps_per_launch"]}
    if w.heightfield is not None:
        h = w.heightfield
        c["heightfield"] = {"nx": h.nx, "ny": h.ny, "cell": h.cell}
    if w.impulse_sweeps > 0:
        c["contact"] = {"mode": "impulse", "sweeps": w.impulse_sweeps}
    if w.model.actuators:
        c["actuators"] = w.model.nu()
    # Joint regularisation the configuration's text does not name (the
    # builder humanoid's hinges carry rotor armature and viscous damping).
    terms = {}
    for key in ("armature", "damping", "stiffness"):
        vals = sorted({round(float(getattr(b.joint, key)), 12) for b in w.model.bodies if b.joint.ndof() == 1})
        if any(x != 0.0 for x in vals):
            terms[f"hinge_{key}"] = vals[0] if len(vals) == 1 else {"min": vals[0], "max": vals[-1]}
    if terms:
        c["joint_terms"] = terms
    if w.index in W.MJCF_WORKLOADS:
        c["file_dt"] = float(W.mjcf_model(W.MJCF_WORKLOADS[w.index][0]).dt)
        c["dt_note"] = "every MJCF workload steps at 1 ms; file_dt is the model file's own timestep"
    return c


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps of the headline workload (default: its rollout length)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warmup steps of the headline workload (default: five timed spans)")
    ap.add_argument("--workload", type=int, default=2, help="headline workload (default 2: chain7)")
    ap.add_argument("--reps", type=int, default=7)
    ap.add_argument("--settle-ms", type=float, default=60.0,
                    help="untimed device time before the headline's warmup, so a short timed span runs at "
                         "steady clocks (0: none)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines and the parity checks")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the measurement of every benchmark configuration at its own rollout length")
    ap.add_argument("--no-control", action="store_true", help="skip the on-device control-loop measurement")
    ap.add_argument("--no-impulse", action="store_true",
                    help="skip the terrain + impulse-contact measurement (workload 6)")
    ap.add_argument("--no-mjcf", action="store_true",
                    help="skip the MJCF-model measurements (workloads 7-9)")
    ap.add_argument("--only", action="store_true", help="measure the headline workload only (profiling runs)")
    ap.add_argument("--control-only", action="store_true", help="measure only the control loop")
    ap.add_argument("--no-ppo", action="store_true", help="skip the PPO update pass measurement")
    ap.add_argument("--no-sweep", action="store_true", help="skip the chain7 world-count sweep")
    ap.add_argument("--sweep-only", action="store_true", help="measure only the chain7 world-count sweep")
    ap.add_argument("--ppo-only", action="store_true", help="measure only the PPO update pass")
    ap.add_argument("--precision", choices=["f32", "f64"], default=None,
                    help="headline precision (default: f32 where the workload runs it)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB five times (HBM counter calibration)")
    args = ap.parse_args()
    if args.calibrate_copy:
        import torch
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "launches": 5}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported (worlds are independent: "
              "a multi-GPU run is N disjoint world ranges, one per GPU).", file=sys.stderr)
        sys.exit(2)

    if args.control_only:
        print(json.dumps(run_control_loop("f32", args.reps, not args.no_cpu)), flush=True)
        return
    if args.ppo_only:
        print(json.dumps(run_ppo_update(args.reps, not args.no_cpu)), flush=True)
        return
    if args.sweep_only:
        print(json.dumps({"world_sweep": run_world_sweep()}), flush=True)
        return

    from phyz_amd import workloads as W
    with_cpu = not args.no_cpu
    w = W.config(args.workload)
    if args.steps is None:
        args.steps = w.nsteps
    if args.warmup is None:
        # Five spans: a freshly idle MI355X takes about five chain7 launches
        # (~20 ms) to reach its steady clocks (rocprof: 4.9, 4.7, 3.5, 3.5,
        # 3.4, then 3.2-3.3 ms per 1000-step launch).
        args.warmup = 5 * args.steps
    prec = args.precision or ("f32" if "f32" in w.precisions else w.precisions[0])

    # ── headline: the workload at the requested span ──
    r = measure(w, [prec], args.steps, args.warmup, args.reps, with_cpu, settle_ms=args.settle_ms)
    p = r["results"][prec]
    line = {
        "metric": METRIC,
        "value": p["value"],
        "unit": "world-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": p["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": prec,
        "data": "synthetic",
        "config": config_of(w, p),
        "roofline": p["roofline"],
        "cpu_baseline": r["cpu"],
        "wall_ms_per_span": p["wall_ms_per_span"],
        "event_ms_per_span": p["event_ms_per_span"],
        "kernel": p["kernel"],
    }
    if "clock_settle" in p:
        line["clock_settle"] = p["clock_settle"]
    if r["cpu"]:
        line["gpu_over_cpu"] = round(p["value"] / r["cpu"]["value"], 1)
    if with_cpu:
        line["parity"] = p["parity"]
    if args.only:
        print(json.dumps(line), flush=True)
        return

    # ── every benchmark configuration at its own rollout length, in each of its precisions ──
    if not args.no_configs:
        line["configs"] = {}
        for idx in W.ALL:
            wc = W.config(idx)
            rc = measure(wc, list(wc.precisions), wc.nsteps, 5 * wc.nsteps, 5, with_cpu)
            entry = {"config": config_of(wc, next(iter(rc["results"].values()))), "cpu_baseline": rc["cpu"]}
            for pr, res in rc["results"].items():
                entry[pr] = {k: res[k] for k in ("value", "unit", "ms_per_step", "world_steps_per_s_event_median",
                                                 "event_ms_per_span", "finite_worlds", "roofline", "kernel", "io")}
                if with_cpu:
                    entry[pr]["parity"] = res["parity"]
                    entry[pr]["gpu_over_cpu"] = round(res["value"] / rc["cpu"]["value"], 1)
            line["configs"][f"{idx}_{wc.name}"] = entry
    if not args.no_impulse and args.workload != 6:
        wi = W.config(6)
        ri = measure(wi, ["f32"], wi.nsteps, wi.nsteps, min(args.reps, 5), with_cpu)
        pi = ri["results"]["f32"]
        line["terrain_impulse"] = {"value": pi["value"], "unit": "world-steps/s", "dtype": "f32",
                                   "ms_per_step": pi["ms_per_step"], "config": config_of(wi, pi),
                                   "roofline": pi["roofline"], "cpu_baseline": ri["cpu"],
                                   "event_ms_per_span": pi["event_ms_per_span"], "kernel": pi["kernel"],
                                   "parity": pi.get("parity")}
    if not args.no_mjcf and args.workload not in W.MJCF_WORKLOADS:
        line["mjcf"] = {}
        for idx in sorted(W.MJCF_WORKLOADS):
            wm = W.config(idx)
            rm = measure(wm, ["f32"], wm.nsteps, wm.nsteps, 3, with_cpu, cpu_budget_s=5.0)
            pm = rm["results"]["f32"]
            # The reference's explicit joint-limit law diverges on these models'
            # lightest links (the oracle diverges identically): the value counts
            # only the worlds still finite after the timed span.
            line["mjcf"][wm.name] = {"value": round(pm["value"] * pm["finite_worlds"], 1), "unit": "world-steps/s",
                                     "value_counts": "worlds finite at the end of the span",
                                     "all_worlds_value": pm["value"], "dtype": "f32",
                                     "finite_worlds": pm["finite_worlds"], "config": config_of(wm, pm),
                                     "roofline": pm["roofline"], "cpu_baseline": rm["cpu"],
                                     "event_ms_per_span": pm["event_ms_per_span"], "kernel": pm["kernel"],
                                     "parity": pm.get("parity")}
    if not args.no_sweep:
        line["world_sweep"] = run_world_sweep()
    if not args.no_control:
        line["control_loop"] = run_control_loop("f32", min(args.reps, 5), with_cpu)
    if not args.no_ppo:
        line["ppo_update"] = run_ppo_update(min(args.reps, 5), with_cpu)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark: world-steps/s of the fused step kernel on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload 2] [--no-cpu]

A "step" is one physics step (control noise, PD, contact, ABA, integrate) of
every world of the workload. The default workload is the 7-link chain, 65536
worlds, f32 and f64 (the f32 run is the headline `value`; the f64 run is
reported under "f64"). W warmup steps run untimed, then exactly K steps are
timed with the device synchronized on both sides; the kernel's own time comes
from hipEvents recorded on the sim's stream around the same span. State stays
resident in HBM for the whole measurement.

roofline: algorithmic FLOPs per launch (tests/golden/flops_per_world_step.json,
counted on the oracle's structure-exploiting formulation x worlds x steps per
launch) over the event-timed launch duration, against MI355X's vector peak
(FP64 78.6 TFLOP/s; FP32 157.3 TFLOP/s published). `traffic` is read from the
committed rocprofv3 --pmc summary when one matches the workload.

cpu_baseline: the f64 CPU oracle (a port of the reference's CPU step), threaded
over worlds on the host cores, timed on a bounded sample of the same workload;
it also checks one device step of the sampled worlds against the oracle.
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


def run_gpu(w, prec, steps, warmup, reps):
    from phyz_amd.sim import from_workload
    sim = from_workload(w, prec, nworld=w.nworld, device=0)
    q, v, c, tg = w.initial_state()
    sim.load_states(q, v, c)
    if tg is not None:
        sim.set_position_targets(tg)
    sim.compile()
    # Warm up with whole spans of the timed length so the timed span replays a
    # captured graph.
    span = steps
    done = 0
    while done < warmup:
        sim.step_many(span)
        done += span
    # Every timed span is the workload's own rollout from its seeded initial
    # state (reloaded untimed), so the state stays on the configured horizon.
    sim.load_states(q, v, c)
    sim.synchronize()
    t0 = time.perf_counter()
    sim.step_many(steps)
    sim.synchronize()
    wall = time.perf_counter() - t0
    ev = []
    for _ in range(reps):  # hipEvents on the sim's stream around each span
        sim.load_states(q, v, c)
        ev.extend(sim.time_step_many(steps, 1))
    sim.load_states(q, v, c)
    sim.step_many(steps)
    info = sim.kernel_info()
    return sim, wall, np.array(ev), info, done


def launches_per_span(steps, info):
    per = max(1, int(info["max_steps_per_launch"]))
    return (steps + per - 1) // per


def roofline(w, prec, steps, ev_ms, info, flops_tab, traffic_tab):
    f = flops_tab[w.name]
    nl = launches_per_span(steps, info)
    steps_per_launch = steps / nl
    flops_per_launch = f["flops_per_world_step"] * w.nworld * steps_per_launch
    launch_s = float(np.median(ev_ms)) / 1e3 / nl
    achieved = flops_per_launch / launch_s / 1e12
    traffic = None
    key = f"{w.name}_{prec}_{int(steps_per_launch)}"
    if traffic_tab and key in traffic_tab:
        traffic = traffic_tab[key]["hbm_bytes_per_launch"]
    algo_bytes = f["bytes_per_world_step"][prec] * w.nworld  # one state round trip per launch
    return {
        "bound": "valu",
        "achieved": round(achieved, 4),
        "peak": PEAK_TFLOPS[prec],
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_TFLOPS[prec], 5),
        "traffic": traffic,
        "flops_per_world_step": f["flops_per_world_step"],
        "launch_ms": round(launch_s * 1e3, 4),
        "steps_per_launch": int(steps_per_launch),
        "hbm_frac": round(algo_bytes / launch_s / 1e9 / HBM_PEAK_GBS, 6),
    }


def cpu_baseline(w, sim, prec, budget_s=20.0):
    """Oracle (f64 port of the reference CPU step) on the host cores, on a bounded
    sample of the workload; plus a one-step parity check of the sampled worlds."""
    from tests.helpers import as_precision, oracle_for, rel_err_rows
    threads = max(1, min(16, os.cpu_count() or 1))
    orc = oracle_for(w)
    # Parity: one more device step from the benchmark's late states, sampled worlds.
    qg, vg = sim.readback_states()
    sim.step()
    ctrl = as_precision(sim.readback_controls(), prec)
    qdd = sim.readback_qdd()
    idx = np.linspace(0, w.nworld - 1, 64).astype(int)
    ext = [orc.contact(qg[k], vg[k])[0] if w.contact is not None else None for k in idx]
    want = np.stack([orc.aba(qg[k], vg[k], ctrl[k], ext[i]) for i, k in enumerate(idx)])
    err = float(rel_err_rows(qdd[idx], want).max())
    # Timing: the same workload's initial states, n worlds x s steps within the budget.
    n = min(w.nworld, 4096)
    q, v, c, tg = w.initial_state(n)
    rng = orc.rng_states(n)
    t0 = time.perf_counter()
    orc.step_batch(q, v, c, 2, targets=tg, rng=rng, threads=threads)
    probe = time.perf_counter() - t0
    rate = 2 * n / max(probe, 1e-6)
    s = max(2, int(budget_s * rate / n))
    q, v, c, tg = w.initial_state(n)
    rng = orc.rng_states(n)
    t0 = time.perf_counter()
    orc.step_batch(q, v, c, s, targets=tg, rng=rng, threads=threads)
    dt = time.perf_counter() - t0
    n1 = min(n, 256)
    q1, v1, c1, tg1 = w.initial_state(n1)
    t1 = time.perf_counter()
    orc.step_batch(q1, v1, c1, max(2, s // 16), targets=tg1, rng=orc.rng_states(n1), threads=1)
    dt1 = time.perf_counter() - t1
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(n * s / dt, 1),
        "unit": "world-steps/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{w.name}: first {n} worlds x {s} steps, f64 oracle, {threads} threads ({dt:.1f} s)",
        "single_thread_value": round(n1 * max(2, s // 16) / dt1, 1),
        "cpu": cpu_model,
    }, {"worlds_checked": len(idx), "qdd_rel_err_max": err}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default: the workload's rollout length)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed warmup steps (default: one timed span)")
    ap.add_argument("--workload", type=int, default=2)
    ap.add_argument("--reps", type=int, default=7)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--precision", choices=["f32", "f64"], default=None, help="run one precision only")
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

    from phyz_amd import workloads as W
    w = W.config(args.workload)
    if args.steps is None:
        args.steps = w.nsteps
    if args.warmup is None:
        args.warmup = args.steps
    flops_tab = json.load(open(FLOPS_JSON))
    traffic_tab = json.load(open(TRAFFIC_JSON)) if os.path.exists(TRAFFIC_JSON) else None
    precs = [args.precision] if args.precision else list(w.precisions)
    primary = "f32" if "f32" in precs else precs[0]
    results = {}
    sims = {}
    for prec in precs:
        log(f"[bench] {w.name} {prec}: {w.nworld} worlds, warmup {args.warmup}, timed {args.steps} steps")
        sim, wall, ev, info, warm_done = run_gpu(w, prec, args.steps, args.warmup, args.reps)
        sims[prec] = sim
        ws = w.nworld * args.steps / wall
        med = float(np.median(ev))
        spread = (max(ev) - min(ev)) / med if med > 0 else 0.0
        results[prec] = {
            "value": round(ws, 1),
            "ms_per_step": round(wall * 1e3 / args.steps, 6),
            "event_ms_per_span": {"median": round(med, 4), "min": round(float(min(ev)), 4),
                                  "max": round(float(max(ev)), 4), "reps": len(ev), "noisy": bool(spread > 0.25)},
            "world_steps_per_s_event_median": round(w.nworld * args.steps / (med / 1e3), 1),
            "roofline": roofline(w, prec, args.steps, ev, info, flops_tab, traffic_tab),
            "kernel": info,
            "warmup_steps_run": warm_done,
        }
        log(f"[bench] {prec}: {ws:.4g} world-steps/s, {results[prec]['roofline']['achieved']:.3f} TFLOP/s "
            f"({100 * results[prec]['roofline']['frac']:.2f}% of peak)")
    cpu = None
    parity = {}
    if not args.no_cpu:
        for prec in precs:
            log(f"[bench] cpu_baseline + parity check ({prec})")
            c, p = cpu_baseline(w, sims[prec], prec)
            parity[prec] = p
            if prec == primary:
                cpu = c
    r = results[primary]
    line = {
        "metric": METRIC,
        "value": r["value"],
        "unit": "world-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": primary,
        "data": "synthetic",
        "config": {"workload": w.name, "config_index": w.index, "nworld": w.nworld, "bodies": w.model.nbodies,
                   "nv": w.model.nv, "dt": w.model.dt, "steps_per_launch": r["roofline"]["steps_per_launch"]},
        "roofline": r["roofline"],
        "cpu_baseline": cpu,
        "event_ms_per_span": r["event_ms_per_span"],
        "kernel": r["kernel"],
    }
    if cpu:
        line["gpu_over_cpu"] = round(r["value"] / cpu["value"], 1)
    for prec in precs:
        if prec != primary:
            line[prec] = results[prec]
    if parity:
        line["parity"] = parity
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark of the NR uplink engine hot path on one MI355X: robot-slots/s of the RL-scale workload.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--out-format reference|compact] [--no-cpu]
    python bench.py --workload wifi_dcf [--envs-per-wave G]     (level WIFI: station-substeps/s)
    python bench.py --workload wifi_dcf_slots [--envs-per-wave G]  (level WIFI_DCF: station-steps/s)
    python bench.py --workload mc_interf     (three cells with UL interference, 1024 envs x 64 robots: robot-slots/s)
    python bench.py --workload freq_sel      (16384 envs x 128 robots, 273 PRB in 8 RBGs, K = 20: robot-slots/s)
    python bench.py --summarize-counters DIR KERNEL NAME   (rocprofv3 --pmc CSVs under DIR -> profiles/NAME.json)
    python bench.py --phase-clocks [...]     (loads libinet_nr_phase.so, built by isaac-net_amd/build.py
                                              --phase-clocks, and adds the step kernel's per-phase clocks of the last
                                              launch to the line; its timings are not the product library's)

A step is one control step of every env: this step's message arrivals and step (poses in, the reference's output dict
out), one launch of the fused step kernel that enqueues the arrivals first (--separate-submit: submit_counts and step,
two launches; --graph: both replayed from HIP graphs recorded after the warm-up). Inputs (poses and arrival counts of every
step) are generated before the timed region and are resident in HBM. The timed region is K steps bracketed by
torch.cuda.synchronize(); value = E * R * K_ul * K / seconds (robot-slots/s, K_ul = 10 UL slots per step).
The step kernel's average duration is measured live with HIP events recorded around each launch on the launch
stream (the engine's kernel_events hook); roofline.achieved is the kernel's algorithmic HBM bytes per launch (the
canonical compact layout's bytes per robot-step times the robots: 2,362 B at the RL-scale shape) over that duration.
The bytes of this engine's own layout (reference output dtypes, the whole FIFO) and the bytes touched at the measured
queue occupancy are reported beside it; roofline.traffic (rocprofv3 FETCH_SIZE + WRITE_SIZE) and valu_issue_util
(SQ_INSTS_VALU) come from the counter summary under profiles/ recorded on the loaded library's sources, else null. The CPU baseline times the oracle (a torch-CPU restatement of the reference path) on the first envs of the
same workload.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "robot-slots/sec @4096 envs×32 robots K=10; achieved HBM GB/s vs peak"
PEAK_GBS = 8000.0


def load_package():
    if "isaac_net_amd" in sys.modules:
        return sys.modules["isaac_net_amd"]
    d = os.path.join(ROOT, "isaac-net_amd")
    spec = importlib.util.spec_from_file_location("isaac_net_amd", os.path.join(d, "__init__.py"),
                                                  submodule_search_locations=[d])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["isaac_net_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def canonical_bytes_per_robot_step(eng):
    """The algorithmic bytes of one robot-step in the canonical compact layout (each state word at its smallest
    width, the FIFO at 18 B per frame): 2 B_rw + B_ro + B_in + B_out with B_rw = 12 S + 32 + 32 P + 18 F (fading and CSI, MAC scalars, HARQ processes,
    frame FIFO, read and written once), B_ro = 8 (Rician phasor), B_in = 10 (pose and arrivals) and B_out = 9 F + 16.
    2,362 B at S = 13, P = 8, F = 32."""
    S, P, F = eng.S, eng.P, eng.F
    return 2 * (12 * S + 32 + 32 * P + 18 * F) + 8 + 10 + 9 * F + 16


def counter_summary(name):
    """The rocprofv3 counter summary profiles/<name>.json if it was recorded on this library's sources (its "src"
    equals the hash the loaded library was built from), else None."""
    from isaac_net_amd import _lib
    path = os.path.join(ROOT, "profiles", name + ".json")
    if not name or not os.path.exists(path):
        return None
    d = json.load(open(path))
    built = _lib.load().inet_nr_build_info().decode().rsplit("src=", 1)[-1]
    return d if d.get("src") == built else None


def measured_fields(name, k_avg_ms):
    """roofline fields from the counter summary profiles/<name>.json recorded on the loaded library's sources:
    traffic (HBM bytes per launch, rocprofv3 FETCH_SIZE + WRITE_SIZE scaled by a copy-kernel calibration),
    valu_issue_util (a wave64 VALU instruction occupies a 16-lane SIMD for 4 cycles; 1024 SIMDs at 2.4 GHz, over the
    kernel's measured duration) and the summary's source hash; all null when there is no such summary."""
    cs = counter_summary(name)
    if not cs:
        return {"traffic": None, "valu_issue_util": None, "counters_src": None}
    valu = cs.get("valu_insts_per_dispatch")
    return {"traffic": cs.get("bytes_per_launch"),
            "valu_issue_util": valu * 4 / (1024 * k_avg_ms * 1e-3 * 2.4e9) if valu else None,
            "counters_src": cs.get("src")}


def step_kernel_bytes(eng):
    """Algorithmic HBM bytes of one step-kernel launch: per robot-step 2 B_rw + B_ro + B_in + B_out over this
    engine's state layout (every per-robot state word read and written once, the whole frame FIFO included),
    plus the per-env words (RNG key and counters, epoch, shadowing field, per-env counters and histograms)."""
    cfg, E, R, S, P, F = eng.config, eng.E, eng.R, eng.S, eng.P, eng.F
    p = eng._cparams
    b_rw = 9 * 4 + S * 4 + P * 6 * 4 + F * 6 * 4           # MAC scalars, CSI, HARQ processes, FIFO frames
    if cfg.fading:
        b_rw += 2 * S * 4                                   # fading state
    if p.comb == 2:
        b_rw += 2 * P * 4                                   # IR log-sum and PRB count
    b_ro = 3 * 4 if p.rician else 0                         # Rician phasor and K
    b_in = 8                                                # pose
    if p.out_ref:
        b_out = F * (3 + 8 + 8 + 4) + 8 + 8 + 8 + 4 + 4     # delivered/timed/dropped, cap, cls, delay; per robot
    else:
        b_out = F * (1 + 4 + 1 + 4) + 8 + 8 + 4 + 4
    per_env = 5 * 4 + p.n_fields * p.n_modes * 3 * 4 + 2 * 8 * 10 + 2 * 8 * 3 * (cfg.max_harq_tx + 1) + 9
    per_robot = 2 * b_rw + b_ro + b_in + b_out
    return E * R * per_robot + E * per_env, per_robot


def dl_step_kernel_bytes(eng):
    """Algorithmic HBM bytes of one DL step-kernel launch: per robot-step the DL link's state read and written once
    (MAC scalars, CSI, HARQ processes, the DL frame FIFO of 5 words per frame, dl_newest), the shared state it only
    reads (fading state, Rician phasor and K), the pose, and the outputs dl_newest / dl_queue_len; plus the per-env
    words (RNG key, epoch, shadowing field, DL counters and histograms)."""
    cfg, E, R, S, P, F = eng.config, eng.E, eng.R, eng.S, eng.P, eng.F
    p = eng._cparams
    b_rw = 8 * 4 + S * 4 + P * 6 * 4 + F * 5 * 4          # MAC scalars + dl_newest, CSI, HARQ processes, frames
    if p.comb == 2:
        b_rw += 2 * P * 4
    b_ro = (2 * S * 4 if cfg.fading else 0) + (3 * 4 if p.rician else 0)
    per_robot = 2 * b_rw + b_ro + 8 + 2 * 8
    per_env = 4 * 4 + p.n_fields * p.n_modes * 3 * 4 + 2 * 8 * 10 + 2 * 8 * 3 * (cfg.max_harq_tx + 1)
    return E * R * per_robot + E * per_env, per_robot


def mc_step_kernel_bytes(eng):
    """Algorithmic HBM bytes of one multi-cell step-kernel launch (inet_nr_step_cells): step_kernel_bytes with the
    fading state of every robot-cell link (2 C S floats instead of 2 S) and the association words (serving cell, A3
    candidate and count, interruption end, handover count: 5 int32) read and written, the shadowing fields of every
    cell; per env each gNB's N+I estimate (C S floats), the I/N statistic and the pending flag, read and written."""
    total, per_robot = step_kernel_bytes(eng)
    C, S, E, R = eng.C, eng.S, eng.E, eng.R
    p = eng._cparams
    extra_robot = 2 * (2 * (C - 1) * S * 4) + 2 * 5 * 4
    extra_env = (C - 1) * p.n_fields * p.n_modes * 3 * 4 + 2 * (C * S * 4 + 4 + 4)
    return total + E * R * extra_robot + E * extra_env, per_robot + extra_robot


def step_kernel_touched_bytes(eng, qlen_mean, kept_mean):
    """HBM bytes the kernel actually moves for the measured queue occupancy: the frame FIFO is touched only up to
    each robot's queue length (qlen_mean frames read, kept_mean rewritten), everything else as in step_kernel_bytes."""
    total, per_robot = step_kernel_bytes(eng)
    F = eng.F
    fifo_full = 2 * F * 6 * 4
    fifo_touched = qlen_mean * 6 * 4 + kept_mean * 6 * 4
    return total - eng.E * eng.R * (fifo_full - fifo_touched)


def copy_calibration(args, res, torch, dev):
    """--copy-mib: copy a buffer of known size three times after the run (the byte counters' calibration kernel)."""
    if args.copy_mib > 0:
        src = torch.ones(args.copy_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        res["copy_calibration_bytes"] = 2 * src.numel()


def wifi_step_bytes(eng, n_cls):
    """Algorithmic HBM bytes of one Wi-Fi step-kernel launch: per station-step the frame FIFO (F slots of cap, cls,
    det, hid, rem, f_nact, f_snr, f_own = 29 B) and the per-station words (queue length, last SNR, roaming, serving AP,
    contention count, log-failure sum, credit, tau = 32 B) read and written once, the pose (8 B), the [E,R,F] outputs
    (delivered, timed out, cap, cls, delay = 22 B per slot) and the per-station outputs (4 int64 + 6 float32 = 56 B);
    per env the background station's tau, clock, hazard id, RNG key and counters and the shadowing field. The step's
    enqueue adds the arrival counts (n_cls B) and accepted messages (4 B) per station and the env's submit counter."""
    p = eng._cparams
    F = eng.F
    per_robot = 2 * (F * 29 + 32) + 8 + F * 22 + 56 + n_cls + 4
    per_env = 2 * (4 + 8 + 8 + 1 + 4 * 4) + p.n_fields * p.n_modes * 3 * 4 + 2 * 4
    return eng.E * eng.R * per_robot + eng.E * per_env, per_robot


def dcf_step_bytes(eng, n_cls):
    """Algorithmic HBM bytes of one WIFI_DCF step-kernel launch: per station-step the frame FIFO (29 B per slot) read
    and written once, the queue length (read and written), last SNR and serving AP (written), the backoff counter,
    retry stage and contention flag (9 B, read and written), the pose (8 B), the [E,R,F] outputs (22 B per slot) and
    the per-station outputs (56 B); per env the clock, step counter and idle anchor (read and written), the hazard id,
    RNG key, episode, pending flag, det_env and t, and the shadowing field. The step's enqueue adds the arrival counts
    (n_cls B) and accepted messages (4 B) per station and the env's submit counter."""
    p = eng._cparams
    F = eng.F
    per_robot = 2 * F * 29 + 8 + 4 + 4 + 2 * 9 + 8 + F * 22 + 56 + n_cls + 4
    per_env = 2 * (8 + 4 + 4) + 8 + 4 + 4 + 1 + 1 + 8 + p.n_fields * p.n_modes * 3 * 4 + 2 * 4
    return eng.E * eng.R * per_robot + eng.E * per_env, per_robot


def wifi_cpu_baseline(wl, cfg, E_cpu, steps, warmup, slots=False):
    import torch

    from oracle.dcf_oracle import DcfOracle
    from oracle.wifi_oracle import WifiOracle
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    R = wl.R
    ora = (DcfOracle if slots else WifiOracle)(E_cpu, R, cfg, seed=0)
    poses = wl.poses[:, :E_cpu].cpu()
    counts = wl.counts[:, :E_cpu].cpu().numpy()

    def one(s):
        c = counts[s]
        for ci in range(c.shape[-1]):
            for i in range(int(c[..., ci].max())):
                ora.submit(None, torch.from_numpy((c[..., ci] > i).astype("int64") * (ci + 1)))
        ora.step(None, poses[s])
    for s in range(warmup):
        one(s)
    t0 = time.perf_counter()
    for s in range(warmup, warmup + steps):
        one(s)
    dt = time.perf_counter() - t0
    if slots:
        att = int(ora.tot["att"].sum())
        return {"value": E_cpu * R * steps / dt, "unit": "station-steps/s", "cores": threads, "kind": "port",
                "sample": f"oracle (per-env event loop in numpy) on the first {E_cpu} of the {wl.E} envs x {R} "
                          f"stations, {steps} timed steps after {warmup} warm-up, {dt:.1f} s",
                "ms_per_step": 1e3 * dt / steps, "attempts_per_env_step": att / (E_cpu * (steps + warmup))}
    return {"value": E_cpu * R * ora.K * steps / dt, "unit": "station-substeps/s", "cores": threads, "kind": "port",
            "sample": f"oracle (torch CPU restatement of the reference WifiNet) on the first {E_cpu} of the "
                      f"{wl.E} envs x {R} stations, {steps} timed steps after {warmup} warm-up, {dt:.1f} s",
            "ms_per_step": 1e3 * dt / steps}


def run_wifi(args, P, torch):
    """The Wi-Fi workloads: level WIFI (station-substeps/s) or level WIFI_DCF (station-steps/s), one line with the
    step kernel's roofline fields."""
    from isaac_net_amd import scenarios as S
    slots = args.workload == "wifi_dcf_slots"
    dev = "cuda:0"
    E = args.envs if args.envs_set else 2048
    R = args.robots if args.robots_set else 16
    n_graph = 0 if args.no_graph_window else args.steps
    total = args.warmup + args.steps + (n_graph + 2 if n_graph else 0)
    print(f"# workload {args.workload} {E}x{R}, {total} steps of inputs", file=sys.stderr, flush=True)
    wl = S.Workload(E, R, total, seed=0, device=dev, name=args.workload)
    cfg = wl.cfg
    from isaac_net_amd.engine import KernelTimer
    from isaac_net_amd.wifi_engine import HipWifiDcfEngine, HipWifiEngine
    eng = (HipWifiDcfEngine if slots else HipWifiEngine)(E, R, dev, cfg, seed=0, envs_per_wave=args.envs_per_wave)
    eng.static_outputs = True       # every step writes the same output tensors (the reference graph backend's form)
    K = eng.K
    # one launch per control step: the step enqueues the step's arrival counts itself (step(counts=), the same state
    # as submit_counts + step)
    for s in range(args.warmup):
        eng.step(None, wl.poses[s], counts=wl.counts[s])
    torch.cuda.synchronize()
    eng.kernel_events = ev = KernelTimer(args.steps, dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        s = args.warmup + i
        eng.step(None, wl.poses[s], counts=wl.counts[s])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    eng.kernel_events = None
    # At this size the host loop is slower than the GPU, so an event pair recorded in the timed loop also holds the
    # idle gap before its launch. The kernel durations come from the same launches queued behind a GPU spin: the
    # spin outlasts the host's enqueueing, and each event pair then brackets its kernel alone.
    eng.kernel_events = ev = KernelTimer(args.steps, dev)
    torch.cuda._sleep(int(2e6 + 4e5 * args.steps))
    for i in range(args.steps):
        s = args.warmup + i
        eng.step(None, wl.poses[s], counts=wl.counts[s])
    torch.cuda.synchronize()
    eng.kernel_events = None
    k_ms = sorted(ev.ms())
    k_avg = sum(k_ms) / len(k_ms)
    nbytes, per_robot = (dcf_step_bytes if slots else wifi_step_bytes)(eng, wl.counts.shape[-1])
    achieved = nbytes / (k_avg * 1e-3) / 1e9
    if slots:
        metric, value, unit = (f"station-steps/sec @{E} envs×{R} stations (level WIFI_DCF, per-slot CSMA/CA)",
                               E * R * args.steps / dt, "station-steps/s")
    else:
        metric, value, unit = (f"station-substeps/sec @{E} envs×{R} stations K={K} (level WIFI, DCF)",
                               E * R * K * args.steps / dt, "station-substeps/s")
    res = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": 1e3 * dt / args.steps, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
           "config": {"workload": f"{args.workload}: {E} envs x {R} stations at one AP, DCF (CWmin 15, CWmax 1023, "
                                  "7 attempts), 802.11ax 20 MHz 12 MCS, "
                                  + ("per-slot CSMA/CA over the 20 ms step" if slots else f"K={K} sub-steps of 1 ms")
                                  + ", 1500 B @0.4 per station-step, FIFO 16, 50 m disc, log-distance + shadowing",
                      "envs": E, "stations": R, "substeps_per_step": K, "envs_per_wave": args.envs_per_wave,
                      "parallelism": "single GPU",
                      "launch": "eager, one launch per step (the enqueue in the step kernel), static output "
                                "buffers overwritten by every step (as the reference's graph backend returns them)"},
           "env_steps_per_s": E * args.steps / dt,
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s",
                        "frac": achieved / PEAK_GBS, "kernel": "wifi_step_kernel",
                        "kernel_ms_avg": k_avg, "kernel_ms_median": k_ms[len(k_ms) // 2],
                        **measured_fields(f"wifi_step_kernel_counters_{args.workload}_epw{args.envs_per_wave}"
                                          if (E, R) == (2048, 16) else "", k_avg),
                        "kernel_timing": "HIP events around each launch on the launch stream, the timed loop's "
                                         "launches repeated behind a GPU spin",
                        "algorithmic_bytes_per_launch": nbytes, "algorithmic_bytes_per_station_step": per_robot}}
    if n_graph:
        # the next n_graph steps as replays of the recorded graph (counts-form enqueue + step), after the timed eager
        # steps and the spin-timed repeat of their launches; the first two replays (recording) are not timed
        g = eng.graph_step()
        base = args.warmup + args.steps
        for s in range(base, base + 2):
            g(wl.poses[s], wl.counts[s])
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for s in range(base + 2, base + 2 + n_graph):
            g(wl.poses[s], wl.counts[s])
        torch.cuda.synchronize()
        gms = 1e3 * (time.perf_counter() - t1) / n_graph
        # the same replays with the inputs left in the graph's buffers (a producer writing them in place)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(n_graph):
            g.replay(0)
        torch.cuda.synchronize()
        bms = 1e3 * (time.perf_counter() - t1) / n_graph
        res["graph_replay"] = {"ms_per_step": gms, "steps": n_graph, "wall_over_kernel": gms / k_avg,
                               "launch": "HIP graph replay of the step with its enqueue (one kernel node), the inputs "
                                         "copied into the graph's buffers first",
                               "in_place_ms_per_step": bms, "in_place_wall_over_kernel": bms / k_avg}
    copy_calibration(args, res, torch, dev)
    if not args.no_cpu:
        print("# cpu baseline (oracle)", file=sys.stderr, flush=True)
        res["cpu_baseline"] = wifi_cpu_baseline(wl, cfg, min(args.cpu_envs, E), args.cpu_steps, 1, slots=slots)
    print(json.dumps(res), flush=True)


def cpu_baseline(P, wl, cfg, E_cpu, steps, warmup):
    import torch

    from oracle import nr_oracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    R = wl.R
    ora = O.OracleEngine(E_cpu, R, cfg, seed=0)
    poses = wl.poses[:, :E_cpu].cpu()
    counts = wl.counts[:, :E_cpu].cpu().numpy()
    dl_bytes = None if wl.dl_bytes is None else wl.dl_bytes[:, :, :E_cpu].cpu()

    def one(s):
        c = counts[s]
        for ci in range(c.shape[-1]):
            for i in range(int(c[..., ci].max())):
                ora.submit(None, torch.from_numpy((c[..., ci] > i).astype("int64") * (ci + 1)))
        if dl_bytes is not None:
            for i in range(dl_bytes.shape[1]):
                ora.add_dl_frames(None, dl_bytes[s, i])
        ora.step(None, poses[s])
    for s in range(warmup):
        one(s)
    t0 = time.perf_counter()
    for s in range(warmup, warmup + steps):
        one(s)
    dt = time.perf_counter() - t0
    k_ul = sum(1 for x in cfg.schedule(0) if x[2]) + sum(1 for x in cfg.schedule(0) if x[1])
    return {"value": E_cpu * R * k_ul * steps / dt, "unit": "robot-slots/s", "cores": threads, "kind": "port",
            "sample": f"oracle (torch CPU restatement of the reference path) on the first {E_cpu} of the {wl.E} envs "
                      f"x {R} robots, {steps} timed steps after {warmup} warm-up, {dt:.1f} s",
            "ms_per_step": 1e3 * dt / steps}


def run_dl(args, P, torch):
    """The RL-scale workload with the downlink on: one line with robot-slots/s over the UL and DL data slots and the
    roofline fields of the slower of the two step kernels (both are reported)."""
    from isaac_net_amd import scenarios as S
    from isaac_net_amd.engine import KernelTimer
    dev = "cuda:0"
    E = args.envs if args.envs_set else 4096
    R = args.robots if args.robots_set else 32
    total = args.warmup + args.steps
    print(f"# workload rl_scale_dl {E}x{R}, {total} steps of inputs", file=sys.stderr, flush=True)
    wl = S.Workload(E, R, total, seed=0, device=dev, name="rl_scale_dl")
    cfg = wl.cfg
    eng = P.make_engine("L2", E, R, dev, cfg, seed=0, out_format=args.out_format)
    sched = cfg.schedule(0)
    k_ul, k_dl = sum(1 for x in sched if x[2]), sum(1 for x in sched if x[1])

    def one(s):
        for i in range(wl.dl_bytes.shape[1]):
            eng.add_dl_frames(None, wl.dl_bytes[s, i])
        eng.step(None, wl.poses[s], arrivals=wl.counts[s])
    for s in range(args.warmup):
        one(s)
    torch.cuda.synchronize()
    eng.kernel_events, eng.dl_kernel_events = KernelTimer(args.steps, dev), KernelTimer(args.steps, dev)
    ev_ul, ev_dl = eng.kernel_events, eng.dl_kernel_events
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        one(args.warmup + i)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    eng.kernel_events = eng.dl_kernel_events = None
    ms = {}
    for name, ev, fn in (("nr_step_kernel", ev_ul, step_kernel_bytes), ("nr_step_kernel<dl>", ev_dl,
                                                                       dl_step_kernel_bytes)):
        k = sorted(ev.ms())
        avg = sum(k) / len(k)
        nb, per_robot = fn(eng)
        extra = {}
        if fn is step_kernel_bytes:                         # the UL kernel: the canonical bytes, as rl_scale's line
            extra = {"layout_bytes_per_launch": nb, "layout_bytes_per_robot_step": per_robot}
            per_robot = canonical_bytes_per_robot_step(eng)
            nb = E * R * per_robot
        ach = nb / (avg * 1e-3) / 1e9
        tag = "nr_step_kernel_counters_rl_scale_dl_" + ("ul" if fn is step_kernel_bytes else "dl")
        meas = measured_fields(tag, avg) if (E, R) == (4096, 32) and args.out_format == "reference" else \
            measured_fields("", avg)
        ms[name] = {"bound": "hbm", "achieved": ach, "peak": PEAK_GBS, "unit": "GB/s", "frac": ach / PEAK_GBS,
                    "kernel": name, "kernel_ms_avg": avg, "kernel_ms_median": k[len(k) // 2],
                    "algorithmic_bytes_per_launch": nb, "algorithmic_bytes_per_robot_step": per_robot, **extra,
                    **meas}
    dom = max(ms.values(), key=lambda r: r["kernel_ms_avg"])
    c = eng.counters()
    res = {"metric": f"robot-slots/sec (UL + DL data slots) @{E} envs×{R} robots K_ul={k_ul} K_dl={k_dl}",
           "value": E * R * (k_ul + k_dl) * args.steps / dt, "unit": "robot-slots/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": 1e3 * dt / args.steps,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
           "config": {"workload": f"rl_scale_dl: rl_scale ({E} envs x {R} robots, DDDSU at 25 ms, 52 PRB, PF, 8 HARQ, "
                                  f"Rician K 3 dB, UMi LOS) with the downlink: {k_dl} DL data slots and CQI every 10 "
                                  "slots, 2000 B DL messages at Poisson 0.5 per robot-step",
                      "envs": E, "robots": R, "ul_slots_per_step": k_ul, "dl_slots_per_step": k_dl,
                      "parallelism": "single GPU", "out_format": args.out_format, "launch": "eager"},
           "env_steps_per_s": E * args.steps / dt,
           "roofline": dom, "kernels": ms,
           "dl_tb_per_robot_step": c["dl"]["tb_new"] / (E * R * (args.warmup + args.steps))}
    copy_calibration(args, res, torch, dev)
    if not args.no_cpu:
        print("# cpu baseline (oracle)", file=sys.stderr, flush=True)
        # the oracle runs 40 DL and 10 UL data slots per step: a smaller sample keeps it to about 15 s
        res["cpu_baseline"] = cpu_baseline(P, wl, cfg, min(args.cpu_envs, 256), min(args.cpu_steps, 4), 1)
    print(json.dumps(res), flush=True)


def run_mc(args, P, torch):
    """Config 3: three cells per env with same-slot UL interference (NRNet.step_cells), one line with robot-slots/s
    and the step kernel's measured duration against its algorithmic HBM bytes. The kernel is bound by its per-lane
    arithmetic (the fading draws and gains of 3 links per robot, the per-cell schedulers and the interference sums),
    not by HBM: roofline.frac says how far from the HBM bound it runs."""
    from isaac_net_amd import scenarios as S
    from isaac_net_amd.engine import KernelTimer
    dev = "cuda:0"
    E = args.envs if args.envs_set else 1024
    R = args.robots if args.robots_set else 64
    total = args.warmup + args.steps
    print(f"# workload mc_interf {E}x{R}, {total} steps of inputs", file=sys.stderr, flush=True)
    wl = S.Workload(E, R, total, seed=0, device=dev, name="mc_interf")
    cfg = wl.cfg
    eng = P.make_engine("L2", E, R, dev, cfg, seed=0, out_format=args.out_format)
    k_ul = sum(1 for x in cfg.schedule(0) if x[2])
    for s in range(args.warmup):
        eng.step(None, wl.poses[s], arrivals=wl.counts[s])
    torch.cuda.synchronize()
    eng.kernel_events = ev = KernelTimer(args.steps, dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        s = args.warmup + i
        eng.step(None, wl.poses[s], arrivals=wl.counts[s])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    eng.kernel_events = None
    k_ms = sorted(ev.ms())
    k_avg = sum(k_ms) / len(k_ms)
    nbytes, per_robot = mc_step_kernel_bytes(eng)
    achieved = nbytes / (k_avg * 1e-3) / 1e9
    st = eng.owner_state()
    noise = 10 ** (cfg.noise_dbm_per_prb("gnb") / 10)
    res = {"metric": f"robot-slots/sec @{E} envs×{R} robots K={k_ul}, 3 cells with UL interference",
           "value": E * R * k_ul * args.steps / dt, "unit": "robot-slots/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": 1e3 * dt / args.steps, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
           "config": {"workload": f"mc_interf: {E} envs x {R} robots, 3 hex cells 150 m apart, nearest-gNB "
                                  "association, no handover, thermal noise + same-slot UL interference of the other "
                                  f"cells' scheduled robots, fractional UL power control, PF over 106 PRB (14 RBGs), "
                                  f"K={k_ul} UL slots/step (DDDSU, 25 ms), 1200 B at Poisson 0.3, FIFO 16, UMi LOS",
                      "envs": E, "robots": R, "cells": 3, "ul_slots_per_step": k_ul, "parallelism": "single GPU",
                      "out_format": args.out_format, "launch": "eager: one launch per step (arrivals enqueued "
                                                               "inside the step kernel)"},
           "env_steps_per_s": E * args.steps / dt,
           "mean_interference_over_thermal_db": float(10 * torch.log10((st["net.ni_ul"] / noise).mean())),
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s",
                        "frac": achieved / PEAK_GBS, "kernel": "nr_step_kernel<cells 3>",
                        "kernel_ms_avg": k_avg, "kernel_ms_median": k_ms[len(k_ms) // 2],
                        "algorithmic_bytes_per_launch": nbytes, "algorithmic_bytes_per_robot_step": per_robot,
                        **measured_fields("nr_step_kernel_counters_mc_interf" if (E, R) == (1024, 64) and
                                          args.out_format == "reference" else "", k_avg),
                        "note": "arithmetic-bound kernel: frac is the distance from the HBM bound"}}
    if args.phase_clocks:
        rb = 1 << (R - 1).bit_length()                   # robots per segment: the next power of two
        res["phase_clocks"] = phase_clocks("mc", (E * rb + 63) // 64)
    copy_calibration(args, res, torch, dev)
    if not args.no_cpu:
        print("# cpu baseline (oracle)", file=sys.stderr, flush=True)
        res["cpu_baseline"] = cpu_baseline(P, wl, cfg, min(args.cpu_envs, 512), min(args.cpu_steps, 4), 1)
    print(json.dumps(res), flush=True)


def run_freq_sel(args, P, torch):
    """Config 5: 16384 envs x 128 robots (two wavefronts per env), 273 PRB in 8 RBGs, i.i.d. Rayleigh per subband,
    PF, K = 20: one line with robot-slots/s and the step kernel's measured duration against its algorithmic bytes."""
    from isaac_net_amd import scenarios as S
    from isaac_net_amd.engine import KernelTimer
    dev = "cuda:0"
    E = args.envs if args.envs_set else 16384
    R = args.robots if args.robots_set else 128
    total = args.warmup + args.steps
    print(f"# workload freq_sel {E}x{R}, {total} steps of inputs", file=sys.stderr, flush=True)
    wl = S.Workload(E, R, total, seed=0, device=dev, name="freq_sel")
    cfg = wl.cfg
    eng = P.make_engine("L2", E, R, dev, cfg, seed=0, out_format=args.out_format)
    k_ul = sum(1 for x in cfg.schedule(0) if x[2])
    for s in range(args.warmup):
        eng.step(None, wl.poses[s], arrivals=wl.counts[s])
    torch.cuda.synchronize()
    eng.kernel_events = ev = KernelTimer(args.steps, dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        s = args.warmup + i
        eng.step(None, wl.poses[s], arrivals=wl.counts[s])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    eng.kernel_events = None
    k_ms = sorted(ev.ms())
    k_avg = sum(k_ms) / len(k_ms)
    layout_bytes, layout_per_robot = step_kernel_bytes(eng)
    per_robot = canonical_bytes_per_robot_step(eng)
    nbytes = E * R * per_robot
    achieved = nbytes / (k_avg * 1e-3) / 1e9
    res = {"metric": f"robot-slots/sec @{E} envs×{R} robots K={k_ul}, 273 PRB in 8 RBGs",
           "value": E * R * k_ul * args.steps / dt, "unit": "robot-slots/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": 1e3 * dt / args.steps, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
           "config": {"workload": f"freq_sel: {E} envs x {R} robots (two wavefronts per env), one cell, 273 PRB "
                                  f"(100 MHz at 30 kHz) in 8 RBGs of 35, i.i.d. Rayleigh per subband and slot, PF, "
                                  f"K={k_ul} UL slots/step (DDDSU, 50 ms), 8 HARQ x 4 tx, 800 B at Poisson 0.2, "
                                  "FIFO 16, UMi LOS",
                      "envs": E, "robots": R, "ul_slots_per_step": k_ul, "parallelism": "single GPU",
                      "out_format": args.out_format, "launch": "eager: one launch per step (arrivals enqueued "
                                                               "inside the step kernel)"},
           "env_steps_per_s": E * args.steps / dt,
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s",
                        "frac": achieved / PEAK_GBS, "kernel": "nr_step_kernel<two waves>",
                        "kernel_ms_avg": k_avg, "kernel_ms_median": k_ms[len(k_ms) // 2],
                        "algorithmic_bytes_per_launch": nbytes, "algorithmic_bytes_per_robot_step": per_robot,
                        "layout_bytes_per_launch": layout_bytes, "layout_bytes_per_robot_step": layout_per_robot,
                        **measured_fields("nr_step_kernel_counters_freq_sel" if (E, R) == (16384, 128) and
                                          args.out_format == "reference" else "", k_avg)}}
    if args.phase_clocks:
        res["phase_clocks"] = phase_clocks("w2", 2 * E)
    copy_calibration(args, res, torch, dev)
    if not args.no_cpu:
        print("# cpu baseline (oracle)", file=sys.stderr, flush=True)
        res["cpu_baseline"] = cpu_baseline(P, wl, cfg, min(args.cpu_envs, 128), min(args.cpu_steps, 3), 1)
    print(json.dumps(res), flush=True)


PHASES = ("prologue", "fading draws", "SR/grants/estimate/MCS/metric", "retx admission", "RBG allocation",
          "link adaptation", "binding/CSI gains/interference", "decoding", "HARQ/OLLA/PF/counters/RLC pointer",
          "epilogue frames", "empty-slot outputs/compaction", "stores/env reductions")


def phase_clocks(unit, n_waves):
    """Per-phase shader clocks (s_memtime cycles) of every wavefront of the last step-kernel launch of the phase build
    (unit: the translation unit that holds the kernel): the mean wave, the slowest wave and the phases' shares."""
    import ctypes
    import numpy as np
    from isaac_net_amd import _lib
    lib = _lib.load()
    fn = getattr(lib, f"inet_nr_phase_clocks_{unit}")
    fn.restype = ctypes.c_int
    a = np.zeros((n_waves, len(PHASES)), dtype=np.uint64)
    rc = fn(a.ctypes.data_as(ctypes.c_void_p), ctypes.c_int(n_waves))
    if rc != 0:
        raise RuntimeError(f"inet_nr_phase_clocks_{unit}: {rc}")
    a = a.astype(np.float64)
    tot = a.sum(1)
    slow = int(tot.argmax())
    top = np.argsort(tot)[-max(1, n_waves // 100):]          # the slowest 1% of the waves
    return {"unit": "cycles (s_memtime)", "waves": n_waves,
            "wave_total": {"min": float(tot.min()), "median": float(np.median(tot)), "mean": float(tot.mean()),
                           "max": float(tot.max())},
            "phases": {name: {"mean": float(a[:, i].mean()), "slowest_wave": float(a[slow, i]),
                              "slowest_1pct_mean": float(a[top, i].mean()),
                              "share_mean": float(a[:, i].mean() / tot.mean())}
                       for i, name in enumerate(PHASES)}}


def summarize_counters(d, kernel, name):
    """Read the rocprofv3 --pmc CSV outputs under d (passes FETCH_SIZE, WRITE_SIZE and the SQ_* counters of bench runs
    made with --copy-mib), scale the byte counters by what they read for the copy kernel of known size, and write
    profiles/<name>.json tagged with the loaded library's source hash. Prints the summary."""
    import csv
    import glob
    from isaac_net_amd import _lib
    rows = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        rows += list(csv.DictReader(open(f)))

    def per_dispatch(counter, match):
        vals = {}
        for r in rows:
            if r["Counter_Name"] == counter and match(r["Kernel_Name"]):
                vals[r.get("Dispatch_Id", len(vals))] = vals.get(r.get("Dispatch_Id", len(vals)), 0.0) + \
                    float(r["Counter_Value"])
        return [vals[k] for k in sorted(vals, key=lambda x: int(x))]
    copy = lambda k: "copyBuffer" in k  # noqa: E731
    mine = lambda k: kernel in k  # noqa: E731
    res = {"kernel": kernel, "workload": name, "src": _lib.load().inet_nr_build_info().decode().rsplit("src=", 1)[-1]}
    # the calibration copies: the three largest copy dispatches (the run's input copies are small)
    cf, cw = sorted(per_dispatch("FETCH_SIZE", copy))[-3:], sorted(per_dispatch("WRITE_SIZE", copy))[-3:]
    kf, kw = per_dispatch("FETCH_SIZE", mine)[2:], per_dispatch("WRITE_SIZE", mine)[2:]      # steady state
    copy_kib = None
    for a in sys.argv:
        if a.startswith("--copy-mib="):
            copy_kib = int(a.split("=")[1]) * 1024
    copy_kib = copy_kib or 256 * 1024
    if cf and kf:
        fs = copy_kib / (sum(cf) / len(cf))
        ws = copy_kib / (sum(cw) / len(cw))
        res.update({"fetch_scale": fs, "write_scale": ws, "fetch_kib_per_dispatch": sum(kf) / len(kf),
                    "write_kib_per_dispatch": sum(kw) / len(kw)})
        res["fetch_bytes"] = res["fetch_kib_per_dispatch"] * fs * 1024
        res["write_bytes"] = res["write_kib_per_dispatch"] * ws * 1024
        res["bytes_per_launch"] = res["fetch_bytes"] + res["write_bytes"]
    for c in ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_WR",
              "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES"):
        v = per_dispatch(c, mine)[2:]
        if v:
            res[c.lower() + "_per_dispatch"] = sum(v) / len(v)
    if "sq_insts_valu_per_dispatch" in res:
        res["valu_insts_per_dispatch"] = res["sq_insts_valu_per_dispatch"]
    json.dump(res, open(os.path.join(ROOT, "profiles", name + ".json"), "w"), indent=1)
    print(json.dumps(res, indent=1))


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-counters":
        load_package()
        return summarize_counters(sys.argv[2], sys.argv[3], sys.argv[4])
    if "--phase-clocks" in sys.argv:
        os.environ["INET_NR_LIB"] = os.path.join(ROOT, "isaac-net_amd", "libinet_nr_phase.so")
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="rl_scale",
                    choices=("rl_scale", "rl_scale_dl", "mc_interf", "freq_sel", "wifi_dcf", "wifi_dcf_slots"),
                    help="rl_scale: the NR engine's RL-scale workload (the headline metric); rl_scale_dl: the same with "
                         "the downlink on; mc_interf: three cells with UL interference (1024 x 64); freq_sel: 16384 x "
                         "128, 273 PRB, K = 20; wifi_dcf: level WIFI; wifi_dcf_slots: level WIFI_DCF on the same "
                         "inputs")
    ap.add_argument("--envs", type=int, default=None)
    ap.add_argument("--robots", type=int, default=None)
    ap.add_argument("--envs-per-wave", type=int, default=1, help="level WIFI: envs per 64-lane wavefront")
    ap.add_argument("--out-format", default="reference", choices=("reference", "compact"))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="replay submit and step from HIP graphs recorded after the warm-up instead of launching them "
                         "from Python every step (on this stack the eager launches are the faster of the two)")
    ap.add_argument("--no-graph-window", action="store_true",
                    help="skip the graph-replay window timed after the eager one (rl_scale)")
    ap.add_argument("--steady", type=int, default=0, metavar="N",
                    help="instead of the bench line: run N steps of rl_scale from a fresh engine and print the step "
                         "kernel's mean duration and queue occupancy per 50-step window")
    ap.add_argument("--separate-submit", action="store_true",
                    help="enqueue each step's arrivals with submit_counts (its own launch) instead of inside the step")
    ap.add_argument("--cpu-envs", type=int, default=2048)
    ap.add_argument("--cpu-steps", type=int, default=8)
    ap.add_argument("--phase-clocks", action="store_true",
                    help="load libinet_nr_phase.so and add the step kernel's per-phase clocks to the line")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="after the run, copy a buffer of this many MiB three times (a plain copy kernel of known "
                         "size, the calibration of the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this engine runs on one GPU (envs are independent; sharding is a design note); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    import torch
    P = load_package()
    args.envs_set, args.robots_set = args.envs is not None, args.robots is not None
    if args.workload in ("wifi_dcf", "wifi_dcf_slots"):
        return run_wifi(args, P, torch)
    if args.workload == "rl_scale_dl":
        return run_dl(args, P, torch)
    if args.workload == "mc_interf":
        return run_mc(args, P, torch)
    if args.workload == "freq_sel":
        return run_freq_sel(args, P, torch)
    from isaac_net_amd import scenarios as S
    from isaac_net_amd.engine import KernelTimer
    dev = "cuda:0"
    E = args.envs if args.envs_set else 4096
    R = args.robots if args.robots_set else 32
    # (after the timed window: the same number of steps as HIP graph replays, reported beside the eager figure)
    n_graph = 0 if (args.graph or args.no_graph_window) else args.steps
    total = args.warmup + args.steps + (n_graph + 2 if n_graph else 0)
    if args.steady:
        total = max(total, args.steady)
    print(f"# workload rl_scale {E}x{R}, {total} steps of inputs", file=sys.stderr, flush=True)
    wl = S.Workload(E, R, total, seed=0, device=dev)
    cfg = wl.cfg
    eng = P.make_engine("L2", E, R, dev, cfg, seed=0, out_format=args.out_format)
    k_ul = sum(1 for x in cfg.schedule(0) if x[2])
    if args.steady:
        return steady_state(eng, wl, args, torch, dev, k_ul)
    q_pre, q_post = [], []
    for s in range(args.warmup):
        eng.submit_counts(wl.counts[s])
        q_pre.append(float(eng.st["qlen"].float().mean()))
        eng.step(None, wl.poses[s])
        q_post.append(float(eng.st["qlen"].float().mean()))
    torch.cuda.synchronize()
    graph = eng.graph_step() if args.graph else None        # submit + step recorded once, replayed every step
    eng.kernel_events = ev = KernelTimer(args.steps, dev)    # HIP events around each step-kernel launch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        s = args.warmup + i
        if graph is not None:
            graph(wl.poses[s], wl.counts[s])
        elif args.separate_submit:
            eng.submit_counts(wl.counts[s])
            eng.step(None, wl.poses[s])
        else:                                        # the arrivals enqueued inside the step's launch
            eng.step(None, wl.poses[s], arrivals=wl.counts[s])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    eng.kernel_events = None
    k_ms = sorted(ev.ms())
    k_avg = sum(k_ms) / len(k_ms)
    qlen_mean = sum(q_pre) / max(len(q_pre), 1)
    kept_mean = sum(q_post) / max(len(q_post), 1)
    layout_bytes, layout_per_robot = step_kernel_bytes(eng)
    touched = step_kernel_touched_bytes(eng, qlen_mean, kept_mean)
    per_robot = canonical_bytes_per_robot_step(eng)
    nbytes = E * R * per_robot
    achieved = nbytes / (k_avg * 1e-3) / 1e9
    value = E * R * k_ul * args.steps / dt
    # HBM bytes per launch measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (scaled by a copy-kernel
    # calibration) and VALU instructions (SQ_INSTS_VALU) of this workload, from the counter summary recorded on the
    # loaded library's sources; null when there is none
    cs = counter_summary(f"nr_step_kernel_counters_rl_scale_{args.out_format}") if (E, R) == (4096, 32) else None
    traffic = cs.get("bytes_per_launch") if cs else None
    # VALU issue utilisation: a wave64 VALU instruction occupies a 16-lane SIMD for 4 cycles; 1024 SIMDs at 2.4 GHz
    valu_util = (cs["valu_insts_per_dispatch"] * 4 / (1024 * k_avg * 1e-3 * 2.4e9)) if cs else None
    res = {"metric": METRIC, "value": value, "unit": "robot-slots/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": 1e3 * dt / args.steps, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
           "config": {"workload": f"rl_scale: {E} envs x {R} robots, K={k_ul} UL slots/step (DDDSU, 25 ms), 52 PRB "
                                  "(13 RBGs), PF alpha 0.01, 8 HARQ x 5 tx, Rician K 3 dB, 200 B @0.8 + 4000 B @0.1 "
                                  "per robot-step, FIFO 32, UMi LOS",
                      "envs": E, "robots": R, "ul_slots_per_step": k_ul, "global_batch": E * R,
                      "parallelism": "single GPU", "out_format": args.out_format,
                      "launch": "hip graph replay" if args.graph else
                      ("eager: submit_counts + step" if args.separate_submit else "eager: one launch per step "
                       "(arrivals enqueued inside the step kernel)")},
           "env_steps_per_s": E * args.steps / dt,
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s",
                        "frac": achieved / PEAK_GBS, "traffic": traffic,
                        "kernel": "nr_step_kernel", "kernel_ms_avg": k_avg, "kernel_ms_median": k_ms[len(k_ms) // 2],
                        "algorithmic_bytes_per_launch": nbytes, "algorithmic_bytes_per_robot_step": per_robot,
                        "layout_bytes_per_launch": layout_bytes, "layout_bytes_per_robot_step": layout_per_robot,
                        "touched_bytes_per_launch": touched, "queue_frames_per_robot": qlen_mean,
                        "valu_issue_util": valu_util,
                        "counters_src": cs.get("src") if cs else None}}
    if n_graph:
        # the next n_graph steps as replays of the recorded step graph (counts-form enqueue + step); the first two
        # replays (recording) are not timed
        g = eng.graph_step()
        base = args.warmup + args.steps
        for s in range(base, base + 2):
            g(wl.poses[s], wl.counts[s])
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for s in range(base + 2, base + 2 + n_graph):
            g(wl.poses[s], wl.counts[s])
        torch.cuda.synchronize()
        res["graph_replay"] = {"ms_per_step": 1e3 * (time.perf_counter() - t1) / n_graph, "steps": n_graph,
                               "launch": "HIP graph replay of submit_counts + step, the inputs copied into the "
                                         "graph's buffers first"}
    if args.phase_clocks:
        res["phase_clocks"] = phase_clocks("s13" if eng.S == 13 else "s8", (E * R + 63) // 64)
    copy_calibration(args, res, torch, dev)
    if not args.no_cpu:
        print("# cpu baseline (oracle)", file=sys.stderr, flush=True)
        res["cpu_baseline"] = cpu_baseline(P, wl, cfg, min(args.cpu_envs, E), args.cpu_steps, 1)
    print(json.dumps(res), flush=True)


def steady_state(eng, wl, args, torch, dev, k_ul):
    """The whole run of the workload (args.steady steps, from a fresh engine): the step kernel's mean duration (HIP
    events) and the mean queue length per window of 50 steps, to show whether a short window after a few warm-up
    steps measures the steady state."""
    from isaac_net_amd.engine import KernelTimer
    n = args.steady
    eng.kernel_events = ev = KernelTimer(n, dev)
    q = []
    for s in range(n):
        eng.step(None, wl.poses[s], arrivals=wl.counts[s])
        if s % 10 == 9:
            q.append((s, float(eng.st["qlen"].float().mean())))
    torch.cuda.synchronize()
    ms = ev.ms()
    win = []
    for a in range(0, n, 50):
        w = ms[a:a + 50]
        qq = [v for (s, v) in q if a <= s < a + 50]
        win.append({"steps": f"{a}..{a + len(w) - 1}", "kernel_ms_avg": sum(w) / len(w),
                    "queue_frames_per_robot": sum(qq) / max(len(qq), 1)})
    print(json.dumps({"workload": "rl_scale steady-state check", "steps": n, "windows": win}), flush=True)


if __name__ == "__main__":
    main()

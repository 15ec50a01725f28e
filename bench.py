#!/usr/bin/env python3
"""Benchmark of the batched F-16 step on one MI355X, with each kernel's roofline fraction
(algorithmic FLOPs or bytes per launch over its measured duration) and a CPU baseline.

A "step" is one decision of the batched flight model: every aircraft of 16,384 tail-chase
engagements (32,768 aircraft) advances 6 substeps of 1/60 s with its random 21-bin action
held (BASELINE configs[1] model at the metric's 16k-engagement size).  Inputs are resident in
HBM before the timed region.  Prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--nenv 16384] [--substeps 6]
                    [--cpu-seconds 10] [--no-cpu]
"""
import argparse
import ctypes
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = "2026_ai_pilot_challenge-1st_solution_amd"

# Algorithmic FP64 work of one aircraft-substep (adds, subs, muls, divs, sqrts and libm calls
# each 1), counted by the operation-counting build of the CPU restatement on the headline
# workload (tests/golden/fdm_flops.json, c2_tailchase); the reference model's static count is
# 1,550.
def _flop_per_substep(sample="c2_tailchase"):
    path = os.path.join(ROOT, "tests", "golden", "fdm_flops.json")
    try:
        return float(json.load(open(path))["per_aircraft_substep"][sample]["flop"])
    except (OSError, KeyError, ValueError):
        return 1550.0


FLOP_PER_SUBSTEP = _flop_per_substep()
# Algorithmic HBM bytes of one aircraft per launch of the fp64 flight model: the 66 state doubles
# a launch reads, the 101 it writes, and its 4 action doubles (half of it in the fp32 build)
FDM_BYTES_PER_AIRCRAFT = (66 + 101 + 4) * 8
PEAK_FP64_TFLOPS = 78.6
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
# reference's published GpuDogfight.step rate at 16k envs (RTX 3070 Ti, cuda_fdm/README.md:130)
REF_PUBLISHED_SUBSTEPS = 37.0e6


def _regions(run, reps, reset=None):
    """Time `run` (one region of GPU work on the current stream) `reps` times with HIP events
    on that stream, `reset` (untimed) before each; returns the per-region milliseconds."""
    import torch
    out = []
    for _ in range(reps):
        if reset is not None:
            reset()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        run()
        e1.record()
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1))
    return out


def profiled_traffic(name="fdm_step_quad_kernel_tailchase16k.md"):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE/WRITE_SIZE (copy-calibrated) and
    recorded in the kernel's profile summary; None when no summary is present."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":")[1])
    return None


def _host_info():
    """CPU model, sockets and the compiler/flags the CPU paths were built with."""
    model, sockets = "unknown", set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("physical id"):
                sockets.add(line.split(":", 1)[1].strip())
    except OSError:
        pass
    try:
        import subprocess
        cc = subprocess.run(["gcc", "--version"], capture_output=True, text=True).stdout
        cc = cc.splitlines()[0] if cc else "gcc (unknown)"
    except OSError:
        cc = "gcc (unknown)"
    flags = "unknown"
    for line in open(os.path.join(ROOT, "oracle", "Makefile")):
        if line.startswith("CFLAGS"):
            flags = line.split("=", 1)[1].strip()
    return {"cpu_model": model, "sockets": max(1, len(sockets)), "compiler": cc,
            "flags": flags, "host_threads": len(os.sched_getaffinity(0))}


def _fdm_runner(fcs_rate, substeps):
    """The reference's own C model (oracle/_ref, fdm.cuh built from its sources) for the host;
    the C restatement (oracle/liborc.so) where that is absent."""
    D = ctypes.POINTER(ctypes.c_double)
    ref = os.path.join(ROOT, "oracle", "_ref", f"libf16ref_{fcs_rate}.so")
    if os.path.exists(ref):
        fn = ctypes.CDLL(ref).ref_fdm_rollout
        fn.argtypes = [D, D, ctypes.c_long, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        return "reference", lambda st, act, nac, ndec, nth: fn(
            st.ctypes.data_as(D), act.ctypes.data_as(D), nac, ndec, substeps, nth)
    fn = ctypes.CDLL(os.path.join(ROOT, "oracle", "liborc.so")).orc_fdm_rollout
    fn.argtypes = [D, D, ctypes.c_long, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    return "port", lambda st, act, nac, ndec, nth: fn(
        st.ctypes.data_as(D), act.ctypes.data_as(D), nac, ndec, substeps, fcs_rate, nth)


def _threads_run(fns):
    """Run the callables on host threads (ctypes calls release the GIL)."""
    import threading
    ts = [threading.Thread(target=f) for f in fns]
    for t in ts:
        t.start()
    for t in ts:
        t.join()


def cpu_baseline(states0_aos, actions_host, substeps, cpu_seconds, icm):
    """The reference path on the host cores, bounded samples (each stated in its entry):
      value: the FDM (16k tail-chase, the GPU's timed decisions cycled for ~cpu_seconds) with
             the reference's own C model on every host thread, plus a 1-thread figure;
      c1_full: BASELINE C1 end to end (64 head-on engagements, 600 decisions, 120 Hz FCS);
      obs_reward_c3: advance + reward + termination + the 184-D observation (the C restatement
             of BatchObsReward, oracle/obs_oracle.c) over 32,768 aircraft, every host thread;
      gae_c4: the reference's GAE recurrence (oracle/gae_oracle.py, numpy float32) over
             [64, 16384, 2];
      env_transitions_per_s: one env decision at 16k engagements = FDM (60 Hz FCS lineage) +
             obs/reward, both on every host thread."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib
    kind, run = _fdm_runner(120, substeps)
    cores = len(os.sched_getaffinity(0))
    nac = states0_aos.shape[0]
    st = states0_aos.copy()
    acts = np.ascontiguousarray(actions_host)
    ndec = 0
    t0 = time.perf_counter()
    while True:
        run(st, acts, nac, acts.shape[0], cores)
        ndec += acts.shape[0]
        dt = time.perf_counter() - t0
        if dt >= cpu_seconds:
            break
    # one thread: the first 1,024 aircraft, decisions cycled for at least 2 s
    n1 = min(nac, 1024)
    st1 = np.ascontiguousarray(states0_aos[:n1])
    a1 = np.ascontiguousarray(actions_host[:, :n1])
    nd1, t1 = 0, time.perf_counter()
    while True:
        run(st1, a1, n1, a1.shape[0], 1)
        nd1 += a1.shape[0]
        dt1 = time.perf_counter() - t1
        if dt1 >= 2.0:
            break
    out = {"value": nac * substeps * ndec / dt, "unit": "aircraft-substeps/s", "cores": cores,
           "kind": kind,
           "sample": f"{nac} aircraft x {ndec} decisions x {substeps} substeps, fp64, OpenMP "
                     f"over aircraft on {cores} host threads ({dt:.1f} s)",
           "single_thread": n1 * substeps * nd1 / dt1,
           "single_thread_sample": f"{n1} aircraft x {nd1} decisions x {substeps} substeps on "
                                   f"one thread ({dt1:.1f} s)"}
    out.update(_host_info())
    orc = oracle_lib.load()
    # C1 in full: 128 aircraft x 600 decisions, seeded by the C restatement
    c1_ic = icm.sample_headon(64, seed=0)
    c1 = orc.seed(c1_ic, 120)
    c1_act = np.ascontiguousarray(icm.random_bin_actions(600, 128, seed=0))
    t0 = time.perf_counter()
    run(c1, c1_act, 128, 600, cores)
    dt = time.perf_counter() - t0
    out["c1_full"] = {"value": 128 * 600 * substeps / dt, "unit": "aircraft-substeps/s",
                      "seconds": dt, "cores": cores,
                      "sample": "C1: 128 aircraft x 600 decisions x 6 substeps, fp64"}
    # obs / reward on the 32,768 bench aircraft (16k engagements), one oracle per host thread
    nenv = nac // 2
    K = max(1, min(cores, 64))
    while nenv % K:
        K -= 1
    per = nenv // K
    s_all = np.ascontiguousarray(states0_aos)
    obs_parts = []
    for k in range(K):
        ob = oracle_lib.ObrOracle(orc, per)
        sub = np.ascontiguousarray(s_all[2 * per * k:2 * per * (k + 1)])
        obs_parts.append((ob, sub, np.ascontiguousarray(actions_host[0, 2 * per * k:2 * per * (k + 1)])))

    obs_parts[0][0].state9(obs_parts[0][1][:2])                # one-time init, one thread

    def obs_decision():
        _threads_run([lambda ob=ob, sub=sub, a=a: (lambda s9: (ob.step(s9, a), ob.build_obs(s9)))(
            ob.state9(sub)) for ob, sub, a in obs_parts])
    obs_decision()                                              # anchors prev state
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 3.0:
        obs_decision()
        reps += 1
    obs_dt = (time.perf_counter() - t0) / reps
    out["obs_reward_c3"] = {"value": nac / obs_dt, "unit": "aircraft/s", "cores": K,
                            "ms_per_decision": obs_dt * 1e3, "kind": "port",
                            "sample": f"{nac} aircraft (16k engagements) x {reps} decisions: "
                                      "state9 + advance/reward/termination + 184-D observation"}
    # GAE over [64, 16384, 2] float32 (numpy, one thread)
    import importlib.util
    spec = importlib.util.spec_from_file_location("gae_oracle", os.path.join(ROOT, "oracle", "gae_oracle.py"))
    GO = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(GO)
    rng = np.random.default_rng(0)
    T = 64
    rew = rng.standard_normal((T, nac)).astype(np.float32)
    val = rng.standard_normal((T, nac)).astype(np.float32)
    done = (rng.random((T, nenv)) < 0.01).astype(np.float32)
    lv = rng.standard_normal(nac).astype(np.float32)
    nd = np.zeros(nenv, np.float32)
    t0 = time.perf_counter()
    GO.gae_f32(rew, val, done, lv, nd, 0.99, 0.95, nagents=2)
    gdt = time.perf_counter() - t0
    out["gae_c4"] = {"value": T * nac / gdt, "unit": "elements/s", "cores": 1, "kind": "port",
                     "ms": gdt * 1e3, "sample": "[64, 16384, 2] float32, numpy"}
    # one env decision on the host: FDM (60 Hz lineage) + obs/reward, every thread
    kind60, run60 = _fdm_runner(60, substeps)
    st60 = states0_aos.copy()
    a60 = np.ascontiguousarray(actions_host[:1])
    t0 = time.perf_counter()
    for _ in range(3):
        run60(st60, a60, nac, 1, cores)
    fdm_dt = (time.perf_counter() - t0) / 3
    out["env_transitions_per_s"] = nenv / (fdm_dt + obs_dt)
    out["env_step_sample"] = (f"{nenv} engagements: FDM decision ({kind60} C model, 60 Hz FCS, "
                              f"{fdm_dt * 1e3:.1f} ms) + obs/reward ({obs_dt * 1e3:.1f} ms), "
                              f"{cores} host threads")
    return out


# Algorithmic HBM bytes of one aircraft in the fused post-physics kernel: reads the 15 state
# doubles position..fuel (kinematics, reward, fuel) + the physics launch's finite flag (1 byte)
# + actions 4 + reconstructor (hp, fuel, prev_att 3, act_hist 16, prev_x, prev_alt_log, flags,
# t, ...: 27); writes reconstructor (hp, hp_loss, fuel, pqr 3, prev_att 3, act_hist 20, dealt,
# taken, prev_x, prev_alt_log, flags, t) + reward + terminal and live observations (2 x 184
# f32) + terminal HP/altitude.  Without the flag (F16EnvStepIO.state_finite NULL) the launch
# reads the other 86 state doubles instead of the byte.
POST_BYTES_PER_AIRCRAFT = (15 + 4 + 27) * 8 + 1 + 2 + (34 + 3) * 8 + 2 * 184 * 4 + 4
POST_BYTES_SCAN_EXTRA = 86 * 8 - 1
# The one-launch step (f16_env_step): the physics' bytes (66 state doubles read, 101 written,
# 4 actions read) and the post-physics step's, less the 15 state doubles the post-physics phase
# reads back from L2 (the same workgroup stored them)
STEP_BYTES_PER_AIRCRAFT = (66 + 101 + 4) * 8 + POST_BYTES_PER_AIRCRAFT - 15 * 8
# The 214-D post-physics launch of the league rollout: the 184-D bytes, 30 more float32
# columns in each of the two observation rows, the previous NED velocity read and it and the
# acceleration written (9 doubles), and the opponent draw's id written on autoreset (ignored)
POST_BYTES_214_PER_AIRCRAFT = POST_BYTES_PER_AIRCRAFT + 2 * 30 * 4 + 9 * 8
# reference's published full env step at 16,384 envs: 10.3 ms (RTX 3070 Ti,
# cuda_fdm/README.md:225) = 1.59 M env transitions/s
REF_PUBLISHED_ENV_TRANSITIONS = 16384 / 10.3e-3
STAGGER_STEPS = 2000          # = the 200 s engagement limit: episode clocks spread over it


def _env_timed(env, acts, warmup, steps):
    import torch
    for k in range(warmup):
        env.step(acts[k])
    torch.cuda.synchronize()
    # the timed steps: nothing but env.step (the done flags are kept and summed afterwards)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    dones = []
    e0.record()
    t0 = time.perf_counter()
    for k in range(steps):
        _, _, done, _ = env.step(acts[warmup + k])
        dones.append(done)
    host = (time.perf_counter() - t0) * 1e3 / steps     # issue time of one step on the host
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, int(torch.stack(dones).sum().item()), host


def _env_kernel_ms(env, acts, warmup, n):
    """Mean launch times from a pass with events around each launch: (FDM, post-physics) for
    the two-launch step, (None, None) and the one launch's for f16_env_step's fused kernel."""
    import torch
    env.kernel_events, env.sim.kernel_events = [], []
    for k in range(n):
        env.step(acts[warmup + k])
    torch.cuda.synchronize()
    mean = lambda ev: float(np.mean([a.elapsed_time(b) for a, b in ev])) if ev else None
    post, fdm = mean(env.kernel_events), mean(env.sim.kernel_events)
    env.kernel_events = env.sim.kernel_events = None
    return (fdm, post, None) if fdm is not None else (None, None, post)


# env step variants: (fused_step, fused_finite)
ENV_VARIANTS = {"one_launch": (True, True), "two_launch": (False, True),
                "state_scan": (False, False)}


def env_step_bench(pkg, nenv, steps, warmup, scan_finite=False, ab=True, stagger=True,
                   pool_tables=True, two_launch=False, reps=5):
    """Full environment transitions: GpuDogfightVecEnv.step = FDM decision (6 substeps, FCS 60 Hz)
    + the fused post-physics step (advance, reward, termination, terminal observation, pool
    autoreset, new observation), contest ICs with the staggered reset spread over the whole
    200 s engagement (so timeouts and deaths autoreset engagements inside the timed loop),
    random 4-channel actions resident on the device.  Three variants are timed on the same
    steps (A/B in one process): f16_env_step's single launch (the default), the physics launch
    and the post-physics launch separately (the physics launch's per-aircraft finite flags
    handed over; each launch timed on its own), and the two launches with the post-physics
    launch re-reading the state for the finite flag.  ab=False: time only one variant, the
    single launch, or with two_launch / scan_finite that one; stagger=False starts every
    engagement at t = 0 (no autoresets in the window); pool_tables=False rebuilds autoreset rows
    instead of copying them (profiling aids)."""
    import torch
    env_mod = importlib.import_module(PKG + ".rl_env")
    env = env_mod.GpuDogfightVecEnv(nenv, seed=0)
    env.pool_tables = pool_tables
    env.reset(stagger=stagger, max_stagger_steps=STAGGER_STEPS)
    g = torch.Generator(device="cuda").manual_seed(0)
    acts = torch.rand(warmup + steps, 2 * nenv, 4, generator=g, device="cuda",
                      dtype=torch.float64) * 2 - 1
    acts[..., 3] = (acts[..., 3] + 1) / 2
    snap_states = env.sim.states.clone()
    snap_obr = env.obr.clone_state()
    snap_steps = env._post_steps
    post_bytes = POST_BYTES_PER_AIRCRAFT * 2 * nenv
    if ab:
        # mirrored order: whichever variant runs first after the warm-up pays for it; the
        # default variant then runs to `reps` regions in all
        order = ("one_launch", "two_launch", "state_scan", "state_scan", "two_launch",
                 "one_launch") + ("one_launch",) * max(0, reps - 2)
    else:
        order = (("state_scan",) if scan_finite else ("two_launch",) if two_launch else
                 ("one_launch",)) * reps
    runs = {}
    for name in order:
        env.fused_step, env.fused_finite = ENV_VARIANTS[name]
        env.sim.states.copy_(snap_states)        # every variant steps the same engagements
        env.obr.restore(snap_obr)
        env._post_steps = snap_steps
        ms, done, host = _env_timed(env, acts, warmup, steps)
        runs.setdefault(name, []).append((ms, done) + _env_kernel_ms(env, acts, warmup,
                                                                       min(steps, 20)) + (host,))
    env.fused_step, env.fused_finite = ENV_VARIANTS["one_launch"]
    res = {}
    for name, r in runs.items():
        med = lambda i: None if r[0][i] is None else float(np.median([x[i] for x in r]))
        ms, done, fdm_ms, post_ms, step_ms, host = (med(i) for i in range(6))
        res[name] = {"ms_per_step": ms, "episodes_done": int(round(done)),
                     "host_issue_ms_per_step": host, "regions": len(r),
                     "ms_per_step_regions": [x[0] for x in r]}
        if step_ms is not None:
            res[name]["step_kernel_ms"] = step_ms
        else:
            b = post_bytes + (POST_BYTES_SCAN_EXTRA * 2 * nenv if name == "state_scan" else 0)
            res[name].update({"fdm_kernel_ms": fdm_ms, "post_kernel_ms": post_ms,
                              "algorithmic_bytes": b,
                              "achieved_GBs": b / (post_ms * 1e-3) / 1e9,
                              "hbm_frac": b / (post_ms * 1e-3) / 1e9 / PEAK_HBM_GBS})
    main_name = order[0]
    main = res[main_name]
    out = {"workload": "contest_env_step_16k", "engagements": nenv, "obs_dim": 184,
           "substeps": env.substeps, "fcs_rate_hz": env.sim.fcs_rate,
           "reset": f"stagger over {STAGGER_STEPS} decisions" if stagger else "no stagger",
           "pool_tables": pool_tables, "variant": main_name,
           "transitions_per_s": nenv / (main["ms_per_step"] * 1e-3),
           "ms_per_step": main["ms_per_step"], "episodes_done": main["episodes_done"],
           "host_issue_ms_per_step": main["host_issue_ms_per_step"],
           "vs_published": nenv / (main["ms_per_step"] * 1e-3) / REF_PUBLISHED_ENV_TRANSITIONS}
    if "step_kernel_ms" in main:
        sb = STEP_BYTES_PER_AIRCRAFT * 2 * nenv
        out["step_kernel"] = {"kernel": "env_step_quad_kernel<60,184>",
                              "kernel_ms": main["step_kernel_ms"], "algorithmic_bytes": sb,
                              "achieved_GBs": sb / (main["step_kernel_ms"] * 1e-3) / 1e9,
                              "hbm_frac": sb / (main["step_kernel_ms"] * 1e-3) / 1e9 /
                              PEAK_HBM_GBS}
    two = res.get("two_launch", res.get("state_scan"))
    if two is not None:
        out["fdm_kernel_ms"], out["post_kernel_ms"] = two["fdm_kernel_ms"], two["post_kernel_ms"]
        out["post_kernel"] = {"kernel": "env_post_step_quad_kernel<184>",
                              "variant": "two_launch" if "two_launch" in res else "state_scan",
                              "algorithmic_bytes": two["algorithmic_bytes"],
                              "achieved_GBs": two["achieved_GBs"], "hbm_frac": two["hbm_frac"]}
    if ab:
        out["two_launch_ab"] = {"what": "f16_fdm_step_batch_keep then f16_env_post_step (the "
                                        "physics launch's finite flags handed over)",
                                **res["two_launch"]}
        out["state_scan_ab"] = {"what": "the two launches with the post-physics launch "
                                        "re-reading the 86 other state doubles for the finite "
                                        "flag instead of the physics launch's flag",
                                **res["state_scan"]}
    return out


PEAK_BF16_TFLOPS = 2500.0


def obs_reward_c3_bench(nenv=16384, steps=50, reps=5):
    """BASELINE C3, the fused observation/reward kernel alone: 16,384 engagements whose
    aircraft hold random valid states (ic.sample_random_valid: +-20 km, 100-350 m/s, any
    attitude, alpha/beta inside the tables, fuel U[0.2, 1]), a fresh reconstructor anchored on
    them, random actions.  The timed launch is f16_env_post_step without a physics launch
    before it: advance (action history, damage, HP, fuel, body rates, time), reward and
    termination for both aircraft, terminal and new 184-D observations and autoreset from the
    IC pool; with no physics launch to hand over the finite flags, it tests the state itself
    (reads all 101 doubles).  `steps` launches per region on the same states (regions start
    from the same reconstructor), median of `reps` regions."""
    import torch
    env_mod = importlib.import_module(PKG + ".rl_env")
    icm = importlib.import_module(PKG + ".ic")
    env = env_mod.GpuDogfightVecEnv(nenv, seed=0)
    env.reset(stagger=False)
    env.sim.seed_rows(torch.as_tensor(icm.sample_random_valid(nenv, seed=3), device="cuda"))
    env.obr.reset_all()
    env.obr.kernel_init_reward_state(env.sim.states)
    env._ensure_ic_pool()
    nac = env.nac
    g = torch.Generator(device="cuda").manual_seed(3)
    a = torch.rand(nac, 4, generator=g, device="cuda", dtype=torch.float64) * 2 - 1
    a[:, 3] = (a[:, 3] + 1) / 2
    env.sim.actions.copy_(a)
    snap, snap_obr, snap_steps = env.sim.states.clone(), env.obr.clone_state(), env._post_steps
    f64, b = dict(dtype=torch.float64, device="cuda"), dict(dtype=torch.bool, device="cuda")
    reward, thp, talt = (torch.empty(nac, **f64) for _ in range(3))
    tobs = torch.empty(nac, 184, dtype=torch.float32, device="cuda")
    term, trunc, done, fin = (torch.empty(nenv, **b) for _ in range(4))
    io = env._io(None)
    io.reward, io.terminal_obs = reward.data_ptr(), tobs.data_ptr()
    io.terminal_hp, io.terminal_alt_m = thp.data_ptr(), talt.data_ptr()
    io.term, io.trunc, io.done, io.terminal_finite = (t.data_ptr() for t in (term, trunc, done, fin))
    io.state_finite = None
    env._call_tensors = ()

    def run():
        for _ in range(steps):
            env._post(io)

    def reset():
        env.sim.states.copy_(snap)
        env.obr.restore(snap_obr)
        env._post_steps = snap_steps
    reset()
    run()                                              # warm-up
    ms = _regions(run, reps, reset)
    reset()
    env.kernel_events = []
    run()
    torch.cuda.synchronize()
    kms = float(np.median([x.elapsed_time(y) for x, y in env.kernel_events]))
    env.kernel_events = None
    done_n = int(done.sum().item())
    m = float(np.median(ms)) / steps
    byt = (POST_BYTES_PER_AIRCRAFT + POST_BYTES_SCAN_EXTRA) * nac
    return {"workload": "obs_reward_c3_random_16k", "engagements": nenv, "obs_dim": 184,
            "kernel": "env_post_step_quad_kernel<184>", "launches_per_region": steps,
            "regions": reps, "ms_per_launch": m, "ms_per_launch_regions": [x / steps for x in ms],
            "kernel_ms_per_launch_events": kms,
            "engagements_per_s": nenv / (m * 1e-3), "aircraft_per_s": nac / (m * 1e-3),
            "algorithmic_bytes": byt, "achieved_GBs": byt / (m * 1e-3) / 1e9,
            "frac_hbm_peak": byt / (m * 1e-3) / 1e9 / PEAK_HBM_GBS,
            "episodes_done_last_launch": done_n}


def rollout_bench(nenv, T=64, reps=5, stagger=True):
    """BASELINE C4: nenv engagements x T-step self-play rollout (FDM + fused obs/reward + norm
    update + fused bf16 actor/critic with Philox draw) then GAE (gamma 0.99, lambda 0.95) over
    [T, nenv, 2].  Weights N(0, 0.02), draw seed 0.  The collector records the rollout as a HIP
    graph and replays it (its results equal the eager collector's bit for bit); a separate eager
    rollout with events around the policy launches gives the policy kernel's time."""
    import torch
    env_mod = importlib.import_module(PKG + ".rl_env")
    pol = importlib.import_module(PKG + ".policy")
    ppo = importlib.import_module(PKG + ".ppo")

    def make(graph):
        env = env_mod.GpuDogfightVecEnv(nenv, seed=0)
        net = pol.MLPActorCritic(184, init="normal", init_std=0.02,
                                 generator=torch.Generator().manual_seed(0)).to("cuda")
        ro = ppo.SelfPlayRollout(env, net, T=T, gamma=0.99, lam=0.95, seed=0, stats=False,
                                 graph=graph)
        ro.reset(stagger=stagger, max_stagger_steps=STAGGER_STEPS)
        return ro
    ro = make(True)
    ro.collect()                                    # eager warm-up (allocations)
    ro.collect()                                    # records the graph, replays it
    res = {}

    def one():
        res["out"] = ro.collect()
    regions = _regions(one, reps)
    adv, ret, stats = res["out"]
    if not bool(stats["trajectory_finite"]) or not bool(torch.isfinite(adv).all()):
        raise FloatingPointError("non-finite rollout")
    ms = float(np.median(regions))
    done = float(ro.b_done[1:].sum().item() + ro.next_done.sum().item())
    del ro
    eager = make(False)
    eager.collect()
    torch.cuda.synchronize()
    eager.policy_events = []
    t0 = time.perf_counter()
    eager.collect()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3
    pol_ms = float(np.mean([a.elapsed_time(b) for a, b in eager.policy_events]))
    flop = ppo.POLICY_FLOP_PER_ROW[184] * 2 * nenv
    return {"workload": "selfplay_rollout_16k_T64", "engagements": nenv, "T": T,
            "reset": f"stagger over {STAGGER_STEPS} decisions" if stagger else "no stagger",
            "episodes_done_per_rollout": done,
            "hip_graph": True, "ms_per_rollout": ms, "ms_per_rollout_regions": regions,
            "eager_ms_per_rollout": eager_ms,
            "transitions_per_s": nenv * T / (ms * 1e-3),
            "aircraft_transitions_per_s": 2 * nenv * T / (ms * 1e-3),
            "policy_kernel_ms": pol_ms,
            "policy_mfma": {"kernel": "policy_kernel<192>", "flop_per_launch": flop,
                            "achieved_TFLOPs": flop / (pol_ms * 1e-3) / 1e12,
                            "peak_TFLOPs": PEAK_BF16_TFLOPS,
                            "frac": flop / (pol_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}}


def update_bench(nenv, T=64, reps=5):
    """The PPO update after a BASELINE C4 rollout (PPOGPUTrainer.update, ppo_gpu.py:2019-2145):
    both aircraft's transitions (T x 2 nenv), the reference's PPOConfig (clip 0.2, 8 minibatches,
    Adam 3e-4 / eps 1e-5, max grad norm 0.5) with all 4 epochs (no KL early stop, so every run
    does the same work).  Per minibatch: f16_ppo_grad (forward, loss, backward, weight gradients)
    and f16_ppo_adam_step (clip + Adam + blob repack)."""
    import torch
    env_mod = importlib.import_module(PKG + ".rl_env")
    pol = importlib.import_module(PKG + ".policy")
    ppo = importlib.import_module(PKG + ".ppo")
    U = importlib.import_module(PKG + ".ppo_update")
    env = env_mod.GpuDogfightVecEnv(nenv, seed=0)
    net = pol.MLPActorCritic(184, init="normal", init_std=0.02,
                             generator=torch.Generator().manual_seed(0)).to("cuda")
    ro = ppo.SelfPlayRollout(env, net, T=T, gamma=0.99, lam=0.95, seed=0, stats=False)
    ro.reset(stagger=False)
    adv, ret, _ = ro.collect()
    up = U.PPOUpdater(net, U.UpdateConfig(target_kl=None), seed=0)
    up.update(ro, adv, ret)                         # warm-up (workspace allocation)
    hold = {}

    def one():
        hold["res"] = up.update(ro, adv, ret)
    regions = _regions(one, reps)
    res = hold["res"]
    ms = float(np.median(regions))
    # one epoch with events around each call
    obs, act = ro.b_obs.flatten(0, 1), ro.b_act.flatten(0, 1)
    logp, a, r = ro.b_logp.flatten(), adv.reshape(-1), ret.reshape(-1)
    count = obs.shape[0]
    mb = (count + 7) // 8
    perm = torch.randperm(count, device="cuda")
    ev = []
    for s in range(0, count, mb):
        t = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        t[0].record()
        up.minibatch_grad(obs, act, logp, a, r, perm[s:s + mb], up.stats[0])
        t[1].record()
        up.optimizer_step()
        t[2].record()
        ev.append(t)
    torch.cuda.synchronize()
    grad_ms = float(np.mean([x[0].elapsed_time(x[1]) for x in ev]))
    adam_ms = float(np.mean([x[1].elapsed_time(x[2]) for x in ev]))
    flop_mb = U.update_flop_per_row(184) * mb
    if not bool(torch.isfinite(up.flat).all()):
        raise FloatingPointError("non-finite parameters after the update")
    return {"workload": "ppo_update_selfplay_16k_T64", "transitions": count, "epochs": res["epochs"],
            "minibatches": (count + mb - 1) // mb, "minibatch_rows": mb, "ms_per_update": ms,
            "ms_per_update_regions": regions,
            "transitions_per_s": count * res["epochs"] / (ms * 1e-3),
            "minibatch_grad_ms": grad_ms, "optimizer_step_ms": adam_ms,
            "mfma": {"what": "f16_ppo_grad (all its launches)", "flop_per_minibatch": flop_mb,
                     "achieved_TFLOPs": flop_mb / (grad_ms * 1e-3) / 1e12,
                     "peak_TFLOPs": PEAK_BF16_TFLOPS,
                     "frac": flop_mb / (grad_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS},
            "stats": {k: float(res[k]) for k in ("pl", "vl", "ent", "kl", "cf", "ev")}}


def league_bench(nenv=65536, T=128, nopp=8, reps=5):
    """BASELINE C5: nenv engagements x T-step league rollout with the 214-D observation: the
    learner (plane 0) and 8 frozen random-init opponents (plane 1, bf16 N(0, 0.02)) assigned per
    engagement from Zipf(1.1) weights, evaluated as one grouped launch; fuel exhaustion and
    ground-collision (hard deck) terminations, autoreset with opponent redraw inside the step
    kernel; GAE over [T, nenv].  Recorded as a HIP graph and replayed; one eager rollout with
    events gives the per-kernel times."""
    import torch
    env_mod = importlib.import_module(PKG + ".rl_env")
    pol = importlib.import_module(PKG + ".policy")
    ppo = importlib.import_module(PKG + ".ppo")

    def make(graph):
        env = env_mod.GpuDogfightVecEnv(nenv, seed=0, obs_dim=214, fuel_exhaustion=True,
                                        fuel_lbs_range=(100.0, 3000.0))
        mk = lambda s: pol.MLPActorCritic(214, init="normal", init_std=0.02,
                                          generator=torch.Generator().manual_seed(s)).to("cuda")
        net, opps = mk(0), [mk(100 + k) for k in range(nopp)]
        ro = ppo.LeagueRollout(env, net, opps, T=T, gamma=0.99, lam=0.95, seed=0, graph=graph)
        ro.reset(stagger=False)
        return ro
    ro = make(True)
    ro.collect()
    ro.collect()
    res = {}

    def one():
        res["out"] = ro.collect()
    regions = _regions(one, reps)
    adv, ret, stats = res["out"]
    if not bool(stats["trajectory_finite"]) or not bool(torch.isfinite(adv).all()):
        raise FloatingPointError("non-finite league rollout")
    ms = float(np.median(regions))
    done = float(ro.b_done[1:].sum().item() + ro.next_done.sum().item())
    del ro
    eager = make(False)
    eager.collect()
    torch.cuda.synchronize()
    env = eager.env
    # (65,536 engagements exceed the single-launch step's residency: f16_env_step issues the
    # same two launches as fused_step=False, which lets the events time each of them)
    env.fused_step = False
    eager.policy_events, eager.opp_events, env.kernel_events, env.sim.kernel_events = [], [], [], []
    eager.collect()
    torch.cuda.synchronize()
    avg = lambda ev: float(np.mean([a.elapsed_time(b) for a, b in ev]))
    nac = 2 * nenv
    fdm_ms, post_ms = avg(env.sim.kernel_events), avg(env.kernel_events)
    lp_ms, op_ms = avg(eager.policy_events), avg(eager.opp_events)
    fdm_flop = _flop_per_substep("contest_60hz") * nac * env.substeps
    post_b = POST_BYTES_214_PER_AIRCRAFT * nac
    pol_flop = ppo.POLICY_FLOP_PER_ROW[214] * nenv
    opp_flop = (ppo.POLICY_FLOP_PER_ROW[214] - 2 * (256 * 214 + 256 * 256 + 256)) * nenv
    kernels = {
        "fdm": {"kernel": "fdm_step_quad_kernel<60, false, 2>", "ms": fdm_ms,
                "flop": fdm_flop, "achieved_TFLOPs": fdm_flop / (fdm_ms * 1e-3) / 1e12,
                "frac_fp64_peak": fdm_flop / (fdm_ms * 1e-3) / 1e12 / PEAK_FP64_TFLOPS},
        "post": {"kernel": "env_post_step_split_kernel<214, false>", "ms": post_ms,
                 "algorithmic_bytes": post_b, "achieved_GBs": post_b / (post_ms * 1e-3) / 1e9,
                 "frac_hbm_peak": post_b / (post_ms * 1e-3) / 1e9 / PEAK_HBM_GBS},
        "learner_policy": {"kernel": "policy_kernel (actor + critic, plane 0)", "ms": lp_ms,
                           "flop": pol_flop, "achieved_TFLOPs": pol_flop / (lp_ms * 1e-3) / 1e12,
                           "frac_bf16_peak": pol_flop / (lp_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS},
        "opponents_policy": {"kernel": "policy_kernel (8 grouped actors, plane 1)", "ms": op_ms,
                             "flop": opp_flop,
                             "achieved_TFLOPs": opp_flop / (op_ms * 1e-3) / 1e12,
                             "frac_bf16_peak": opp_flop / (op_ms * 1e-3) / 1e12 /
                             PEAK_BF16_TFLOPS}}
    out = {"workload": "league_rollout_64k_T128_214d_8opp", "engagements": nenv, "T": T,
           "opponents": nopp, "opponent_weights": "zipf(1.1)", "hip_graph": True,
           "ms_per_rollout": ms, "ms_per_rollout_regions": regions,
           "transitions_per_s": nenv * T / (ms * 1e-3),
           "aircraft_transitions_per_s": 2 * nenv * T / (ms * 1e-3),
           "learner_policy_ms": lp_ms, "opponents_policy_ms": op_ms,
           "fdm_kernel_ms": fdm_ms, "post_kernel_ms": post_ms, "kernels": kernels,
           "episodes_done_per_rollout": done,
           "streams": "opponents' grouping + launch on a second stream beside the learner's "
                      "normalisation + launch (the policy times overlap)"}
    return out


def fdm_section(pkg, icm, nenv, S, steps, warmup, reps, label, check_replay=True,
                require_finite=True, precision="fp64"):
    """The batched flight model alone: nenv tail-chase engagements (BASELINE configs[1]
    initial conditions), random 21-bin actions held per decision, `steps` decisions of S
    substeps per timed region, inputs resident in HBM.  Each region is timed `reps` times
    (median reported):
      graph  -- the `steps` GpuDogfight.step launches recorded once as a HIP graph and
                replayed: one launch per step back to back, the kernel's own rate;
      eager  -- the same steps as Python calls of GpuDogfight.step (each also validates its
                arguments and records its tensors' stream use on the host).
    A third pass with HIP events around each launch gives the launch duration on its own and
    checks that it reproduces the eager region's states bit for bit.  Every region starts from
    the same states (those after the warm-up decisions), so all regions time one trajectory.
    precision="fp32": the single-precision build (its state, actions and bytes in float)."""
    import torch
    nac = 2 * nenv
    sim = pkg.GpuDogfight(nenv, substeps=S, fcs_rate=120, precision=precision)
    bits = torch.int64 if precision == "fp64" else torch.int32
    sim.seed_rows(torch.as_tensor(icm.sample_tailchase(nenv, seed=0), device="cuda"))
    acts_host = icm.random_bin_actions(warmup + steps, nac, seed=0)
    acts = torch.as_tensor(acts_host, device="cuda", dtype=sim.dtype).contiguous()
    torch.cuda.synchronize()
    states0 = sim.states.cpu().numpy().copy()
    for k in range(warmup):
        sim.step(acts[k], want_obs=False)
    torch.cuda.synchronize()
    snap = sim.states.clone()

    def eager():
        for k in range(steps):
            sim.step(acts[warmup + k], want_obs=False)

    def reset():
        sim.states.copy_(snap)
    t0 = time.perf_counter()
    eager_ms = _regions(eager, reps, reset)
    wall = (time.perf_counter() - t0) / reps
    nonfinite = int((~torch.isfinite(sim.states).all(1)).sum())
    if require_finite and nonfinite:
        raise FloatingPointError("non-finite state after the timed steps")
    out = {"workload": label, "engagements": nenv, "aircraft": nac, "substeps_per_step": S,
           "fcs_rate_hz": 120, "steps_per_region": steps, "regions": reps,
           "precision": precision}
    if check_replay:
        # the launch on its own: one region again from the snapshot, events around each launch
        sim.states.copy_(snap)
        eager()
        after = sim.states.clone()
        sim.states.copy_(snap)
        sim.kernel_events = []
        eager()
        torch.cuda.synchronize()
        kev, sim.kernel_events = sim.kernel_events, None
        if not torch.equal(sim.states.view(bits), after.view(bits)):
            raise RuntimeError("the instrumented pass did not reproduce the timed steps")
        out["kernel_ms_per_launch_events"] = float(np.median([a.elapsed_time(b) for a, b in kev]))
    # the same steps recorded as a HIP graph
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            eager()
    torch.cuda.current_stream().wait_stream(side)
    graph_ms = _regions(g.replay, reps, reset)
    end = sim.states.clone()
    sim.states.copy_(snap)
    eager()
    if not torch.equal(sim.states.view(bits), end.view(bits)):
        raise RuntimeError("the graph replay did not reproduce the eager steps")
    del g
    gm, em = float(np.median(graph_ms)) / steps, float(np.median(eager_ms)) / steps
    flop = FLOP_PER_SUBSTEP * nac * S
    word = 8 if precision == "fp64" else 4
    peak = PEAK_FP64_TFLOPS if precision == "fp64" else PEAK_FP32_TFLOPS
    out.update({
        "nonfinite_aircraft_after_region": nonfinite,
        "ms_per_step": gm, "aircraft_substeps_per_s": nac * S / (gm * 1e-3),
        "graph_ms_per_step_regions": [x / steps for x in graph_ms],
        "eager_ms_per_step": em, "eager_aircraft_substeps_per_s": nac * S / (em * 1e-3),
        "eager_ms_per_step_regions": [x / steps for x in eager_ms],
        "eager_host_ms_per_step": wall * 1e3 / steps,
        "flop_per_launch": flop,
        "achieved_TFLOPs": flop / (gm * 1e-3) / 1e12,
        f"frac_{precision}_peak": flop / (gm * 1e-3) / 1e12 / peak,
        "algorithmic_bytes": FDM_BYTES_PER_AIRCRAFT // 8 * word * nac,
        "achieved_GBs": FDM_BYTES_PER_AIRCRAFT // 8 * word * nac / (gm * 1e-3) / 1e9})
    out["frac_hbm_peak"] = out["achieved_GBs"] / PEAK_HBM_GBS
    out["_states0"] = states0
    out["_acts_host"] = acts_host[warmup:]
    return out



def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--reps", type=int, default=5,
                    help="timed regions per section; each section reports the median")
    ap.add_argument("--nenv", type=int, default=16384)
    ap.add_argument("--substeps", type=int, default=6)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-rollout", action="store_true")
    ap.add_argument("--no-league", action="store_true")
    ap.add_argument("--no-update", action="store_true")
    ap.add_argument("--scan-finite", action="store_true",
                    help="with --only env: time only the two-launch step whose post-physics "
                         "launch re-reads the state for the finite flags (profiling aid)")
    ap.add_argument("--two-launch", action="store_true",
                    help="with --only env: time only the two-launch step (physics launch, then "
                         "post-physics launch; profiling aid)")
    ap.add_argument("--no-stagger", action="store_true",
                    help="with --only env or rollout: every engagement starts at t = 0 (profiling aid)")
    ap.add_argument("--rebuild-resets", action="store_true",
                    help="with --only env: autoresets rebuild their rows instead of copying the "
                         "pool tables (profiling aid)")
    ap.add_argument("--only", choices=["fdm", "env", "c3", "rollout", "league", "update"],
                    default=None,
                    help="profiling aid: run only this section and print its own JSON line "
                         "(not the contract line)")
    ap.add_argument("--precision", choices=["fp64", "fp32"], default="fp64",
                    help="with --only fdm: time this build of the flight model (profiling aid)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (rocprof counter "
                         "calibration: FETCH_SIZE/WRITE_SIZE of a copy of known size)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 8
        src = torch.ones(n, dtype=torch.float64, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 8, "copies": 5}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        sys.stderr.write("bench.py measures one GPU only: this build has no multi-GPU path "
                         "(engagements shard with zero communication).\n")
        sys.exit(2)

    import torch
    sys.path.insert(0, ROOT)
    pkg = importlib.import_module(PKG)
    icm = importlib.import_module(PKG + ".ic")
    if args.only in ("env", "c3", "rollout", "league", "update"):
        part = {"env": lambda: env_step_bench(pkg, args.nenv, args.steps, args.warmup,
                                              scan_finite=args.scan_finite, ab=False,
                                              stagger=not args.no_stagger,
                                              pool_tables=not args.rebuild_resets,
                                              two_launch=args.two_launch, reps=args.reps),
                "c3": lambda: obs_reward_c3_bench(args.nenv, args.steps, args.reps),
                "rollout": lambda: rollout_bench(args.nenv, reps=args.reps,
                                                 stagger=not args.no_stagger),
                "league": lambda: league_bench(reps=args.reps),
                "update": lambda: update_bench(args.nenv, reps=args.reps)}[args.only]()
        print(json.dumps(part), flush=True)
        return

    nenv, S = args.nenv, args.substeps
    nac = 2 * nenv
    # (long regions, as C2's 1,000 decisions, fly some aircraft past the model's range: counted,
    # not an error)
    prec = args.precision if args.only == "fdm" else "fp64"
    head = fdm_section(pkg, icm, nenv, S, args.steps, args.warmup, args.reps,
                       ("fdm_tailchase_16k" if nenv == 16384 else f"fdm_tailchase_{nenv}")
                       + ("_fp32" if prec == "fp32" else ""),
                       require_finite=args.steps <= 100, precision=prec)
    states0, acts_host = head.pop("_states0"), head.pop("_acts_host")
    if args.only == "fdm":
        print(json.dumps(head), flush=True)
        return
    # the other named sizes of the flight model: BASELINE C2 (4,096 tail-chase engagements,
    # its 1,000 decisions as one region), C5's 65,536 engagements, and one GPU's share of C4
    # on 8 and 2 GPUs (2,048 and 8,192 engagements: occupancy and tail effects)
    sizes = {}
    # and the single-precision build (GpuDogfight precision="fp32") at 16,384 and 65,536
    for ne, steps, label, prec in ((4096, 1000, "fdm_c2_tailchase_4k_1000dec", "fp64"),
                                   (65536, args.steps, "fdm_tailchase_64k", "fp64"),
                                   (2048, args.steps, "fdm_tailchase_2k", "fp64"),
                                   (8192, args.steps, "fdm_tailchase_8k", "fp64"),
                                   (16384, args.steps, "fdm_tailchase_16k_fp32", "fp32"),
                                   (65536, args.steps, "fdm_tailchase_64k_fp32", "fp32")):
        # C2 has no termination: over 1,000 decisions some aircraft fly into the ground and
        # past the model's range (counted in nonfinite_aircraft_after_region)
        r = fdm_section(pkg, icm, ne, S, steps, args.warmup, args.reps, label,
                        check_replay=False, require_finite=ne != 4096, precision=prec)
        r.pop("_states0"), r.pop("_acts_host")
        sizes[label] = r
    env_line = env_step_bench(pkg, nenv, args.steps, args.warmup, reps=args.reps)
    c3_line = obs_reward_c3_bench(nenv, args.steps, args.reps)
    rollout_line = None if args.no_rollout else rollout_bench(nenv)
    league_line = None if args.no_league else league_bench()
    update_line = None if args.no_update else update_bench(nenv)

    value = head["aircraft_substeps_per_s"]
    ms_step = head["ms_per_step"]
    line = {
        "metric": "aircraft FDM substeps/s + env transitions/s at 16k engagements; % vector roofline",
        "value": value,
        "unit": "aircraft-substeps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "regions": args.reps,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": value / REF_PUBLISHED_SUBSTEPS,
        "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": "fdm_tailchase_16k", "engagements": nenv, "aircraft": nac,
                   "substeps_per_step": S, "fcs_rate_hz": 120,
                   "actions": "i.i.d. uniform 21-bin per channel, held per decision",
                   "obs17": "not written (want_obs=False); the reference's kernel always "
                            "writes the 17-value output",
                   "timing": f"median of {args.reps} regions of {args.steps} steps, the steps "
                             "recorded once as a HIP graph and replayed (eager Python calls "
                             "reported beside it in fdm)"},
        "fdm": head,
        "fdm_sizes": sizes,
        "env_transitions_per_s": env_line["transitions_per_s"],
        "env_step": env_line,
        "obs_reward_c3": c3_line,
        "rollout": rollout_line,
        "league": league_line,
        "ppo_update": update_line,
        "roofline": {"bound": "valu", "achieved": head["achieved_TFLOPs"],
                     "peak": PEAK_FP64_TFLOPS, "unit": "TFLOP/s",
                     "frac": head["frac_fp64_peak"], "traffic": profiled_traffic(),
                     "kernel": "fdm_step_quad_kernel<120, false, 2>", "kernel_ms": ms_step,
                     "kernel_ms_source": "HIP events around each graph replay of one launch per "
                                         "step, / steps; median of the regions",
                     "kernel_ms_per_launch_events": head.get("kernel_ms_per_launch_events"),
                     "flop_per_launch": head["flop_per_launch"],
                     "flop_per_substep": FLOP_PER_SUBSTEP,
                     "flop_source": "op-counted CPU restatement, tests/golden/fdm_flops.json"},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(states0, acts_host, S, args.cpu_seconds, icm)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

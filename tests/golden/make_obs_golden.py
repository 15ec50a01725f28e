#!/usr/bin/env python3
"""Write the observation/reward golden vectors (tests/golden/obs_golden.npz) from the reference.

Why an import is used: the composed 184-D observation, the state9 bridge, the advance/reward/
termination sequence and the masked-reset re-initialisation have no host-compilable C source
(the reference's obs_kernel.cu is device-only) and no golden file; nothing else pins them.
This script imports the reference's own CPU torch path
  research/competition_36500/runtime/cuda_fdm/obs_reward.py  BatchObsReward(device="cpu",
      enable_kernel=False): push_actions, advance, compute_reward, build_obs,
      reset_envs, initialize_reward_state
  research/competition_36500/runtime/cuda_fdm/rl_env.py  kinematics_state,
      ned_from_ecef_altasl (the state9 bridge) and the _termination rule
IN THE BUILD CONTAINER ONLY, and stores inputs and outputs as arrays.  The aircraft states fed
in are produced here by the CPU restatement of the flight model (oracle/liborc.so) from
scripted initial conditions that force tail-chase damage, head-on mutual damage, hard-deck
exits, an HP death, a timeout and masked resets.

Usage:  python tests/golden/make_obs_golden.py [--ref /root/reference]
"""
import argparse
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, ROOT)

NENV = 12
STEPS = 10
MODES = (0, 1, 2, 3)


def scenario_ics():
    """(2*NENV, 10) IC rows and per-env (hp, t) overrides."""
    import importlib
    icm = importlib.import_module("2026_ai_pilot_challenge-1st_solution_amd.ic")
    rows, hp0, t0 = [], np.ones(2 * NENV), np.zeros(NENV)
    rng = np.random.default_rng(7)

    def pair(n_own, n_tgt, alt_own, alt_tgt, psi_own, psi_tgt, spd, e_off=0.0):
        la, lo, h = icm.ned_to_geodetic(np.array([n_own, n_tgt]), np.array([0.0, e_off]),
                                        -np.array([alt_own, alt_tgt]))
        return [icm.ic_row(la[0], lo[0], h[0], spd / 0.3048, psi_own, 6000.0),
                icm.ic_row(la[1], lo[1], h[1], spd / 0.3048, psi_tgt, 6000.0)]
    for e in range(NENV):
        if e < 3:        # tail chase 550-800 m: pursuer (plane 0) inside the tier-1 cone
            gap = 550.0 + 120.0 * e
            rows += pair(3500.0 - gap, 3500.0, 5000.0, 5000.0, 0.0, 0.0, 250.0)
        elif e < 5:      # head-on 700 m: mutual damage
            rows += pair(3500.0 - 350.0, 3500.0 + 350.0, 6000.0, 6000.0, 0.0, 180.0, 230.0)
        elif e < 7:      # one aircraft below the 304.8 m hard deck
            rows += pair(3500.0, 6500.0, 280.0 if e == 5 else 5000.0, 5000.0 if e == 5 else 250.0,
                         90.0, 270.0, 220.0)
        elif e == 7:     # timeout during the rollout
            rows += pair(2000.0, 6000.0, 7000.0, 7000.0, 30.0, 200.0, 240.0)
            t0[e] = 199.75
        elif e == 8:     # HP death: the target of a close tail chase starts nearly dead
            rows += pair(3500.0 - 600.0, 3500.0, 4000.0, 4000.0, 0.0, 0.0, 260.0)
            hp0[2 * e + 1] = 0.02
        else:            # random geometry, long range
            rows += pair(rng.uniform(0, 5000), rng.uniform(0, 5000), rng.uniform(2000, 9000),
                         rng.uniform(2000, 9000), rng.uniform(0, 360), rng.uniform(0, 360),
                         rng.uniform(180, 320), rng.uniform(-3000, 3000))
    return np.array(rows), hp0, t0


def make_inputs():
    import oracle_lib
    orc = oracle_lib.load()
    ic, hp0, t0 = scenario_ics()
    st = orc.seed(ic, 60)
    rng = np.random.default_rng(11)
    acts = rng.uniform(-0.3, 0.3, size=(STEPS, 2 * NENV, 4))
    acts[..., 3] = rng.uniform(0.5, 0.9, size=(STEPS, 2 * NENV))
    reset = np.zeros((STEPS, NENV), bool)
    reset[3, [5, 10]] = True           # re-seed two engagements after step 3
    reset[6, [0, 11]] = True
    fresh = orc.seed(scenario_ics()[0][::-1].copy(), 60)   # reseed rows (different ICs)
    states, states_reset = [], []
    for k in range(STEPS):
        orc.step(st, acts[k], 6, 60, want_obs=False)
        states.append(st.copy())
        if reset[k].any():
            for e in np.nonzero(reset[k])[0]:
                st[2 * e:2 * e + 2] = fresh[2 * e:2 * e + 2]
        states_reset.append(st.copy())
    return dict(states=np.array(states), states_reset=np.array(states_reset), actions=acts,
                reset=reset, hp0=hp0, t0=t0)


def child(ref_root, inp_path, out_path):
    R = os.path.join(ref_root, "research/competition_36500/runtime")
    for p in (os.path.join(ref_root, "src"), R):
        sys.path.insert(0, p)
    import torch
    from cuda_fdm import obs_reward as OR          # reference, build container only
    from cuda_fdm import rl_env as RE
    from dogfight.envs.termination import time_limit_reached
    inp = dict(np.load(inp_path))
    cfg = dict(OR.RW.MY_REWARD_CONFIG)

    def state9(st):
        ecef_m, euler, vuvw, alt_ft = RE.kinematics_state(torch.as_tensor(st))
        n, e, d = RE.ned_from_ecef_altasl(ecef_m, alt_ft * RE.FT2M)
        return torch.cat([torch.stack([n, e, d], 1), euler * RE.R2D, vuvw * RE.FT2M], 1)

    out = {}
    nenv = inp["reset"].shape[1]
    for mode in MODES:
        obr = OR.BatchObsReward(nenv, device="cpu", enable_kernel=False)
        obr.hp.copy_(torch.as_tensor(inp["hp0"]))
        obr.t_sec.copy_(torch.as_tensor(inp["t0"]))
        s9_0 = state9(inp["states"][0] * 0 + inp["states"][0])
        # the episode's first reward anchor comes from the initial (pre-step) state; use the
        # state after the first decision as the anchor for a deterministic fixture
        obr.initialize_reward_state(s9_0, None, cfg)
        rec = {k: [] for k in ("s9", "reward", "term", "trunc", "obs", "hp", "fuel", "t_sec",
                               "pqr", "hp_loss", "dealt", "taken", "prev_x", "prev_alt_log",
                               "act_hist", "obs_reset", "s9_reset")}
        for k in range(inp["actions"].shape[0]):
            obr.push_actions(torch.as_tensor(inp["actions"][k]))
            s9 = state9(inp["states"][k])
            obr.advance(s9)
            s9v = s9.view(nenv, 2, 9)
            alt = -s9v[:, :, 2]
            fin = torch.isfinite(s9v).all(dim=2)
            hp = obr.hp.view(nenv, 2)
            term = ((alt < RE.HARD_DECK_M).any(1) | (hp <= 0.0).any(1) | (~fin).any(1))
            trunc = time_limit_reached(obr.t_sec, 200.0) & (~term)
            r = obr.compute_reward(s9, term, cfg, trunc, reward_mode=mode, alt_hunt_coef=5.0)
            obs = obr.build_obs(s9)
            for key, val in (("s9", s9), ("reward", r), ("term", term), ("trunc", trunc),
                             ("obs", obs), ("hp", obr.hp), ("fuel", obr.fuel),
                             ("t_sec", obr.t_sec), ("pqr", obr.pqr), ("hp_loss", obr.hp_loss),
                             ("dealt", obr.last_dmg_dealt), ("taken", obr.last_dmg_taken),
                             ("prev_x", obr.prev_x), ("prev_alt_log", obr.prev_alt_log),
                             ("act_hist", obr.act_hist)):
                rec[key].append(val.clone().numpy())
            mask = torch.as_tensor(inp["reset"][k])
            s9r = state9(inp["states_reset"][k])
            if bool(mask.any()):
                obr.reset_envs(mask)
                obr.initialize_reward_state(s9r, mask, cfg)
            rec["obs_reset"].append(obr.build_obs(s9r).numpy())
            rec["s9_reset"].append(s9r.numpy())
        for key, v in rec.items():
            out[f"m{mode}_{key}"] = np.array(v)
    np.savez_compressed(out_path, **out)


def child_root214(ref_root, inp_path, out_path):
    """The root lineage's CPU torch path (cuda_fdm/obs_reward.py, 214-D observation): advance
    forms the NED-velocity step difference (cuda_fdm/obs_reward.py:569-575) and build_obs writes
    it through the 10 accel (vector, frame) pairs (:702-712; layout claude_code/my_observation.py
    VECTOR_SPECS).  Same scripted states and resets as the 184-D golden; reward mode 0 only
    (the reconstructor and the observation do not depend on the mode)."""
    for p in (os.path.join(ref_root, "src"), ref_root):
        sys.path.insert(0, p)
    import torch
    from cuda_fdm import obs_reward as OR          # reference, build container only
    from cuda_fdm import rl_env as RE
    from dogfight.envs.termination import time_limit_reached
    assert OR.OBS_SIZE == 214
    inp = dict(np.load(inp_path))
    cfg = dict(OR.RW.MY_REWARD_CONFIG)

    def state9(st):
        ecef_m, euler, vuvw, alt_ft = RE.kinematics_state(torch.as_tensor(st))
        n, e, d = RE.ned_from_ecef_altasl(ecef_m, alt_ft * RE.FT2M)
        return torch.cat([torch.stack([n, e, d], 1), euler * RE.R2D, vuvw * RE.FT2M], 1)

    nenv = inp["reset"].shape[1]
    obr = OR.BatchObsReward(nenv, device="cpu", enable_kernel=False)
    obr.hp.copy_(torch.as_tensor(inp["hp0"]))
    obr.t_sec.copy_(torch.as_tensor(inp["t0"]))
    obr.initialize_reward_state(state9(inp["states"][0]), None, cfg)
    rec = {k: [] for k in ("obs", "accel", "prev_vel_ned", "reward", "term", "trunc",
                           "obs_reset", "accel_reset", "prev_vel_ned_reset")}
    for k in range(inp["actions"].shape[0]):
        obr.push_actions(torch.as_tensor(inp["actions"][k]))
        s9 = state9(inp["states"][k])
        obr.advance(s9)
        s9v = s9.view(nenv, 2, 9)
        fin = torch.isfinite(s9v).all(dim=2)
        hp = obr.hp.view(nenv, 2)
        term = ((-s9v[:, :, 2] < RE.HARD_DECK_M).any(1) | (hp <= 0.0).any(1) | (~fin).any(1))
        trunc = time_limit_reached(obr.t_sec, 200.0) & (~term)
        r = obr.compute_reward(s9, term, cfg, trunc, reward_mode=0, alt_hunt_coef=5.0)
        for key, val in (("obs", obr.build_obs(s9)), ("accel", obr.accel),
                         ("prev_vel_ned", obr.prev_vel_ned), ("reward", r), ("term", term),
                         ("trunc", trunc)):
            rec[key].append(val.clone().numpy())
        mask = torch.as_tensor(inp["reset"][k])
        s9r = state9(inp["states_reset"][k])
        if bool(mask.any()):
            obr.reset_envs(mask)
            obr.initialize_reward_state(s9r, mask, cfg)
        rec["obs_reset"].append(obr.build_obs(s9r).numpy())
        rec["accel_reset"].append(obr.accel.clone().numpy())
        rec["prev_vel_ned_reset"].append(obr.prev_vel_ned.clone().numpy())
    np.savez_compressed(out_path, **{f"a214_{k}": np.array(v) for k, v in rec.items()})


def main_root214(ref):
    """Write obs214_golden.npz from the inputs stored in obs_golden.npz."""
    g = dict(np.load(os.path.join(HERE, "obs_golden.npz")))
    inp = {k[3:]: v for k, v in g.items() if k.startswith("in_")}
    with tempfile.TemporaryDirectory() as td:
        ip, op = os.path.join(td, "in.npz"), os.path.join(td, "out.npz")
        np.savez(ip, **inp)
        subprocess.run([sys.executable, __file__, "--ref", ref, "--child-root214", ip, op],
                       check=True)
        res = dict(np.load(op))
    np.savez_compressed(os.path.join(HERE, "obs214_golden.npz"), **res)
    print("wrote obs214_golden.npz", len(res), "arrays",
          os.path.getsize(os.path.join(HERE, "obs214_golden.npz")) // 1024, "KiB")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--child", nargs=2)
    ap.add_argument("--child-root214", nargs=2)
    ap.add_argument("--root214", action="store_true",
                    help="write obs214_golden.npz (root lineage, 214-D) from obs_golden's inputs")
    a = ap.parse_args()
    if a.child:
        child(a.ref, *a.child)
        return
    if a.child_root214:
        child_root214(a.ref, *a.child_root214)
        return
    if a.root214:
        main_root214(a.ref)
        return
    inp = make_inputs()
    with tempfile.TemporaryDirectory() as td:
        ip, op = os.path.join(td, "in.npz"), os.path.join(td, "out.npz")
        np.savez(ip, **inp)
        subprocess.run([sys.executable, __file__, "--ref", a.ref, "--child", ip, op], check=True)
        res = dict(np.load(op))
    # observations and reconstructor state do not depend on the reward mode: keep mode 0's
    for key in list(res):
        mode, name = key.split("_", 1)
        if mode != "m0" and name not in ("reward", "prev_x", "prev_alt_log"):
            assert np.array_equal(res[key], res["m0_" + name]), key
            del res[key]
    res.update({f"in_{k}": v for k, v in inp.items()})
    np.savez_compressed(os.path.join(HERE, "obs_golden.npz"), **res)
    print("wrote obs_golden.npz", len(res), "arrays",
          os.path.getsize(os.path.join(HERE, "obs_golden.npz")) // 1024, "KiB")


if __name__ == "__main__":
    main()

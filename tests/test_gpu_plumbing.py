"""The CPU-runnable NR plumbing workload (64 envs x 8 robots, one cell, K = 4 UL slots, round robin, 4 HARQ x 4
transmissions, 1500 B at Poisson 0.5, FIFO 16, UMi LOS, i.i.d. Rayleigh fading) at its full size and run length:
1000 control steps on the GPU against the oracle on every env, free running from the same seed, with partial resets.
Every env whose integer results differ from the oracle's must be a proven float-threshold flip."""
import numpy as np
import pytest
import torch

import isaac_net_amd as P
from gpu_util import head, submit_oracle
from oracle import nr_oracle as O
from oracle.tolerance import FlipCounter, engine_radio, sinr_bound

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_plumbing_full_run_against_oracle():
    from isaac_net_amd import scenarios as B
    E, R, steps = 64, 8, 1000
    print(f"plumbing {E}x{R}, {steps} steps, oracle on every env", flush=True)
    wl = B.Workload(E, R, steps, seed=1, name="plumbing")
    cfg = wl.cfg
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=1)
    ora = O.OracleEngine(E, R, cfg, seed=1)
    fc = FlipCounter(E, ora)
    fi, sig, amp = engine_radio(eng)
    rs = np.random.default_rng(5)
    n_tx = 0
    for s in range(steps):
        if s and s % 97 == 0:                            # an episode ends for a few envs now and then
            ids = sorted(rs.choice(E, 3, replace=False).tolist())
            eng.reset(ids)
            ora.reset(ids)
        c = wl.counts[s]
        eng.submit_counts(c.to(DEV))
        submit_oracle(ora, c.numpy())
        x = wl.poses[s]
        og = eng.step(None, x.to(DEV))
        fc.before()
        oo = ora.step(None, x)
        tol = sinr_bound(x.numpy(), eng.st["field"][:, 0, fi].cpu().numpy(), sig, amp, oo["sinr_db"].numpy())
        fc.step(s, og, oo, tol, head(eng.owner_state(), E), lambda o, x=x: o.step(None, x))
        n_tx += int(og["delivered"].sum())
        if s % 200 == 199:
            print(f"step {s + 1}: {fc.report()}", flush=True)
    c = eng.counters()["ul"]
    print(f"delivered {n_tx}; TBs {c['tb_new']:.0f} new, {c['tb_retx']:.0f} retx, {c['exhaust']:.0f} exhausted; "
          f"{fc.report()}", flush=True)
    assert n_tx > 0 and c["tb_retx"] > 0
    assert fc.ok(E * R * steps), fc.report()

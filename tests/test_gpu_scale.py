"""The RL-scale workload (4096 envs x 32 robots, K = 10 UL slots, PF, Rician K 3 dB, two message classes) at its
real shape: queue and HARQ invariants over every env, and parity of its first envs with the oracle over 200 control
steps (envs are independent: the oracle on the first envs sees exactly their inputs and keys), long enough for the PF
averages (EWMA 0.01) to settle and for RLC retransmissions (50 slots after an exhausted HARQ process). Every env whose integer results differ from the oracle's must be a proven float-threshold flip."""
import numpy as np
import pytest
import torch

import isaac_net_amd as P
from gpu_util import head, submit_oracle
from oracle import nr_oracle as O
from oracle.tolerance import FlipCounter, engine_radio, sinr_bound

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_rl_scale_invariants_and_prefix_parity():
    from isaac_net_amd import scenarios as B
    cfg = B.rl_scale_config()
    E, R, steps, E_chk = 4096, 32, 200, 24
    print(f"rl-scale {E}x{R}, {steps} steps, oracle on {E_chk} envs", flush=True)
    wl = B.Workload(E, R, steps, seed=0, device=DEV)
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=0)
    ora = O.OracleEngine(E_chk, R, cfg, seed=0)
    fc = FlipCounter(E_chk, ora)
    fi, sig, amp = engine_radio(eng)
    for s in range(steps):
        counts = wl.counts[s]
        eng.submit_counts(counts)
        submit_oracle(ora, counts[:E_chk].cpu().numpy())
        og = eng.step(None, wl.poses[s])
        x = wl.poses[s][:E_chk].cpu()
        fc.before()
        oo = ora.step(None, x)
        tol = sinr_bound(x.numpy(), eng.st["field"][:E_chk, 0, fi].cpu().numpy(), sig, amp, oo["sinr_db"].numpy())
        st = eng.owner_state()
        fc.step(s, {k: v[:E_chk] for k, v in og.items() if v.dim() >= 2}, oo, tol, head(st, E_chk),
                lambda o, x=x: o.step(None, x))
        if s % 10 == 9 or s == steps - 1:
            qlen = eng.st["qlen"]
            assert int(qlen.max()) <= cfg.frame_buffer and int(qlen.min()) >= 0
            valid = st["ul.q.cap"] >= 0
            assert torch.equal(valid.sum(-1), qlen.long())                 # valid frames form a prefix
            assert bool((valid[..., 1:] <= valid[..., :-1]).all())
            hs = st["ul.h_state"]
            assert bool(((hs == 0) | (hs == 1)).all())
            assert bool((st["ul.sent"] <= st["ul.q.enq"]).all()) and bool((st["ul.floor"] <= st["ul.sent"]).all())
            assert bool((og["queue_bytes"] >= 0).all())
        if s % 50 == 49:
            print(f"step {s + 1}: {fc.report()}", flush=True)
    c = eng.counters()["ul"]
    print(f"prefix parity: {E_chk} envs x {steps} steps: {fc.report()}; TBs {c['tb_new']:.0f} new, "
          f"{c['exhaust']:.0f} exhausted", flush=True)
    assert fc.ok(E_chk * R * steps), fc.report()

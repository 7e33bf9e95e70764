"""The RL-scale workload (4096 envs x 32 robots, K = 10 UL slots, PF, Rician K 3 dB, two message classes) at its
real shape: queue and HARQ invariants over every env, and parity of its first envs with the oracle (envs are
independent: the oracle on the first envs sees exactly their inputs and keys)."""
import numpy as np
import pytest
import torch

import isaac_net_amd as P
from oracle import nr_oracle as O
from oracle.tolerance import FlipCounter, engine_radio, sinr_bound

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_rl_scale_invariants_and_prefix_parity():
    from isaac_net_amd import scenarios as B
    cfg = B.rl_scale_config()
    E, R, steps, E_chk = 4096, 32, 12, 24
    print(f"rl-scale {E}x{R}, {steps} steps", flush=True)
    wl = B.Workload(E, R, steps, seed=0, device=DEV)
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=0)
    ora = O.OracleEngine(E_chk, R, cfg, seed=0)
    fc = FlipCounter(E_chk)
    fi, sig, amp = engine_radio(eng)
    for s in range(steps):
        counts = wl.counts[s]
        eng.submit_counts(counts)
        c = counts[:E_chk].cpu().numpy()
        for ci in range(c.shape[-1]):
            for i in range(int(c[..., ci].max())):
                ora.submit(None, torch.from_numpy(np.where(c[..., ci] > i, ci + 1, 0).astype(np.int64)))
        og = eng.step(None, wl.poses[s])
        oo = ora.step(None, wl.poses[s][:E_chk].cpu())
        tol = sinr_bound(wl.poses[s][:E_chk].cpu().numpy(), eng.st["field"][:E_chk, 0, fi].cpu().numpy(), sig, amp,
                         oo["sinr_db"].numpy())
        fc.step(s, {k: v[:E_chk] for k, v in og.items() if v.dim() >= 2}, oo, tol)
        st = eng.owner_state()
        qlen = eng.st["qlen"]
        assert int(qlen.max()) <= cfg.frame_buffer and int(qlen.min()) >= 0
        cap = st["ul.q.cap"]
        valid = cap >= 0
        assert torch.equal(valid.sum(-1), qlen.long())                     # valid frames form a prefix
        assert bool((valid[..., 1:] <= valid[..., :-1]).all())
        hs = st["ul.h_state"]
        assert bool(((hs == 0) | (hs == 1)).all())
        assert bool((st["ul.sent"] <= st["ul.q.enq"]).all()) and bool((st["ul.floor"] <= st["ul.sent"]).all())
        assert bool((og["queue_bytes"] >= 0).all())
    print(f"prefix parity: {E_chk} envs x {steps} steps, integer flips {fc.flips}, float issues {fc.float_bad}",
          flush=True)
    assert len(fc.flips) <= 1 and not fc.float_bad

"""Envs of 65..128 robots (one workgroup of two wavefronts per env) at the frequency-selective stress shape: 16384
envs x 128 robots, 273 PRB in 8 RBGs, K = 20, against the oracle on the first envs (envs are independent: the
oracle on the first envs sees exactly their inputs and keys), with queue and HARQ invariants over every env."""
import numpy as np
import pytest
import torch

import isaac_net_amd as P
from oracle import nr_oracle as O
from oracle.tolerance import FlipCounter, engine_radio, sinr_bound

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_freq_sel_prefix_parity_and_invariants():
    from isaac_net_amd import scenarios as B
    E, R, steps, E_chk = 16384, 128, 3, 4
    print(f"freq_sel {E}x{R}, {steps} steps", flush=True)
    wl = B.Workload(E, R, steps, seed=0, device=DEV, name="freq_sel")
    cfg = wl.cfg
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=0)
    ora = O.OracleEngine(E_chk, R, cfg, seed=0)
    fc = FlipCounter(E_chk)
    fi, sig, amp = engine_radio(eng)
    for s in range(steps):
        counts = wl.counts[s]
        og = eng.step(None, wl.poses[s], arrivals=counts)
        c = counts[:E_chk].cpu().numpy()
        for ci in range(c.shape[-1]):
            for i in range(int(c[..., ci].max())):
                ora.submit(None, torch.from_numpy(np.where(c[..., ci] > i, ci + 1, 0).astype(np.int64)))
        oo = ora.step(None, wl.poses[s][:E_chk].cpu())
        tol = sinr_bound(wl.poses[s][:E_chk].cpu().numpy(), eng.st["field"][:E_chk, 0, fi].cpu().numpy(), sig, amp,
                         oo["sinr_db"].numpy())
        fc.step(s, {k: v[:E_chk] for k, v in og.items() if v.dim() >= 2}, oo, tol)
        qlen = eng.st["qlen"]
        assert int(qlen.max()) <= cfg.frame_buffer and int(qlen.min()) >= 0
        st = eng.owner_state()
        valid = st["ul.q.cap"] >= 0
        assert torch.equal(valid.sum(-1), qlen.long())
        assert bool((valid[..., 1:] <= valid[..., :-1]).all())
        assert bool(((st["ul.h_state"] == 0) | (st["ul.h_state"] == 1)).all())
        assert bool((st["ul.sent"] <= st["ul.q.enq"]).all()) and bool((st["ul.floor"] <= st["ul.sent"]).all())
    assert eng.counters()["ul"]["tb_new"] > 0
    print(f"prefix parity: {E_chk} envs x {steps} steps, integer flips {fc.flips}, float issues {fc.float_bad}",
          flush=True)
    assert len(fc.flips) <= 1 and not fc.float_bad

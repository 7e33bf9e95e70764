"""Envs of 65..128 robots (one workgroup of two wavefronts per env) at the frequency-selective stress shape: 16384
envs x 128 robots, 273 PRB in 8 RBGs, K = 20, against the oracle on the first envs over 40 control steps (envs are
independent: the oracle on the first envs sees exactly their inputs and keys), with queue and HARQ invariants over
every env. Every env whose integer results differ from the oracle's must be a proven float-threshold flip."""
import pytest

import isaac_net_amd as P
from gpu_util import head, submit_oracle
from oracle import nr_oracle as O
from oracle.tolerance import FlipCounter, engine_radio, sinr_bound

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_freq_sel_prefix_parity_and_invariants():
    from isaac_net_amd import scenarios as B
    E, R, steps, E_chk = 16384, 128, 40, 4
    print(f"freq_sel {E}x{R}, {steps} steps, oracle on {E_chk} envs", flush=True)
    wl = B.Workload(E, R, steps, seed=0, device=DEV, name="freq_sel")
    cfg = wl.cfg
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=0)
    ora = O.OracleEngine(E_chk, R, cfg, seed=0)
    fc = FlipCounter(E_chk, ora)
    fi, sig, amp = engine_radio(eng)
    for s in range(steps):
        counts = wl.counts[s]
        og = eng.step(None, wl.poses[s], arrivals=counts)
        submit_oracle(ora, counts[:E_chk].cpu().numpy())
        x = wl.poses[s][:E_chk].cpu()
        fc.before()
        oo = ora.step(None, x)
        tol = sinr_bound(x.numpy(), eng.st["field"][:E_chk, 0, fi].cpu().numpy(), sig, amp, oo["sinr_db"].numpy())
        st = eng.owner_state()
        fc.step(s, {k: v[:E_chk] for k, v in og.items() if v.dim() >= 2}, oo, tol, head(st, E_chk),
                lambda o, x=x: o.step(None, x))
        if s % 10 == 9:
            qlen = eng.st["qlen"]
            assert int(qlen.max()) <= cfg.frame_buffer and int(qlen.min()) >= 0
            valid = st["ul.q.cap"] >= 0
            assert (valid.sum(-1) == qlen.long()).all()
            assert bool((valid[..., 1:] <= valid[..., :-1]).all())
            assert bool(((st["ul.h_state"] == 0) | (st["ul.h_state"] == 1)).all())
            assert bool((st["ul.sent"] <= st["ul.q.enq"]).all()) and bool((st["ul.floor"] <= st["ul.sent"]).all())
            print(f"step {s + 1}: {fc.report()}", flush=True)
    assert eng.counters()["ul"]["tb_new"] > 0
    print(f"prefix parity: {E_chk} envs x {steps} steps: {fc.report()}", flush=True)
    assert fc.ok(E_chk * R * steps), fc.report()

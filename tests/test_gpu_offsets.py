"""The int32 byte offsets and their 64-bit base (InetNrState.base / InetNrDlState.base): the reference keeps every
byte-stream offset in int64 (isaac_net/core/queues.py:52-60, mac.py:67-81); the step kernel keeps int32 values
and, once a robot's floor reaches the rebase threshold, moves its offsets down by the floor into the base.

- With a 4 KiB threshold every busy robot rebases at almost every step: the reference trajectories must stay
  bit-exact, state included (the reference-layout state adds the base back).
- A run loaded with every offset near 2^31 (beyond the int32 range of the old layout) must equal the oracle,
  whose offsets are int64."""
import numpy as np
import pytest
import torch

import isaac_net_amd as P
from gpu_util import compare, head, load, set_radio_bound, submit_oracle
from oracle import nr_oracle as O
from oracle import replay
from oracle.tolerance import FlipCounter, engine_radio, sinr_bound

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("name", ["c2heavy", "dl_c2", "mc3_ho"])
def test_reference_trajectory_with_rebase_every_step(name):
    print(f"case {name} free running, rebase threshold 4096 B", flush=True)
    ref, cfgd, kind = load(name)
    cfg = P.NRConfig(**cfgd, seed=0)
    E, R = int(ref["E"]), int(ref["R"])
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=0)
    eng.REBASE_AT = 4096
    eng._cparams.rebase_at = 4096
    bad, n_reb = [], [0]

    def on_step(s, o, acc):
        set_radio_bound(ref, s, cfg, eng, kind)
        bi, bf, _ = compare(ref, s, o, eng.owner_state(), E, R)
        if bi or bf:
            bad.append((s, bi, bf))
        n_reb[0] = int((eng.st["base"] > 0).sum())
    replay.run(eng, ref, kind, on_step=on_step, to=lambda a: torch.from_numpy(np.asarray(a)).to(DEV))
    print(f"{name}: robots with a rebased stream at the end: {n_reb[0]}", flush=True)
    assert not bad, bad[:3]
    assert n_reb[0] > 0


def test_offsets_near_int32_limit_against_oracle():
    """rl_scale shrunk to 16 envs, every byte offset shifted by 2^31 - 5000 after 5 steps, then 30 steps free
    running against the oracle (int64)."""
    from isaac_net_amd import scenarios as B
    E, R, steps, shift = 16, 32, 35, (1 << 31) - 5000
    wl = B.Workload(E, R, steps, seed=2)
    cfg = wl.cfg
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=2)
    ora = O.OracleEngine(E, R, cfg, seed=2)
    fc = FlipCounter(E, ora)
    fi, sig, amp = engine_radio(eng)
    keys = ("sent", "floor", "h_lo", "h_hi", "q.start", "q.end", "q.enq")
    for s in range(steps):
        if s == 5:                                     # shift the streams of both sides
            sd = ora.state()
            for k in keys:
                sd["ul." + k] = sd["ul." + k] + shift
            ora.load_state(sd, ora.T, ora.last_g)
            eng.load_owner_state({k: v.clone() for k, v in ora.state().items()}, T=eng.T, last_g=eng.last_g)
            assert int(eng.st["base"].min()) >= shift and int(eng.st["floor_"].max()) < 1 << 30
        c = wl.counts[s]
        eng.submit_counts(c.to(DEV))
        submit_oracle(ora, c.numpy())
        x = wl.poses[s]
        og = eng.step(None, x.to(DEV))
        fc.before()
        oo = ora.step(None, x)
        tol = sinr_bound(x.numpy(), eng.st["field"][:, 0, fi].cpu().numpy(), sig, amp, oo["sinr_db"].numpy())
        fc.step(s, og, oo, tol, head(eng.owner_state(), E), lambda o, x=x: o.step(None, x))
    st = eng.owner_state()
    assert int(st["ul.q.enq"].max()) > 1 << 31                        # beyond the int32 range
    print(fc.report(), flush=True)
    assert fc.ok(E * R * steps), fc.report()

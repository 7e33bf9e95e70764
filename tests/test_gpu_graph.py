"""HIP-graph replay of a control step (HipNREngine.graph_step) against eager launches of the same engine build.

Two engines with the same seed and inputs: one steps eagerly, the other replays its recorded graphs. Outputs and the
whole state must be bitwise equal after every step, with eager work between the replays (a partial reset, host
syncs, state reads), as the graphs read the control step from the device clock."""
import numpy as np
import pytest
import torch

from conftest import load_package

pytestmark = pytest.mark.gpu


def _same(a, b):
    a, b = a.detach().cpu(), b.detach().cpu()
    if a.dtype.is_floating_point:
        return bool(((a == b) | (torch.isnan(a) & torch.isnan(b))).all())
    return torch.equal(a, b)


def test_graph_replay_matches_eager():
    P = load_package()
    from isaac_net_amd import scenarios as S
    E, R, steps = 64, 32, 9
    wl = S.Workload(E, R, steps, seed=3, device="cuda:0")
    a = P.make_engine("L2", E, R, "cuda:0", wl.cfg, seed=0)
    b = P.make_engine("L2", E, R, "cuda:0", wl.cfg, seed=0)
    for eng in (a, b):                       # the first step has its own fading slot spacing: eager on both
        eng.submit_counts(wl.counts[0])
        eng.step(None, wl.poses[0])
    g = b.graph_step()
    for s in range(1, steps):
        if s == 4:
            a.reset([1, 5, 40])
            b.reset([1, 5, 40])
        a.submit_counts(wl.counts[s])
        oa = a.step(None, wl.poses[s])
        ob = g(wl.poses[s], wl.counts[s])
        torch.cuda.synchronize()
        print(f"step {s}: clock {a.T} / {b.T}", flush=True)
        assert a.T == b.T
        for k in oa:
            assert _same(oa[k], ob[k]), (s, k)
        sa, sb = a.owner_state(), b.owner_state()
        for k in sa:
            if torch.is_tensor(sa[k]):
                assert _same(sa[k], sb[k]), (s, k)
    assert a.counters() == b.counters()


def test_graph_records_one_step_per_schedule():
    """With 3 slots per control step the TDD phase moves from step to step: the graph step records one graph per
    schedule key and replays each, bitwise equal to eager launches over two periods of the pattern."""
    P = load_package()
    from isaac_net_amd import scenarios as S
    E, R = 8, 32
    cfg = S.rl_scale_config(control_step_ms=1.5)
    a = P.make_engine("L2", E, R, "cuda:0", cfg, seed=0)
    b = P.make_engine("L2", E, R, "cuda:0", cfg, seed=0)
    g = b.graph_step()
    gen = torch.Generator().manual_seed(5)
    for s in range(12):
        pos = (torch.rand(E, R, 2, generator=gen) * 100).to("cuda:0")
        cnt = (torch.rand(E, R, 2, generator=gen) < 0.3).to(torch.uint8).to("cuda:0")
        a.submit_counts(cnt)
        oa = a.step(None, pos)
        ob = g(pos, cnt)
        torch.cuda.synchronize()
        for k in oa:
            assert _same(oa[k], ob[k]), (s, k)
        sa, sb = a.owner_state(), b.owner_state()
        for k in sa:
            if torch.is_tensor(sa[k]):
                assert _same(sa[k], sb[k]), (s, k)
    assert 1 < len(g.steps) <= 12

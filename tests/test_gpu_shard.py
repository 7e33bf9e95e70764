"""Shard invariance (isaac_net/core/sharded.py:61-78): an engine keyed by global env ids with set_env_offset gives, for
every env it holds, the bits an unsharded engine gives for that env. Two half-size engines with offsets 0 and E/2 are
run beside one full-size engine on the same inputs (the RL-scale configuration with arrivals inside the step launch,
the three-cell configuration, and level WIFI), step by step, with a partial reset on the way."""
import pytest
import torch

import isaac_net_amd as P
from isaac_net_amd import scenarios as B

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _same(a, b, what):
    for k in b:
        if torch.is_tensor(a[k]):
            x, y = a[k], b[k]
            eq = torch.equal(x, y) if not x.is_floating_point() else \
                bool(((x == y) | (torch.isnan(x) & torch.isnan(y))).all())
            assert eq, f"{what}: {k} differs between the sharded and the unsharded engine"


@pytest.mark.parametrize("name,E,R,steps", [("rl_scale", 8, 32, 12), ("mc_interf", 4, 16, 8)])
def test_nr_shards_equal_unsharded(name, E, R, steps):
    print(f"shards {name} {E}x{R}, {steps} steps", flush=True)
    wl = B.Workload(E, R, steps, seed=7, name=name)
    full = P.make_engine("L2", E, R, DEV, wl.cfg, seed=7)
    h = E // 2
    parts = [P.make_engine("L2", h, R, DEV, wl.cfg, seed=7) for _ in range(2)]
    P.set_env_offset(parts[1], h)
    P.set_env_offset(parts[0], 0)                     # (no change: the ids are already global)
    for s in range(steps):
        if s == steps // 2:
            full.reset([1, h + 1])
            parts[0].reset([1])
            parts[1].reset([1])
        c, x = wl.counts[s].to(DEV), wl.poses[s].to(DEV)
        of = full.step(None, x, arrivals=c)
        o0 = parts[0].step(None, x[:h], arrivals=c[:h].contiguous())
        o1 = parts[1].step(None, x[h:].contiguous(), arrivals=c[h:].contiguous())
        og = {k: torch.cat([o0[k], o1[k]]) for k in of if torch.is_tensor(of[k]) and of[k].dim() > 0}
        _same(of, og, f"{name} step {s}")
    sf = full.owner_state()
    s0, s1 = parts[0].owner_state(), parts[1].owner_state()
    _same(sf, {k: torch.cat([s0[k], s1[k]]) for k in sf if torch.is_tensor(sf[k]) and sf[k].shape[:1] == (E,)},
          f"{name} final state")
    assert int(parts[1].st["env_id"][0]) == h and int(parts[1].st["episode"].max()) == 1


def test_wifi_shards_equal_unsharded():
    E, R, steps = 8, 16, 6
    wl = B.Workload(E, R, steps, seed=5, name="wifi_dcf")
    full = P.make_engine("WIFI", E, R, DEV, wl.cfg, seed=5)
    h = E // 2
    parts = [P.make_engine("WIFI", h, R, DEV, wl.cfg, seed=5) for _ in range(2)]
    P.set_env_offset(parts[1], h)
    for s in range(steps):
        c, x = wl.counts[s].to(DEV), wl.poses[s].to(DEV)
        full.submit_counts(c)
        parts[0].submit_counts(c[:h].contiguous())
        parts[1].submit_counts(c[h:].contiguous())
        of = full.step(None, x)
        o0, o1 = parts[0].step(None, x[:h]), parts[1].step(None, x[h:].contiguous())
        _same(of, {k: torch.cat([o0[k], o1[k]]) for k in of if torch.is_tensor(of[k]) and of[k].dim() > 0},
              f"wifi step {s}")

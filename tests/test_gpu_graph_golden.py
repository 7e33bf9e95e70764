"""HIP-graph replay (HipNREngine.graph_step) against the reference trajectories (tests/golden/traj_*.npz): every
case, the downlink and several-cells cases included, driven through the graph step from the first step (resets and
DL frames eagerly between the replays, the step's messages through the recorded counts-form enqueue). Outputs and
state are compared after every replay with the rules of the free-running parity test (gpu_util.compare)."""
import numpy as np
import pytest
import torch

from conftest import CASES, DL_CASES, MC_CASES
import gpu_util
from gpu_util import compare, load, set_radio_bound
from oracle import replay
import isaac_net_amd as P

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("name", CASES + DL_CASES + MC_CASES)
def test_graph_replay_matches_reference(name):
    print(f"case {name} graph replay", flush=True)
    ref, cfgd, kind = load(name)
    cfg = P.NRConfig(**cfgd, seed=0)
    E, R, T = int(ref["E"]), int(ref["R"]), int(ref["steps"])
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=0)
    g = eng.graph_step(ref["counts"].shape[-1])
    to = lambda a: torch.from_numpy(np.asarray(a)).to(DEV)  # noqa: E731
    bad = []
    for s in range(T):
        ids = np.nonzero(ref["reset_mask"][s])[0]
        if len(ids):
            eng.reset(ids.tolist())
        for nb, cls in replay.dl_frames(ref, s):
            eng.add_dl_frames(None, to(nb), to(cls))
        cnt = to(ref["counts"][s].astype(np.uint8))
        x = to(ref["x"][s])
        vel = to(ref["vel"][s]) if "vel" in ref.files else None
        if kind == "snr3":
            o = g(counts=cnt, snr_db=x)
        elif kind == "pg":
            o = g(counts=cnt, pathgain_db=x)
        else:
            o = g(x, cnt, vel=vel)
        torch.cuda.synchronize()
        set_radio_bound(ref, s, cfg, eng, kind)
        bi, bf, _ = compare(ref, s, o, eng.owner_state(), E, R)
        if bi or bf:
            bad.append((s, bi, bf))
    print(f"{name}: {len(g.steps)} step graphs; max |deviation| "
          f"{ {k: f'{v:.2e}' for k, v in gpu_util.MAX_DEV.items()} }", flush=True)
    gpu_util.MAX_DEV.clear()
    assert not bad, bad[:5]

"""Checkpoints on the GPU (core/checkpoint.py:103-143 semantics): a checkpoint written by the reference's NR engine
(tests/golden/ckpt_*.npz, its state_dict() after 10 steps of a golden case: one cell, the downlink, three cells with
handovers, the 5G-LENA MAC switches with their grant counters and the last PUSCH's PRBs) loads into the hip engine, which then
continues bit for bit along the reference's trajectory (outputs, state and counters as in the free-running parity
test); and checkpoint.save / load of the hip engine resumes exactly like the uninterrupted run."""
import json
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
import gpu_util
from gpu_util import compare, load, set_radio_bound
from oracle import replay
import isaac_net_amd as P
from isaac_net_amd import checkpoint

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def reference_checkpoint(name):
    z = np.load(os.path.join(GOLDEN, f"ckpt_{name}.npz"), allow_pickle=False)
    sd = {k[3:]: torch.from_numpy(np.array(z[k])) for k in z.files if k.startswith("ck/")}
    sd.update(json.loads(bytes(z["host_json"]).decode()))
    return sd, int(z["k_steps"])


@pytest.mark.parametrize("name", ["c2", "dl_c2", "mc3_ho", "lena_v2", "fcorr", "rice_los",
                                  "rice_sto_slow", "fcorr_los"])
def test_reference_checkpoint_resumes_bit_exact(name):
    print(f"reference checkpoint of {name}", flush=True)
    ref, cfgd, kind = load(name)
    cfg = P.NRConfig(**cfgd, seed=0)
    E, R, T = int(ref["E"]), int(ref["R"]), int(ref["steps"])
    sd, k0 = reference_checkpoint(name)
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=123)       # another seed: the checkpoint's key wins
    eng.load_state_dict(sd, strict=True)
    assert eng.T == k0
    to = lambda a: torch.from_numpy(np.asarray(a)).to(DEV)  # noqa: E731
    bad = []
    for s in range(k0, T):
        ids = np.nonzero(ref["reset_mask"][s])[0]
        if len(ids):
            eng.reset(ids.tolist())
        acc = [eng.submit(None, to(send)) for send in replay.submits(ref["counts"][s])]
        for nb, cls in replay.dl_frames(ref, s):
            eng.add_dl_frames(None, to(nb), to(cls))
        if acc and not np.array_equal(np.stack([a.cpu().numpy() for a in acc]), ref[f"s{s:03d}/accepted"]):
            bad.append((s, "accepted"))
        o = eng.step(None, to(ref["x"][s]))
        set_radio_bound(ref, s, cfg, eng, kind)
        bi, bf, _ = compare(ref, s, o, eng.owner_state(), E, R)
        if bi or bf:
            bad.append((s, bi, bf))
    gpu_util.MAX_DEV.clear()
    assert not bad, bad[:5]
    want = json.loads(bytes(ref["counters_json"]))
    got = eng.counters()
    for lk in (("ul", "dl") if cfg.dl else ("ul",)):
        lena = tuple(k for k in ("tb_bytes", "tb_empty", "retx_block") if k in want[lk])   # (5G-LENA switches on)
        for k in ("tb_new", "tb_ok", "tb_fail", "bytes_ok", "prb_used", "prb_avail") + lena:
            assert got[lk][k] == pytest.approx(want[lk][k], rel=1e-6), (lk, k)
        assert got[lk]["rv_tx"] == pytest.approx(want[lk]["rv_tx"])


def test_checkpoint_file_round_trip(tmp_path):
    """save after 6 steps, load into an engine built with another seed, continue 6 steps: every output, the
    owner-key state and the counters equal the uninterrupted run's."""
    ref, cfgd, kind = load("dl_c2")
    cfg = P.NRConfig(**cfgd, seed=0)
    E, R = int(ref["E"]), int(ref["R"])
    a = P.make_engine("L2", E, R, DEV, cfg, seed=0)
    to = lambda v: torch.from_numpy(np.asarray(v)).to(DEV)  # noqa: E731

    def run(eng, s):
        for send in replay.submits(ref["counts"][s]):
            eng.submit(None, to(send))
        for nb, cls in replay.dl_frames(ref, s):
            eng.add_dl_frames(None, to(nb), to(cls))
        return eng.step(None, to(ref["x"][s]))
    for s in range(6):
        run(a, s)
    path = checkpoint.save(a, tmp_path / "ck.pt", extra={"iter": 6})
    b = P.make_engine("L2", E, R, DEV, cfg, seed=99)
    assert checkpoint.load(b, path) == {"iter": 6}
    for s in range(6, 12):
        oa, ob = run(a, s), run(b, s)
        for k in oa:
            assert torch.equal(oa[k].nan_to_num(), ob[k].nan_to_num()), (s, k)
        sa, sb = a.owner_state(), b.owner_state()
        for k in sa:
            assert torch.equal(sa[k].nan_to_num(), sb[k].nan_to_num()), (s, k)
    assert a.counters() == b.counters()
    with pytest.raises(ValueError):
        checkpoint.load(P.make_engine("L2", E + 1, R, DEV, cfg, seed=0), path)

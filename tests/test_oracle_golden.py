"""The oracle against the golden trajectories written from the reference CPU engine (tests/golden/make_fixtures.py):
every step output and every state tensor after every step, bitwise (empty frame slots excepted: their fields are
unspecified in the reference)."""
import os

import numpy as np
import pytest
import torch

from conftest import CASES, DL_CASES, GOLDEN, MC_CASES
from oracle import nr_oracle as O
from oracle import replay
import isaac_net_amd as P


@pytest.mark.parametrize("name", CASES + DL_CASES + MC_CASES)
def test_oracle_bitwise_vs_reference(name):
    torch.set_num_threads(1)
    d, cfgd, kind = replay.load_case(os.path.join(GOLDEN, f"traj_{name}.npz"))
    cfg = P.NRConfig(**cfgd, seed=0)
    eng = O.OracleEngine(int(d["E"]), int(d["R"]), cfg, seed=0)
    bad = []

    def on_step(s, o, acc):
        if int(d[f"s{s:03d}/n_submit"]):
            if not np.array_equal(d[f"s{s:03d}/accepted"], np.stack([a.numpy() for a in acc])):
                bad.append((s, "accepted"))
        for k, v in o.items():
            if not np.array_equal(d[f"s{s:03d}/out.{k}"], v.numpy(), equal_nan=True):
                bad.append((s, "out." + k))
        valid = {lk: d[f"s{s:03d}/{lk}.q.cap"] >= 0 for lk in ("ul", "dl") if f"s{s:03d}/{lk}.q.cap" in d.files}
        for k, v in eng.state().items():
            ref, mine = d[f"s{s:03d}/{k}"], v.numpy()
            if k[3:5] == "q." and k[5:] != "enq":
                ref, mine = np.where(valid[k[:2]], ref, 0), np.where(valid[k[:2]], mine, 0)
            if not np.array_equal(ref, mine, equal_nan=True):
                bad.append((s, k))

    replay.run(eng, d, kind, on_step=on_step)
    assert not bad, bad[:10]
    # the counters of both links, the 5G-LENA grant accounting included (the reference sums them in float32)
    import json
    want_all = json.loads(bytes(d["counters_json"]))
    for lk in eng.links():
        for k, v in lk.ctr.items():
            if k != "prb_avail":
                assert float(v) == pytest.approx(want_all[lk.dir][k], rel=1e-6), (lk.dir, k)


@pytest.mark.parametrize("name,field,wrong", [("tdma", "ul_retx_sched", "ofdma"),
                                              ("amc_prev", "ul_amc_alloc", "current"),
                                              ("mc2_lena", "ul_retx_sched", "ofdma")])
def test_lena_switch_trajectories_pin_the_switch(name, field, wrong):
    """The TDMA retransmission and previous-PUSCH AMC trajectories depend on their switch: the oracle run with the
    switch at its default diverges from them (so the bitwise comparison above pins the switch's code)."""
    import dataclasses
    d, cfgd, kind = replay.load_case(os.path.join(GOLDEN, f"traj_{name}.npz"))
    cfg = dataclasses.replace(P.NRConfig(**cfgd, seed=0), **{field: wrong})
    eng = O.OracleEngine(int(d["E"]), int(d["R"]), cfg, seed=0)
    diff = []

    def on_step(s, o, acc):
        for k in ("ul.h_mcs", "ul.sent", "ul.h_state"):
            if not np.array_equal(d[f"s{s:03d}/{k}"], eng.state()[k].numpy()):
                diff.append((s, k))

    replay.run(eng, d, kind, steps=12, on_step=on_step)
    assert diff


def test_oracle_catches_a_planted_error():
    """A plausible mistake in the oracle (OLLA down-step of the BLER target 0.2 instead of 0.1) must fail the
    golden comparison, so the comparison above pins the OLLA update."""
    d, cfgd, kind = replay.load_case(os.path.join(GOLDEN, "traj_c2.npz"))
    cfg = P.NRConfig(**cfgd, seed=0)
    eng = O.OracleEngine(int(d["E"]), int(d["R"]), cfg, seed=0)
    eng.olla_dn = cfg.olla_up_db * 0.8 / 0.2
    diff = []

    def on_step(s, o, acc):
        if not np.array_equal(d[f"s{s:03d}/ul.olla"], eng.state()["ul.olla"].numpy()):
            diff.append(s)

    replay.run(eng, d, kind, steps=12, on_step=on_step)
    assert diff


@pytest.mark.parametrize("plant", ["ttt_off_by_one", "ewma_ignored"])
def test_oracle_catches_planted_multicell_errors(plant):
    """Plausible mistakes in the multi-cell restatement fail the golden comparison of the handover case: an A3
    time-to-trigger one slot long (fire at ttt - cnt instead of ttt - cnt - 1), and an N+I estimate that ignores the
    EWMA (li_alpha 0.5 read as 1)."""
    import dataclasses
    d, cfgd, kind = replay.load_case(os.path.join(GOLDEN, "traj_mc3_ho.npz"))
    cfg = P.NRConfig(**cfgd, seed=0)
    eng = O.OracleEngine(int(d["E"]), int(d["R"]), cfg, seed=0)
    if plant == "ttt_off_by_one":
        eng.assoc.ttt += 1
    else:
        eng.cfg = dataclasses.replace(cfg, li_alpha=1.0)
    diff = []

    def on_step(s, o, acc):
        st = eng.state()
        for k in ("assoc.serv", "assoc.ho_end", "net.ni_ul", "ul.sent"):
            if not np.array_equal(d[f"s{s:03d}/{k}"], st[k].numpy()):
                diff.append((s, k))

    replay.run(eng, d, kind, on_step=on_step)
    assert diff

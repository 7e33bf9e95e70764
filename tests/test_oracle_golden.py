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
                                              ("mc2_lena", "ul_retx_sched", "ofdma"),
                                              ("fcorr", "fading_delay_spread_ns", 3000.0),
                                              ("fcorr_mc2", "fading_delay_spread_ns", 300.0),
                                              ("rice_sto_slow", "rician_k_ramp_slots", 4),
                                              ("dop", "fading_doppler", "global"),
                                              ("dop", "doppler_min_speed_mps", 0.0),
                                              ("mc2_dop", "carrier_ghz", 3.6),
                                              ("wb_pf", "pf_metric", "subband"),
                                              ("mc2_wb", "scheduler", "pf")])
def test_switch_trajectories_pin_the_switch(name, field, wrong):
    """The TDMA retransmission, previous-PUSCH AMC, frequency-correlated fading and K-ramp trajectories depend on
    their switch: the oracle run with the switch at another value diverges from them (so the bitwise comparison above pins
    the switch's code)."""
    import dataclasses
    d, cfgd, kind = replay.load_case(os.path.join(GOLDEN, f"traj_{name}.npz"))
    cfg = dataclasses.replace(P.NRConfig(**cfgd, seed=0), **{field: wrong})
    eng = O.OracleEngine(int(d["E"]), int(d["R"]), cfg, seed=0)
    diff = []

    def on_step(s, o, acc):
        for k in ("ul.h_mcs", "ul.sent", "ul.h_state", "net.h", "ul.csi"):
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


def test_subband_correlation_factor_matches_the_restatement():
    """The engine's square root of the subband correlation (channels.subband_fading_sqrt, uploaded to the kernels) is
    the oracle's (fcorr_sqrt) for every carrier of the fixtures and a range of delay spreads, and it is one: L L^T
    has the correlation 1 / sqrt(1 + (2 pi df tau)^2) (within float32 rounding), L is lower-triangular with unit rows."""
    import math
    from isaac_net_amd.channels import subband_fading_sqrt
    for n_prb, rbg, mu in ((52, None, 1), (106, None, 1), (273, 35, 1), (273, None, 1), (25, None, 0)):
        for tau in (10.0, 60.0, 300.0, 3000.0):
            kw = dict(n_prb=n_prb, mu=mu, fading_freq_corr=True, fading_delay_spread_ns=tau)
            if rbg:
                kw["rbg_size"] = rbg
            cfg = P.NRConfig(**kw)
            L = subband_fading_sqrt(cfg)
            assert torch.equal(L, O.fcorr_sqrt(cfg))
            S = cfg.n_subbands
            w = torch.tensor([float(x) for x in cfg.subband_prbs], dtype=torch.float64) * 12 * cfg.scs_khz * 1e3
            f = torch.cumsum(w, 0) - w / 2
            c = 1.0 / torch.sqrt(1.0 + (2 * math.pi * (f[:, None] - f[None, :]) * tau * 1e-9) ** 2)
            Ld = L.double()
            assert torch.allclose(Ld @ Ld.T, c, atol=1e-5) or tau < 60.0      # (jittered near-singular cases)
            assert torch.equal(torch.tril(L), L) and torch.allclose(Ld.norm(dim=-1), torch.ones(S, dtype=torch.float64), atol=1e-6)


@pytest.mark.parametrize("plant", ["flush_as_carry", "floor_epre_per_prb", "ds_index_of_cell0"])
def test_oracle_catches_planted_handover_and_link_errors(plant):
    """The reference trajectories of the handover RLC flush, the A3 admission floor and the per-link delay spreads
    with several cells pin those branches of the oracle: a plausible mistake in each fails its comparison.
    flush_as_carry: ho_rlc="flush" read as "carry" (no frame dropped at the switch, mac.py:557-581);
    floor_epre_per_prb: the floor converted with the EPRE over nprb PRBs instead of 12 nprb subcarriers
    (radio.py:337-340); ds_index_of_cell0: every robot-cell link's delay-spread index taken from the LOS state of the
    link to cell 0 instead of its own (nr_engine.py:377-381)."""
    import dataclasses
    import math
    name, keys = {"flush_as_carry": ("mc3_flush", ("ul.q.lost", "ul.q.cap", "ul.sent")),
                  "floor_epre_per_prb": ("mc3_a3floor", ("assoc.serv", "assoc.n_ho", "assoc.a3_cand")),
                  "ds_index_of_cell0": ("mc2_fcorr_los", ("net.h", "net.fc_idx"))}[plant]
    d, cfgd, kind = replay.load_case(os.path.join(GOLDEN, f"traj_{name}.npz"))
    cfg = P.NRConfig(**cfgd, seed=0)
    if plant == "flush_as_carry":
        cfg = dataclasses.replace(cfg, ho_rlc="carry")
    eng = O.OracleEngine(int(d["E"]), int(d["R"]), cfg, seed=0)
    if plant == "floor_epre_per_prb":
        eng.assoc.floor_rx = cfg.a3_min_target_rsrp_dbm - (cfg.gnb_tx_dbm - 10 * math.log10(cfg.nprb) - cfg.ue_tx_dbm)
    elif plant == "ds_index_of_cell0":
        def set_fc_los(los, e=eng):
            los0 = los[:, :, :1].expand_as(los) if los.dim() == 3 else los
            e.fc_idx = torch.where(los0, e.fc_idx_los, e.fc_idx_nlos)
        eng._set_fc_los = set_fc_los
    diff = []

    def on_step(s, o, acc):
        st = eng.state()
        for k in keys:
            ref, mine = d[f"s{s:03d}/{k}"], st[k].numpy()
            if k.startswith("ul.q.") and k != "ul.q.enq":
                v = d[f"s{s:03d}/ul.q.cap"] >= 0
                ref, mine = np.where(v, ref, 0), np.where(v, mine, 0)
            if not np.array_equal(ref, mine):
                diff.append((s, k))

    replay.run(eng, d, kind, on_step=on_step)
    assert diff

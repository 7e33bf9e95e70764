"""Host logic of the engine that needs no GPU: refusals, the per-step slot schedule rows, config validation."""
import math

import numpy as np
import pytest

import isaac_net_amd as P
from isaac_net_amd import engine as EN


def test_refusals_name_each_unimplemented_feature():
    assert EN.refusals(P.NRConfig(n_prb=52)) == []
    assert EN.refusals(P.NRConfig(n_prb=52, dl=True)) == []
    bad = P.NRConfig(n_prb=52, dl=True, duplex="fdd", scheduler="qos", n_cells=3, cell_layout="hex",
                     ul_grant_model="bsr")
    names = " ".join(f for f, _ in EN.refusals(bad))
    for word in ("several cells", "FDD downlink", "bsr", "qos"):
        assert word in names
    assert "ul=False" in " ".join(f for f, _ in EN.refusals(P.NRConfig(n_prb=52, ul=False, dl=True)))
    # three hex cells with thermal noise (interference), power control on by default, 106 PRB (14 RBGs): runs
    mc = dict(mu=1, n_prb=106, n_cells=3, cell_layout="hex", cell_isd_m=150.0, noise_model="thermal")
    assert EN.refusals(P.NRConfig(**mc)) == []
    assert EN.refusals(P.NRConfig(**mc, a3_offset_db=float("inf"), harq_fail="drop", ho_rlc="flush")) == []
    assert EN.refusals(P.NRConfig(**mc, rlf=True, rlf_rlc="flush")) == []
    for n_cells in (4, 5, 6, 7):                           # the hex centre site and the first ring, up to 7
        assert EN.refusals(P.NRConfig(**dict(mc, n_cells=n_cells))) == [], n_cells
    for extra, word in ((dict(dl=True), "downlink with several cells"), (dict(harq_combining="ir_lena"), "HARQ-IR"),
                        (dict(rlf=True, rach=True), "RACH"), (dict(frame_buffer=65), "frame_buffer > 64"),
                        (dict(ul_tpc=True), "TPC")):
        assert word in " ".join(f for f, _ in EN.refusals(P.NRConfig(**dict(mc, **extra)))), extra
    # one cell: the 38.214 RBG counts of the standard carriers run (106 PRB: 14 RBGs, 273: 18, 133: 17, 78: 10),
    # other counts are refused; two cells run
    for n_prb in (106, 273, 133, 78, 24, 162, 245):
        assert EN.refusals(P.NRConfig(mu=1, n_prb=n_prb)) == [], n_prb
    assert "subbands" in " ".join(f for f, _ in EN.refusals(P.NRConfig(mu=1, n_prb=100, rbg_size=4)))   # 25 RBGs
    assert EN.refusals(P.NRConfig(**dict(mc, n_cells=2))) == []
    assert EN.refusals(P.NRConfig(**mc, fading_rician=True, rician_k_db=3.0)) == []    # Rician on every link


def test_make_engine_refuses_before_building():
    with pytest.raises(EN.HipUnsupported):
        P.make_engine("L2", 2, 2, "cuda", P.NRConfig(n_prb=52, ul=False, dl=True))
    with pytest.raises(NotImplementedError):
        P.make_engine("L1", 2, 2, "cuda", P.NRConfig(n_prb=52))
    with pytest.raises(ValueError):
        EN.HipNREngine(2, 2, "cpu", P.NRConfig(n_prb=52))


def test_schedule_rows_of_the_rl_workload():
    """DDDSU at 25 ms: 20 scheduled slots (10 S with an SR opportunity, 10 U with data); with i.i.d. fading
    (rho 0) the S-slot fading draws are skipped (the next slot overwrites the state) and the U slots keep theirs."""
    cfg = P.NRConfig(mu=1, n_prb=52, control_step_ms=25.0, fading_rho_per_ms=0.0)
    eng = EN.HipNREngine.__new__(EN.HipNREngine)
    eng.config, eng.dev, eng._rows, eng._nsym_idx, eng.dl = cfg, "cpu", {}, {12: 0}, False
    rows, n, last_rel, n_ul = eng._rows_for(0, 1)
    r = rows.numpy()
    assert n == 20 and n_ul == 10 and last_rel == 49
    flags = r[:, 2]
    assert np.all((flags[0::2] & 1) == 1) and np.all((flags[1::2] & 2) == 2)
    assert np.all((flags & 4) == 4)                        # every scheduled slot evolves the fading
    assert np.all((flags[0::2] & 8) == 0) and np.all((flags[1::2] & 8) == 8)
    rho = r[:, 4].view(np.float32)
    assert np.all(rho == 0.0)
    assert r[1, 0] == 4 and r[0, 0] == 3
    assert r[1, 6] == EN.salt((1 << 16) | 4) - (1 << 32) if EN.salt((1 << 16) | 4) >= 1 << 31 else True


def test_schedule_rows_correlated_fading_keep_every_draw():
    cfg = P.NRConfig(mu=1, n_prb=52, control_step_ms=10.0)
    eng = EN.HipNREngine.__new__(EN.HipNREngine)
    eng.config, eng.dev, eng._rows, eng._nsym_idx, eng.dl = cfg, "cpu", {}, {12: 0}, False
    rows, n, _, _ = eng._rows_for(20, 4)
    r = rows.numpy()
    assert np.all((r[:n, 2] & 8) == 8)
    rho = r[:n, 4].view(np.float32)
    assert abs(float(rho[0]) - cfg.fading_rho_per_ms ** (4 * 0.5)) < 1e-6
    assert abs(float(rho[1]) - cfg.fading_rho_per_ms ** (1 * 0.5)) < 1e-6


def test_schedule_rows_with_the_downlink():
    """dl=True, DDDSU at 10 ms (20 slots): every slot is scheduled (D and S carry DL data, U UL data); the DL
    rows flag the CQI reports at the first UL-capable slot of each 10-slot window, the DL data slots with their
    symbol-count index, the HARQ-ACK slot (the first UL-capable slot >= g + k1, relative to the step) in bits 8..23,
    and the DL decode stream; the fading flags of both row lists agree where both need the gain."""
    cfg = P.NRConfig(mu=1, n_prb=52, control_step_ms=10.0, fading_rho_per_ms=0.0, dl=True)
    eng = EN.HipNREngine.__new__(EN.HipNREngine)
    dls_syms = sorted({cfg.slot_symbols(p)[0] for p in range(5)} - {0})
    nsyms = sorted(set(dls_syms) | {12})
    eng.config, eng.dev, eng._rows, eng.dl = cfg, "cpu", {}, True
    eng._nsym_idx = {ns: i for i, ns in enumerate(nsyms)}
    rows, n, last_rel, n_ul, dl_rows = eng._rows_for(0, 1)
    sched = cfg.schedule(0)
    assert n == len(sched) == 20 and n_ul == 4
    d = dl_rows.numpy()[:n]
    fl = d[:, 2]
    for k, (rel, dls, uls, sr, cqi, ack) in enumerate(sched):
        assert d[k, 0] == rel
        assert bool(fl[k] & 1) == cqi and bool(fl[k] & 2) == (dls > 0)
        assert ((fl[k] >> 8) & 0xFFFF) == ack == cfg.next_ul_capable(rel + cfg.k1)
        assert d[k, 1] == (eng._nsym_idx[dls] if dls else -1)
        salt = EN.salt((EN.BLER_DL << 16) | rel)
        assert d[k, 7] == (salt - (1 << 32) if salt >= 1 << 31 else salt)
        # i.i.d. fading: the DL needs the gain at its data and CQI rows only
        assert bool(fl[k] & 8) == (dls > 0 or cqi)
    assert sorted(r[0] for r in sched if r[4]) == [3, 13]


def test_hash_helpers_agree():
    for v in (0, 5, (2 << 16) | 7, 0xFFFFFFFF):
        assert EN.salt(v) == (EN.mix32(v) + 0x9E3779B9) & 0xFFFFFFFF
    assert EN.seed_key(0) == EN.mix32(EN.mix32(0) ^ EN.salt(0))


def test_split_offsets_rebases_at_the_floor():
    """Byte offsets as base + int32 values (the step kernel's rebase): the base is the floor once it reaches the
    threshold, offsets at or above the floor stay non-negative, and offsets that do not fit are refused."""
    import torch
    from isaac_net_amd.engine import split_offsets
    big = 3 * (1 << 31) + 12345
    floor = torch.tensor([[0, 1000, big, (1 << 30) - 1]])
    sent = floor + torch.tensor([[5, 0, 70000, 3]])
    enq = sent + torch.tensor([[9, 0, 1 << 20, 0]])
    base, rel = split_offsets(floor, sent, enq, 1 << 30)
    assert base.tolist() == [[0, 0, big, 0]]
    assert rel(floor).tolist() == [[0, 1000, 0, (1 << 30) - 1]] and rel(enq)[0, 2] == 70000 + (1 << 20)
    assert torch.equal(base + rel(enq), enq)
    with pytest.raises(ValueError):
        split_offsets(torch.tensor([[0]]), torch.tensor([[0]]), torch.tensor([[1 << 31]]), 1 << 30)


def test_per_link_delay_spread_and_k_from_los_refusals():
    """Per-link delay spreads (fading_delay_spread_ns=None) run at one cell on UMi, UMa and InH, with the fixed and
    the stochastic LOS state and with Rician K from LOS, and with several cells; InF is refused."""
    one = dict(mu=1, n_prb=52, fading_freq_corr=True, channel="tr38901", gnb_height_m=10.0)
    for scn, los in (("UMi", "stochastic"), ("UMa", "los"), ("InH", "nlos")):
        cfg = P.NRConfig(**one, tr38901_scenario=scn, tr38901_los=los, fading_rician=True)
        assert cfg.freq_corr_mode == "los" and cfg.rician_mode == "los"
        assert EN.refusals(cfg) == [], scn
    mc = P.NRConfig(**dict(one, n_prb=106), n_cells=3, cell_layout="hex", cell_isd_m=150.0, tr38901_scenario="UMi")
    assert EN.refusals(mc) == []
    inf = P.NRConfig(**one, tr38901_scenario="InF-SL", tr38901_los="los")
    assert "per-link delay spreads" in " ".join(f for f, _ in EN.refusals(inf))
    assert EN.refusals(P.NRConfig(**dict(one, n_prb=106), n_cells=3, cell_layout="hex", cell_isd_m=150.0,
                                  tr38901_scenario="UMi", fading_delay_spread_ns=300.0)) == []


def test_wifi_several_aps_refusals():
    """Several APs run on one channel or several (one collision domain per channel); more than 8 APs are refused, and
    level WIFI_DCF keeps one AP. (Several channels with R + A > 64 or (R + A) x channels >= 400 are refused when the
    engine is made, where R is known: the GPU tests cover the accepted sizes.)"""
    from isaac_net_amd.wifi_config import WifiConfig
    from isaac_net_amd.wifi_engine import wifi_refusals
    aps = ((0.0, 0.0), (100.0, 0.0), (50.0, 80.0))
    assert wifi_refusals(P.NRConfig(wifi=WifiConfig(ap_positions_m=aps, roam_ms=2.0))) == []
    assert wifi_refusals(P.NRConfig(wifi=WifiConfig(ap_positions_m=aps, n_channels=3))) == []
    many = tuple((10.0 * i, 0.0) for i in range(9))
    assert "9 access points" in " ".join(f for f, _ in wifi_refusals(P.NRConfig(wifi=WifiConfig(ap_positions_m=many))))


def test_wifi_stochastic_los_refusals():
    """Level WIFI runs the stochastic LOS state (the reference's default) on UMi, UMa up to 13 m and InH; InF and UMa
    above 13 m are refused, as at the NR levels."""
    from isaac_net_amd.wifi_config import WifiConfig
    from isaac_net_amd.wifi_engine import wifi_refusals
    one = dict(channel="tr38901", tr38901_los="stochastic", cell_positions_m=((0.0, 0.0),), wifi=WifiConfig())
    for scn in ("UMi", "UMa", "InH"):
        assert wifi_refusals(P.NRConfig(**one, tr38901_scenario=scn)) == [], scn
    for cfg in (P.NRConfig(**one, tr38901_scenario="InF-SL"), P.NRConfig(**one, tr38901_scenario="UMa",
                                                                           ue_height_m=20.0)):
        assert "stochastic LOS" in " ".join(f for f, _ in wifi_refusals(cfg))


@pytest.mark.parametrize("name", ["fcorr_los", "fcorr_los_dl", "fcorr_los_rice", "mc2_fcorr_los"])
def test_delay_spread_grid_matches_the_reference_table(name):
    """The square roots on the delay-spread grid (channels.delay_spread_grid) equal the reference engine's own
    net.fc_grid_ns / net.fc_tab of the golden trajectory bit for bit (13, 14 and 18 RBGs, two grids)."""
    import os
    import torch
    from conftest import GOLDEN
    from isaac_net_amd.channels import delay_spread_grid
    from oracle import replay
    ref, cfgd, _ = replay.load_case(os.path.join(GOLDEN, f"traj_{name}.npz"))
    grid, tab = delay_spread_grid(P.NRConfig(**cfgd, seed=0))
    assert torch.equal(grid, torch.from_numpy(ref["s000/net.fc_grid_ns"]))
    assert torch.equal(tab, torch.from_numpy(ref["s000/net.fc_tab"]))
    assert torch.equal(tab, tab.tril())

"""Known answers that pin the host tables and the counter hash independently of the golden trajectories:
38.214 TBS / 38.212 segmentation spec examples and numerology (reference tests/test_nr_phy.py:21-69), the hard-coded
hash values of tests/test_rng_levels.py:295-311, the scalar key scheme of tests/test_nr_fast.py:96-124, TR 38.901
hand-computed path losses (tests/test_channels.py:121-147), and the processed PHY tables of the reference."""
import hashlib
import math
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import nr_oracle as O
import isaac_net_amd as P
from isaac_net_amd import phy as PH
from isaac_net_amd import channels as CH
from isaac_net_amd import engine as EN


def test_tbs_spec_examples():
    assert int(PH.tbs_38214(2., 120 / 1024, 1., 12, 12)) == 24
    assert int(PH.tbs_38214(6., 948 / 1024, 50., 12, 12)) == 36896
    assert int(PH.tbs_38214(4., 340 / 1024, 10., 12, 12)) == 1800
    assert int(PH.tbs_38214(2., 193 / 1024, 273., 13, 12)) == 14856
    assert int(PH.tbs_38214(2., 120 / 1024, 1., 14, 0)) == int(PH.tbs_38214(2., 120 / 1024, 1., 13, 0))
    cb, c = PH.segment(36896, 948 / 1024)
    assert int(cb) == 7408 and int(c) == 5


def test_numerology():
    c1 = P.NRConfig(mu=1, bandwidth_mhz=20)
    c0 = P.NRConfig(mu=0, bandwidth_mhz=20, tdd_pattern="DDDSU")
    c2 = P.NRConfig(mu=2, bandwidth_mhz=100, tdd_pattern="DDSU")
    c3 = P.NRConfig(mu=1, bandwidth_mhz=100, tdd_pattern="DSUUU")
    assert (c1.nprb, c1.rbg, c1.n_subbands, c1.subband_prbs[-1]) == (51, 4, 13, 3)
    assert (c0.nprb, c0.rbg) == (106, 8) and (c2.nprb, c2.rbg, c2.n_subbands) == (135, 8, 17)
    assert (c3.nprb, c3.rbg, c3.n_subbands) == (273, 16, 18)
    assert (c3.ul_slots_per_step, c2.slots_per_step, c2.ul_slots_per_step) == (120, 400, 100)
    cs = P.NRConfig(tdd_pattern="DDDSU", special_ul_data=True, special_split=(6, 4, 4))
    assert cs.slot_symbols(3) == (5, 4) and cs.slot_symbols(0) == (13, 0) and cs.slot_symbols(4) == (0, 12)
    # the RL-scale workload: 52 PRB -> 13 RBGs of 4, DDDSU at 25 ms -> 10 UL data slots and 10 SR opportunities
    c = P.NRConfig(mu=1, n_prb=52, control_step_ms=25.0)
    sched = c.schedule(0)
    assert c.n_subbands == 13 and sum(1 for s in sched if s[2]) == 10 and sum(1 for s in sched if s[3]) == 10


def test_phy_tables_equal_reference_processing():
    d = np.load(os.path.join(GOLDEN, "phy_tables.npz"))
    for mt in (1, 2):
        t = PH.PhyTables(mt, max_tx=16)
        assert hashlib.sha256(np.ascontiguousarray(t.bler[None]).tobytes()).digest() == bytes(d[f"t{mt}/bler_sha256"])
        idx = d[f"t{mt}/sample_idx"]
        assert np.array_equal(t.bler[idx[:, 0], idx[:, 1], idx[:, 2]], d[f"t{mt}/sample_val"])
        for k in ("snr_grid", "cbs_axis", "beta", "thr_ref", "se", "mcs_eq"):
            assert np.array_equal(getattr(t, k), d[f"t{mt}/{k}"]), k
        assert np.array_equal(t.thr, d[f"t{mt}/thr"][0])
        for ns in (2, 4, 12, 13):
            tb = t.tbs_all(np.arange(274.0), ns)
            assert np.array_equal(tb, d[f"t{mt}/tbs_ns{ns}"])
            cbs, c = PH.segment(tb, t.r.astype(np.float64))
            assert np.array_equal(cbs, d[f"t{mt}/cbs_ns{ns}"]) and np.array_equal(c, d[f"t{mt}/ncb_ns{ns}"])
    tb = PH.tbs_38214(np.array([2.0, 4.0, 6.0, 8.0]), np.array([0.2, 0.5, 0.7, 0.93]),
                      np.arange(0, 274.0)[:, None], 12, 12, 6, 2)
    assert np.array_equal(tb, d["tbs_oh6_l2"])


def test_bler_table_invariants():
    """Post-processing invariants that hold whatever the Sionna data: BLER in [0, 1], non-increasing in SNR, 1 at
    the padded low end, and every MCS reaches the target inside the grid."""
    t = PH.PhyTables(1)
    assert t.bler.min() >= 0 and t.bler.max() <= 1
    assert np.all(np.diff(t.bler, axis=-1) <= 0)
    assert np.all(t.bler[..., 0] == 1.0)
    assert np.all((t.bler <= 0.1).any(-1))
    # MCS 16 -> 17 (the 16QAM -> 64QAM switch) is not monotone in table 1, so the kernel must use the linear scan
    assert not np.all(np.diff(t.thr_ref) >= 0)


HASH_XS = (0, 1, 2, 12345, 0xDEADBEEF, 0xFFFFFFFF)
HASH_WANT = [0, 2261973619, 229111015, 2258480790, 707447538, 2578835075]


def test_hash_known_values():
    assert [O.mix32(x) for x in HASH_XS] == HASH_WANT
    assert [EN.mix32(x) for x in HASH_XS] == HASH_WANT
    r = O.CounterRNG(12345, 3)
    r.reset_mask(None)
    r.ctr[O.STEP].add_(1)
    u = r._draw(r.ctr[O.STEP], O.STEP, 1, 4, False)
    assert (u.double() * 2 ** 24).to(torch.int64).tolist() == [[10567228, 16700380, 16191287, 1599467],
                                                               [268848, 15326424, 8181290, 3147942],
                                                               [13082027, 15096436, 9686026, 361841]]


def test_key_scheme_scalar_rederivation():
    seed, E = 2 ** 40 + 77, 3
    r = O.CounterRNG(seed, E)
    r.reset_mask(None)
    r.ctr[O.STEP].add_(2)
    u = r.step_uniform(O.BLER_UL, 5, 7)
    s0 = O.mix32(O.mix32(seed & 0xFFFFFFFF) ^ O.salt(seed >> 32))
    assert s0 == EN.seed_key(seed)
    for e in range(E):
        h = O.mix32(s0 ^ O.salt(e))
        h = O.mix32(h ^ O.salt(0))
        h = O.mix32(h ^ O.salt(O.STEP))
        h = O.mix32(h ^ O.salt(2))
        base = O.mix32(h ^ O.salt((O.BLER_UL << 16) | 5))
        for i in range(7):
            x = O.mix32(O.mix32((base + i * 0x9E3779B9) & 0xFFFFFFFF) ^ base)
            assert float(u[e, i]) == (x >> 8) / 16777216.0


def test_rng_vectors_and_box_muller_closed_form():
    d = np.load(os.path.join(GOLDEN, "rng_vectors.npz"))
    r = O.CounterRNG(int(d["seed"]), 6)
    assert r.s0 == int(d["s0"])
    r.episode = torch.as_tensor(d["episode"]).clone()
    r.ctr[O.STEP] = torch.as_tensor(d["ctr_step"]).clone()
    assert np.array_equal(r.step_uniform(2, 5, 37).numpy(), d["u_step_s5"])
    assert np.array_equal(r.reset_uniform(6 << 16, 9).numpy(), d["u_reset_s0"])
    n = r.step_normal(1, 3, 52).numpy()
    assert np.array_equal(n, d["n_step_s3"])
    # Box-Muller closed form on the same hash elements, in float64: agrees to float32 rounding
    base = O.base_key(r.s0, r.env, r.episode, O.STEP, r.ctr[O.STEP], (1 << 16) | 3)[:, None]
    idx = torch.arange(104).view(52, 2)
    h1, h2 = O.elem_hash(base, idx[:, 0]), O.elem_hash(base, idx[:, 1])
    u1 = ((h1 >> 8) + 1).double() / 2 ** 24
    u2 = (h2 >> 8).double() / 2 ** 24
    z = torch.sqrt(-2 * torch.log(u1)) * torch.cos(2 * math.pi * u2)
    assert torch.allclose(torch.from_numpy(n).double(), z, atol=2e-6, rtol=1e-6)


PL_CASES = [("UMi", True, 50.0, 10.0, 79.08964923389806), ("UMi", True, 300.0, 10.0, 98.24426066376931),
            ("UMi", False, 100.0, 10.0, 104.64383201166098), ("UMa", True, 100.0, 25.0, 83.13815667685238),
            ("UMa", True, 1000.0, 25.0, 109.41189477469499), ("UMa", False, 200.0, 25.0, 114.46197311942146),
            ("InH", True, 10.0, 3.0, 60.66494857628214), ("InH", False, 20.0, 3.0, 80.7233937148878),
            ("InF-SL", True, 30.0, 1.5, 73.93539981912798), ("InF-SH", True, 30.0, 8.0, 74.1495789134629)]


@pytest.mark.parametrize("scn,los,d2,hbs,want", PL_CASES)
def test_tr38901_hand_values_through_oracle_radio(scn, los, d2, hbs, want):
    """Oracle radio with the shadowing field zeroed equals the hand-computed TR 38.901 path loss."""
    cfg = P.NRConfig(channel="tr38901", tr38901_scenario=scn, tr38901_los="los" if los else "nlos",
                     cell_positions_m=((0.0, 0.0),))
    rng = O.CounterRNG(0, 1)
    rng.reset_mask(None)
    rad = O.Radio(cfg, 1, rng)
    rad.fields = [(torch.zeros_like(k), torch.full_like(p, math.pi / 2)) for k, p in rad.fields]   # cos(pi/2) ~ 0
    pg = rad.pathgain(torch.tensor([[[d2, 0.0]]]))
    assert abs(-float(pg) - want) < 2e-3
    assert CH.SCENARIOS[scn].h_bs == hbs


def test_breakpoint_distance():
    assert abs(CH.breakpoint_m("UMi", 3.5, 10.0, 1.5) - 210.0) < 1e-9
    with pytest.raises(ValueError):
        CH.breakpoint_m("UMi", 3.5, 10.0, 0.5)


def test_cqi_tables_closed_form():
    """38.214 CQI report (cqi_table="38214"): CQI -> MCS is the highest MCS of no larger spectral efficiency (CQI 1's
    QPSK 78/1024 lies below MCS 0, CQI 7 = 16QAM 378 is MCS 11 of table 1, CQI 15 = 64QAM 948 is MCS 28, or the
    cap); a CQI with an MCS of equal efficiency reports from that MCS's threshold, CQI 1 from MCS 0's shifted by the
    Shannon-gap difference; the thresholds never decrease."""
    import math
    t = PH.PhyTables(1, max_tx=4)
    thr, cm = PH.cqi_tables(t, 1)
    assert cm.shape == (16,) and thr.shape == (15,)
    assert cm[0] == 0 and cm[1] == 0 and cm[7] == 11 and cm[15] == 28
    gap = lambda e: 10 * math.log10(2 ** e - 1)  # noqa: E731
    assert abs(float(thr[0]) - (float(t.thr_ref[0]) + gap(2 * 78 / 1024) - gap(float(t.se[0])))) < 1e-5
    assert float(thr[6]) == float(t.thr_ref[11])
    assert (np.diff(thr) >= 0).all()
    capped = PH.PhyTables(1, max_tx=4, mcs_cap=20)
    assert PH.cqi_tables(capped, 1)[1][15] == 20
    t2 = PH.PhyTables(2, max_tx=4)
    thr2, cm2 = PH.cqi_tables(t2, 2)
    assert cm2[15] == 27 and cm2[12] == 21      # 256QAM 948 is MCS 27 of table 2; 256QAM 711 is MCS 21


def outer_sum_rule(x):
    """The step kernel's order for torch's CPU sum over the robots (dim 1) of an [E,R,C,S] float32 tensor
    (aten_outer_sum in inet_nr_dev.h): columns q = c S + s below 32 floor(C S / 32) add the rows in chunks of 16
    (each chunk from 0, the chunk sums accumulated from 0, then added to the sum of the rows past the last chunk);
    the other columns use four interleaved accumulators combined as ((a0 + a1) + a2) + a3."""
    f = np.float32
    E, R, C, S = x.shape
    n = C * S
    out = np.zeros((E, C, S), np.float32)
    for e in range(E):
        for q in range(n):
            c, s = divmod(q, S)
            v = x[e, :, c, s]
            if q < 32 * (n // 32):
                acc, i = f(0), 0
                while i + 16 <= R:
                    ch = f(0)
                    for k in range(16):
                        ch = f(ch + v[i + k])
                    acc, i = f(acc + ch), i + 16
                tail = f(0)
                for k in range(i, R):
                    tail = f(tail + v[k])
                out[e, c, s] = f(tail + acc)
            else:
                a = [f(0)] * 4
                for i in range(4 * (R // 4)):
                    a[i % 4] = f(a[i % 4] + v[i])
                for i in range(4 * (R // 4), R):
                    a[0] = f(a[0] + v[i])
                out[e, c, s] = f(f(f(a[0] + a[1]) + a[2]) + a[3])
    return out


@pytest.mark.skipif(torch.backends.cpu.get_cpu_capability() != "AVX512",
                    reason="the pinned order is that of torch's AVX512 CPU kernels")
@pytest.mark.parametrize("R,C,S", [(8, 3, 14), (16, 3, 13), (33, 3, 14), (64, 3, 14), (64, 3, 8), (40, 7, 14)])
def test_interference_sum_order_is_torchs(R, C, S):
    """The interference sum of the multi-cell step (_ul_ici: (p_rx * other).sum(1), nr_engine.py:799-816) in the
    order the kernel replays equals torch's bit for bit, on terms spread over ten decades with exact zeros (robots
    of the same cell, RBGs not held); a sequential sum differs (so the test pins the grouping)."""
    g = torch.Generator().manual_seed(R * 100 + C * 10 + S)
    x = (torch.rand(3, R, C, S, generator=g) * (torch.rand(3, R, C, S, generator=g) < 0.5) *
         10 ** (torch.rand(3, R, C, S, generator=g) * 10 - 12)).float()
    want = x.sum(1).numpy()
    assert np.array_equal(outer_sum_rule(x.numpy()), want)
    if R > 16:
        seq = np.zeros_like(want)
        for r in range(R):
            seq = (seq + x.numpy()[:, r]).astype(np.float32)
        assert not np.array_equal(seq, want)


def _search_suffix_min(thr, mcs_max, e):
    """The step kernel's MCS search: three binary levels, then a count inside the last block of four, over the
    suffix minima of thr[0..mcs_max] (NaN past mcs_max, 32 entries)."""
    t = np.full(32, np.nan, np.float32)
    for m in range(mcs_max + 1):
        t[m] = np.min(thr[m:mcs_max + 1])
    m = 16 if e >= t[16] else 0
    m += 8 if e >= (t[24] if m else t[8]) else 0
    m += 4 if e >= (t[m + 4]) else 0
    return m + int(e >= t[m + 1]) + int(e >= t[m + 2]) + int(e >= t[m + 3])


def test_mcs_search_over_suffix_minima_is_the_linear_scan():
    """phy.mcs_at (the highest m <= mcs_max with x >= thr_ref[m], else 0) equals the kernel's binary search over the
    suffix minima for any table: non-monotone, with ties, and at NaN or infinite inputs."""
    rs = np.random.default_rng(5)
    for trial in range(300):
        mcs_max = int(rs.integers(1, 32))
        thr = np.sort(rs.uniform(-10, 25, mcs_max + 1)).astype(np.float32)
        if trial % 3:
            thr = thr + rs.normal(0, 2.0, thr.shape).astype(np.float32)        # non-monotone
        if trial % 5 == 0:
            thr[rs.integers(0, mcs_max + 1)] = thr[rs.integers(0, mcs_max + 1)]  # ties
        xs = np.concatenate([rs.uniform(-15, 30, 40), thr, thr + np.float32(1e-6), [np.nan, -np.inf, np.inf]])
        for e in xs.astype(np.float32):
            lin = max([m for m in range(mcs_max + 1) if e >= thr[m]], default=0)
            assert _search_suffix_min(thr, mcs_max, e) == lin, (trial, e)

"""The level WIFI oracle (oracle/wifi_oracle.py) against the reference's golden trajectories (bitwise, every output
and state tensor after every step), and the parts of the mean-field model that closed forms and textbook tables fix
independently of the reference: Bianchi's saturation fixed point, the Poisson inverse CDF, the 802.11 rate table."""
import math
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import replay
from oracle.wifi_oracle import WifiOracle
import isaac_net_amd as P
from isaac_net_amd.wifi_config import WifiConfig, derive, mcs_table

WIFI_CASES = ["w_snr", "w_mean", "w_logd", "w_tr", "w_sto", "w_multi", "w_chan", "w_chan3", "w_aifs", "w_aifs_cls",
              "w_hidden", "w_hidden_rts", "w_dcf"]


def load(name):
    return replay.load_wifi_case(os.path.join(GOLDEN, f"traj_{name}.npz"), P.NRConfig, WifiConfig)


def run_oracle(name, plant=None, steps=None):
    torch.set_num_threads(1)
    d, cfg, kind = load(name)
    o = WifiOracle(int(d["E"]), int(d["R"]), cfg, seed=0)
    if plant is not None:
        plant(o)
    bad = []

    def cmp(pre, vals):
        for k, v in vals.items():
            if f"{pre}/{k}" in d.files and not np.array_equal(d[f"{pre}/{k}"], np.asarray(v), equal_nan=True):
                bad.append(f"{pre}/{k}")

    cmp("init", o.state())
    for s in range(int(d["steps"]) if steps is None else steps):
        ids = np.nonzero(d["reset_mask"][s])[0]
        if len(ids):
            o.reset(ids.tolist())
            cmp(f"reset{s:03d}", o.state())
        acc = [o.submit(None, torch.from_numpy(send)).numpy() for send in replay.submits(d["counts"][s])]
        if acc and not np.array_equal(np.stack(acc), d[f"s{s:03d}/accepted"]):
            bad.append(f"s{s:03d}/accepted")
        out = o.step(None, torch.from_numpy(d["x"][s]))
        cmp(f"s{s:03d}", {"out." + k: v for k, v in out.items()})
        cmp(f"s{s:03d}", o.state())
    return bad


@pytest.mark.parametrize("name", WIFI_CASES)
def test_wifi_oracle_bitwise_vs_reference(name):
    bad = run_oracle(name)
    assert not bad, bad[:10]


def test_wifi_oracle_catches_a_planted_error():
    """A plausible mistake (fixed-point damping 0.5 instead of the configured 0.6) must fail the comparison."""
    def plant(o):
        o.wc = o.wc.with_(fp_damping=0.5)
    assert run_oracle("w_snr", plant=plant, steps=3)


@pytest.mark.parametrize("plant_name", ["one_domain", "robots_stay_in_domain_0", "sorted_row_sum"])
def test_wifi_oracle_domains_are_pinned(plant_name):
    """Several channels: summing over every station of the env (one domain), leaving the robots in the first domain
    after association, or summing a domain in ATen's vectorized order instead of the batched product's index order
    must each fail the w_chan trajectory."""
    def plant(o):
        if plant_name == "one_domain":
            o.D = 1
        elif plant_name == "robots_stay_in_domain_0":
            o.ap_ch = torch.zeros_like(o.ap_ch)
        else:
            def dom_sum(x, o=o):
                per = (o.chan_oh.transpose(-1, -2) * x[:, None, :]).contiguous().sum(-1)       # [E, D]
                return (o.chan_oh * per[:, None, :]).sum(-1)
            o._dom_sum = dom_sum
    assert run_oracle("w_chan", plant=plant, steps=12)


@pytest.mark.parametrize("plant_name", ["one_zone", "min_over_all_stations", "no_last_zone_factor"])
def test_wifi_oracle_zones_are_pinned(plant_name):
    """AIFS zones: one zone for all, the smallest AIFSN taken over every station instead of the contending ones, or
    the last zone's stationary weight without its 1 / (1 - idle) geometric sum must each fail the w_aifs_cls
    trajectory (six zones)."""
    def plant(o):
        if plant_name == "one_zone":
            o.d.Z = 1
        elif plant_name == "min_over_all_stations":
            o._dom_min = lambda x, mask, o=o: WifiOracle._dom_min(o, x, torch.ones_like(mask))
        else:
            def zones(w, tau, dz, active, o=o):
                S, own, pi = WifiOracle._zones(o, w, tau, dz, active)
                raw = [torch.ones_like(tau)]
                for z in range(1, len(S)):
                    raw.append(raw[-1] * torch.exp(S[z - 1]))
                tot = sum(raw)
                return S, own, [r / tot for r in raw]
            o._zones = zones
    assert run_oracle("w_aifs_cls", plant=plant, steps=12)


@pytest.mark.parametrize("plant_name", ["no_hidden_term", "cca_off_by_1db", "tv_of_data_with_rts"])
def test_wifi_oracle_hidden_nodes_are_pinned(plant_name):
    """Hidden nodes: dropping the hidden-collision term, a CCA threshold 1 dB off, or the data time as the
    vulnerable period under RTS/CTS must each fail its trajectory."""
    def plant(o):
        if plant_name == "no_hidden_term":
            def sensing(*a, o=o):
                WifiOracle._sensing(o, *a)
                o.H = torch.zeros_like(o.H)
            o._sensing = sensing
        elif plant_name == "cca_off_by_1db":
            import dataclasses
            o.wc = dataclasses.replace(o.wc, cca_dbm=o.wc.cca_dbm - 1.0)
        else:
            def times(B, rate, aifsn, o=o):
                ts, tc, tv = WifiOracle._times(o, B, rate, aifsn)
                nsym = torch.ceil((22.0 + 8.0 * (B * o.d.ovh1)) / (rate * o.d.tsym))
                return ts, tc, o.d.pre + o.d.tsym * nsym
            o._times = times
    assert run_oracle("w_hidden_rts" if plant_name == "tv_of_data_with_rts" else "w_hidden", plant=plant, steps=10)


def test_wifi_constants_match_reference_tables():
    """The float32 tables the kernels read (rates, thresholds, EDCA, class ACs, Poisson support) equal the
    reference's WifiNet buffers of every golden case."""
    for name in WIFI_CASES:
        d, cfg, _ = load(name)
        c = derive(cfg, cfg.wifi)
        for k, v in (("rates", c.rates), ("thr", c.thr), ("mcs_ids", c.mcs_ids), ("ac_W0", c.ac_W0),
                     ("ac_Wmax", c.ac_Wmax), ("ac_aifsn", c.ac_aifsn), ("ac_txop", c.ac_txop), ("cls_ac", c.cls_ac)):
            assert np.array_equal(d[f"init/{k}"], v), (name, k)
        assert c.n_acc_max == int(d["n_acc_max"]) and c.K == int(d["K"])
        assert np.float32(c.tau0) == d["init/tau"][0, 0]


def test_rate_tables_textbook():
    """802.11 rates and SNR thresholds: HE 20 MHz 1 SS 0.8 us GI 8.6 .. 143.4 Mb/s; VHT 20 MHz 6.5 .. 78 Mb/s without
    MCS 9; non-HT 6 .. 54 Mb/s; thresholds = sensitivity + 91 dB (MCS 0: 9 dB, HE MCS 11: 39 dB)."""
    r, t = mcs_table("ax", 20, 1, 0.8)
    assert len(r) == 12 and r[0] == pytest.approx(8.6, abs=0.01) and r[-1] == pytest.approx(143.4, abs=0.05)
    assert t[0] == pytest.approx(9.0, abs=0.02) and t[-1] == pytest.approx(39.0, abs=0.02)
    r, _ = mcs_table("ac", 20, 1, 0.8)
    assert len(r) == 9 and r[0] == pytest.approx(6.5, abs=0.01) and r[-1] == pytest.approx(78.0, abs=0.01)
    r, t = mcs_table("a")
    assert r == [6.0, 9.0, 12.0, 18.0, 24.0, 36.0, 48.0, 54.0] and t[1] == pytest.approx(10.0, abs=0.02)


def _bianchi(n, W, m):
    """Bianchi (IEEE JSAC 18(3), 2000) eq. (7)/(9): tau(p) = 2 (1 - 2p) / ((1 - 2p)(W + 1) + p W (1 - (2p)^m)),
    p = 1 - (1 - tau)^(n - 1), solved by bisection on p."""
    lo, hi = 0.0, 0.999999
    for _ in range(200):
        p = 0.5 * (lo + hi)
        tau = 2 * (1 - 2 * p) / ((1 - 2 * p) * (W + 1) + p * W * (1 - (2 * p) ** m))
        if p - (1 - (1 - tau) ** (n - 1)) > 0:
            hi = p
        else:
            lo = p
    return tau, p


@pytest.mark.parametrize("n,W,m", [(5, 32, 3), (10, 32, 5), (20, 16, 6)])
def test_meanfield_matches_bianchi_saturation(n, W, m):
    """n saturated identical stations, no retry limit in effect (60 attempts): the oracle's damped fixed point
    converges to Bianchi's tau and p, and its success rate to tau (1 - tau)^(n-1) / E[slot]."""
    cfg = P.NRConfig(control_step_ms=1.0, wifi=WifiConfig(max_tx=60, fp_iters=400, fp_damping=0.5))
    o = WifiOracle(1, n, cfg)
    w = torch.ones(1, n + 1)
    w[0, n] = 0.0
    W0 = torch.full((1, n + 1), float(W))
    Wm = torch.full((1, n + 1), float(W * 2 ** m))
    Ts, Tc = torch.full((1, n + 1), 300.0), torch.full((1, n + 1), 250.0)
    tau, p, mu, _ = o._solve(w, Ts, Tc, torch.full((1, n + 1), 0.05), o._stage_factors(W0, Wm, 60))
    tb, pb = _bianchi(n, W, m)
    assert float(tau[0, 0]) == pytest.approx(tb, rel=2e-5)
    assert float(p[0, 0]) == pytest.approx(pb, rel=2e-5)
    ptr = 1 - (1 - tb) ** n
    ps = n * tb * (1 - tb) ** (n - 1)
    slot = (1 - ptr) * 9.0 + ps * 300.0 + (ptr - ps) * 250.0
    assert float(mu[0, 0]) == pytest.approx(tb * (1 - tb) ** (n - 1) / slot, rel=1e-4)


def test_poisson_draw_is_the_inverse_cdf():
    """poisson_icdf: the draw is the smallest k with CDF(k) >= u (scipy.stats.poisson.ppf), away from ties."""
    from scipy.stats import poisson
    cfg = P.NRConfig(control_step_ms=1.0, wifi=WifiConfig())
    o = WifiOracle(1, 1, cfg)
    rs = np.random.default_rng(5)
    lam = torch.from_numpy(rs.uniform(0.0, 8.0, 4000).astype(np.float32))
    u = torch.from_numpy((rs.integers(0, 2 ** 24, 4000) / 2 ** 24).astype(np.float32))
    got = o._poisson(lam, u).numpy()
    want = poisson.ppf(u.double().numpy(), lam.double().numpy())
    k = np.minimum(got, want).astype(int)
    far = np.abs(poisson.cdf(k, lam.double().numpy()) - u.double().numpy()) > 1e-5
    assert np.array_equal(got[far], want[far]) and far.mean() > 0.99

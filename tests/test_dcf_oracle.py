"""The DCF level's CPU oracle (oracle/dcf_oracle.py): exchange times from the 802.11 tables by hand, the contention
semantics on hand-set counters, and its saturation statistics against the reference's own CSMA/CA event simulator
(tests/golden/eventsim_sat.npz, written by tests/golden/make_fixtures.py from core/wifi/eventsim.py) and against
Bianchi's fixed point. The draws differ (counter RNG here, numpy PCG64 there), so the comparison is statistical."""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle.dcf_oracle import DcfOracle
import isaac_net_amd as P
from isaac_net_amd.wifi_config import WifiConfig


def sat_cfg(**wkw):
    return P.NRConfig(control_step_ms=20.0, frame_buffer=16, msg_sizes=(500000.0,), timeout_steps=100000,
                      wifi=WifiConfig(access_category="DCF", max_ampdu_bytes=0, **wkw))


def test_exchange_times_by_hand():
    """802.11ax 20 MHz MCS 11 (1950 data bits per 13.6 us symbol), 1472 B in one MSDU with 70 B overhead:
    22 + 8 (1472 + 70) = 12358 bits -> 7 symbols; PPDU = 44 us preamble + 95.2 us; success = PPDU + SIFS 16 us + ACK
    (14 B at 24 Mb/s: 20 + 2 x 4 us = 28 us) = 183.2 us; collision ("difs" model) = PPDU = 139.2 us. With RTS/CTS
    (28 us each): success 183.2 + 28 + 16 + 28 + 16 = 271.2 us, collision 28 + 16 + 28 = 72 us."""
    o = DcfOracle(1, 2, sat_cfg())
    assert o.k["ndbps"][-1] == 1950 and o.k["tsym"] == 13600 and o.k["pre"] == 44000
    assert o.busy(1472, 1950) == (183200, 139200)
    o2 = DcfOracle(1, 2, sat_cfg(rts_cts=True))
    assert o2.busy(1472, 1950) == (271200, 72000)
    # two MSDUs: 1500 B -> 22 + 8 (1500 + 140) = 13142 bits -> 7 symbols
    assert o.busy(1500, 1950)[1] == 44000 + 7 * 13600


def _one_event(b0, b1, fer=0.0):
    """Two stations with hand-set counters and one 1000 B message each: the first event of the step."""
    cfg = P.NRConfig(control_step_ms=1.0, frame_buffer=4, msg_sizes=(1000.0,),
                     wifi=WifiConfig(access_category="DCF", frame_error_rate=fer))
    o = DcfOracle(1, 2, cfg)
    o.submit(None, torch.ones(1, 2, dtype=torch.long))
    o.b[0] = [b0, b1]
    o.had[0] = True                      # no arrival rule: the counters are taken as set
    o.t_idle[0] = -1000000               # idle for 1 ms before the step
    out = o.step(None, torch.full((1, 2), 40.0))
    return o, out


def test_contention_semantics_on_set_counters():
    # distinct counters: the smaller one sends first and succeeds; both messages end within the 1 ms step
    o, out = _one_event(3, 5)
    d = out["delivered"][0].numpy()
    assert d[0, 0] and d[1, 0]
    assert out["delay"][0, 0, 0] < out["delay"][0, 1, 0]
    assert o.tot["fail"][0] == 0 and o.tot["att"][0] == 2
    # equal counters: a collision, then both back off in [0, 2 W0 - 1] at stage 1
    o, out = _one_event(4, 4)
    assert o.tot["fail"][0] >= 2
    # a certain frame error: every attempt fails, the message is dropped after max_tx = 7 attempts
    o, out = _one_event(0, 30, fer=0.999999)
    assert o.tot["succ"][0] == 0
    assert not out["delivered"][0].any()


def _saturation(n, E=4, warm=5, steps=60, seed=1):
    o = DcfOracle(E, n, sat_cfg(), seed=seed)
    snap = None
    for s in range(warm + steps):
        if s == warm:
            snap = {k: v.copy() for k, v in o.tot.items()}
        for _ in range(2):
            o.submit(None, torch.ones(E, n, dtype=torch.long))
        o.step(None, torch.full((E, n), 40.0))
    t = {k: o.tot[k] - snap[k] for k in o.tot}
    p = t["fail"].sum() / t["att"].sum()
    busy = t["busy_ns"].sum() / (E * steps * 20e6)
    return p, busy


@pytest.mark.parametrize("i", [0, 1, 2])
def test_saturation_matches_the_reference_event_simulator(i):
    torch.set_num_threads(1)
    ref = np.load(os.path.join(GOLDEN, "eventsim_sat.npz"))
    n = int(ref["n"][i])
    p, busy = _saturation(n)
    p_ref = 1.0 - ref["n_succ"][i] / ref["n_att"][i]
    assert abs(p - p_ref) < 0.015, (n, p, p_ref)
    assert abs(busy - ref["busy_frac"][i]) < 0.01, (n, busy, ref["busy_frac"][i])


def test_saturation_matches_bianchi():
    """n = 10 stations, W0 = 16, Wmax = 1024, 7 attempts: the mean-field fixed point of the WIFI level."""
    from oracle.wifi_oracle import WifiOracle
    p, _ = _saturation(10)
    cfg = sat_cfg(fp_iters=300)
    mf = WifiOracle(1, 10, cfg)
    w = torch.ones(1, 11)
    w[0, 10] = 0.0
    W0, Wm = torch.full((1, 11), 16.0), torch.full((1, 11), 1024.0)
    ts, tc = torch.full((1, 11), 200.0), torch.full((1, 11), 150.0)
    _, pm, _, _ = mf._solve(w, ts, tc, torch.full((1, 11), 0.1), mf._stage_factors(W0, Wm, 7))
    assert abs(p - float(pm[0, 0])) < 0.02, (p, float(pm[0, 0]))


def test_idle_rebase_changes_nothing():
    """Bursts of traffic between idle stretches of up to 30 steps, with stations losing and regaining their link:
    the oracle with the bounded idle anchor gives the same outputs and FIFO state as with the unbounded one, and its
    integers stay small while the unbounded anchor drifts by the idle time."""
    cfg = P.NRConfig(control_step_ms=2.0, frame_buffer=8, msg_sizes=(1500.0, 9000.0), timeout_steps=40,
                     wifi=WifiConfig(access_category="DCF", max_ampdu_bytes=0))
    E, R = 3, 6
    a, b = DcfOracle(E, R, cfg, seed=5), DcfOracle(E, R, cfg, seed=5)
    b.rebase = False
    rs = np.random.default_rng(2)
    lo_a = lo_b = 0
    for s in range(160):
        if (s // 30) % 2 == 0 or s % 61 == 0:
            send = torch.from_numpy(rs.choice([0, 0, 0, 0, 1, 2], size=(E, R)).astype(np.int64))
            np.testing.assert_array_equal(a.submit(None, send).numpy(), b.submit(None, send).numpy())
        snr = torch.from_numpy(rs.choice([-20.0, 15.0, 40.0], p=[0.1, 0.3, 0.6], size=(E, R)).astype(np.float32))
        oa, ob = a.step(None, snr), b.step(None, snr)
        for k in oa:
            np.testing.assert_array_equal(oa[k].numpy(), ob[k].numpy(), err_msg=f"step {s} {k}")
        np.testing.assert_array_equal(a.rem.numpy(), b.rem.numpy())
        np.testing.assert_array_equal(a.stage, b.stage)
        lo_a, lo_b = min(lo_a, int(a.t_idle.min())), min(lo_b, int(b.t_idle.min()))
        assert a.b.max() < 4 * a.k["Wmax"]
    k = a.k
    assert lo_a >= -(k["sifs"] + (k["aifsn"] + 1) * k["slot"] + k["T"] + 6_000_000)
    assert lo_b < -5 * k["T"]                                 # the unbounded anchor did drift

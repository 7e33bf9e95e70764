"""Level WIFI_DCF on the GPU: the HIP engine against the CPU oracle (oracle/dcf_oracle.py), free running from the same
seed on the same submits and inputs, step by step.

Bar: every integer and boolean (backoff counters, retry stages, contention flags, idle anchors, FIFO fields, queue
lengths, deliveries, timeouts, MCS, counters, clock) bit-exact; the DCF floats are exact too (finish times and delays
are one double division rounded once, the access time, failure share and busy share are the same double sums on both
sides), so they are compared bitwise. SNR from poses (radio model: float32 transcendental functions) within 1e-5
relative and the plane-wave vectors within two float32 ulp, as for level WIFI; the scenarios fed with SNR directly
are exact end to end."""
import zlib

import numpy as np
import pytest
import torch

from oracle.dcf_oracle import DcfOracle
from test_gpu_wifi import FIELD_KEYS, MAX_DEV, close
import isaac_net_amd as P
from isaac_net_amd.wifi_config import WifiConfig

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def scenario(name):
    """(cfg, E, R, steps, arrivals per step (mean), input 'snr' or 'pose', reset every n steps or 0, idle pattern)."""
    W, N = WifiConfig, P.NRConfig
    if name == "snr_basic":
        cfg = N(control_step_ms=20.0, frame_buffer=16, msg_sizes=(1500.0, 20000.0, 120000.0), timeout_steps=30,
                wifi=W())
        return cfg, 64, 16, 25, 0.8, "snr", 0, False
    if name == "pose_rts_fer":
        cfg = N(control_step_ms=10.0, frame_buffer=12, msg_sizes=(3000.0, 64000.0), timeout_steps=20,
                wifi=W(standard="ac", bandwidth_mhz=40, rts_cts=True, frame_error_rate=0.1, collision_time="ack",
                       access_category="VI"))
        return cfg, 48, 16, 20, 0.6, "pose", 0, False
    if name == "saturated_small_fifo":
        cfg = N(control_step_ms=5.0, frame_buffer=4, msg_sizes=(60000.0,), timeout_steps=8,
                wifi=W(access_category="DCF", max_tx=4))
        return cfg, 40, 32, 24, 2.0, "snr", 4, False
    if name == "ragged_idle":
        cfg = N(control_step_ms=2.0, frame_buffer=8, msg_sizes=(1500.0, 9000.5), timeout_steps=40,
                wifi=W(access_category="BK", max_ampdu_bytes=0))
        return cfg, 37, 5, 60, 0.5, "snr", 0, True
    if name == "r64_no_aggregation":
        cfg = N(control_step_ms=20.0, frame_buffer=8, msg_sizes=(1472.0, 2944.0), timeout_steps=10,
                wifi=W(max_ampdu_bytes=0, frame_error_rate=0.02))
        return cfg, 6, 64, 15, 1.0, "snr", 0, False
    if name == "legacy_a_single":
        cfg = N(control_step_ms=20.0, frame_buffer=8, msg_sizes=(1000.0,), timeout_steps=10,
                wifi=W(standard="a", gi_us=0.8, max_ampdu_bytes=0, access_category="VO"))
        return cfg, 16, 1, 15, 3.0, "snr", 0, False
    raise KeyError(name)


SCENARIOS = ["snr_basic", "pose_rts_fer", "saturated_small_fifo", "ragged_idle", "r64_no_aggregation",
             "legacy_a_single"]


class _Ref(dict):
    files = property(lambda self: list(self.keys()))


def compare_all(og, eng, oo, orc):
    ref = _Ref({f"s/out.{k}": v.numpy() for k, v in oo.items()})
    ref.update({f"s/{k}": v.numpy() if torch.is_tensor(v) else np.asarray(v) for k, v in orc.state().items()})
    vals = {"out." + k: v for k, v in og.items()}
    vals.update(eng.state_dict())
    bad = {}
    for k, v in vals.items():
        rk = "s/" + k
        if rk not in ref:
            continue
        m = v.detach().cpu().numpy() if torch.is_tensor(v) else np.asarray(v)
        r = ref[rk]
        if m.dtype == np.bool_ or r.dtype == np.bool_:
            m, r = m.astype(np.int64), r.astype(np.int64)
        ok = close(k, m, r) if k in ("_last_snr", "f_snr", "out.sinr_db") + FIELD_KEYS else \
            (m.shape == r.shape and ((m == r) | ((m != m) & (r != r))).all())
        if not np.all(ok):
            bad[k] = int((~np.asarray(ok)).sum()) if np.shape(ok) else -1
    return bad


@pytest.mark.parametrize("name", SCENARIOS)
def test_dcf_free_running_vs_oracle(name):
    cfg, E, R, T, lam, kind, every, idle = scenario(name)
    print(f"dcf scenario {name}: E={E} R={R} steps={T} input={kind}", flush=True)
    eng = P.make_engine("WIFI_DCF", E, R, DEV, cfg, seed=7)
    orc = DcfOracle(E, R, cfg, seed=7)
    rs = np.random.default_rng(zlib.crc32(name.encode()))
    n_cls = len(cfg.msg_sizes)
    pos = None
    if kind == "pose":
        rad = 40.0 * np.sqrt(rs.uniform(size=(E, R)))
        ang = rs.uniform(0, 2 * np.pi, size=(E, R))
        pos = np.stack([rad * np.cos(ang), rad * np.sin(ang)], -1).astype(np.float32)
    bad = compare_all({}, eng, {}, orc)
    assert not bad, ("init", bad)
    stats = np.zeros(3, np.int64)
    for s in range(T):
        if every and s and s % every == 0:
            ids = np.nonzero(rs.uniform(size=E) < 0.3)[0]
            eng.reset(ids.tolist())
            orc.reset(ids.tolist())
        quiet = idle and (s // 12) % 2 == 1
        counts = np.zeros((E, R), np.int64) if quiet else rs.poisson(lam, size=(E, R))
        for i in range(int(counts.max(initial=0))):
            send = np.where(counts > i, rs.integers(1, n_cls + 1, size=(E, R)), 0).astype(np.int64)
            acc_g = eng.submit(None, torch.from_numpy(send).to(DEV)).cpu().numpy()
            acc_o = orc.submit(None, torch.from_numpy(send)).numpy()
            assert np.array_equal(acc_g, acc_o), (s, "accepted")
        if kind == "pose":
            x = pos
            pos = pos + rs.normal(0, 0.7, size=pos.shape).astype(np.float32)
        else:
            x = rs.choice([-8.0, 3.5, 12.0, 21.0, 33.0, 47.0], p=[0.05, 0.1, 0.15, 0.2, 0.25, 0.25],
                          size=(E, R)).astype(np.float32) + rs.uniform(-2, 2, size=(E, R)).astype(np.float32)
        og = eng.step(None, torch.from_numpy(x).to(DEV))
        oo = orc.step(None, torch.from_numpy(x))
        bad = compare_all(og, eng, oo, orc)
        assert not bad, (s, bad)
        stats[2] += int(og["delivered"].sum())
    stats[0], stats[1] = int(orc.tot["att"].sum()), int(orc.tot["fail"].sum())
    print(f"{name}: attempts {stats[0]}, failed {stats[1]}, deliveries {stats[2]}; "
          f"max |deviation| { {k: f'{v:.2e}' for k, v in MAX_DEV.items()} }", flush=True)
    MAX_DEV.clear()
    assert stats[0] > 0 and stats[2] > 0


def test_dcf_parameters_match_the_oracle():
    """The engine's integer timing table equals the oracle's, for every standard the scenarios use."""
    for name in SCENARIOS:
        cfg, E, R, *_ = scenario(name)
        eng = P.make_engine("WIFI_DCF", 1, R, DEV, cfg, seed=0)
        k = DcfOracle(1, R, cfg).k
        p = eng._cdparams
        assert list(p.ndbps)[:len(k["ndbps"])] == k["ndbps"], name
        for f in ("T", "tsym", "pre", "sifs", "slot", "t_ack", "t_rts", "t_cts", "W0", "Wmax", "aifsn", "ovh",
                  "payload"):
            assert getattr(p, f) == k[f], (name, f)


def test_dcf_teacher_forced_from_oracle_state():
    """Load the oracle's full state (FIFO, counters, stages, idle anchor) into the engine at every step of a
    saturated run and compare one step: the kernel's event loop from arbitrary mid-run states."""
    cfg, E, R, T, lam, kind, every, idle = scenario("saturated_small_fifo")
    eng = P.make_engine("WIFI_DCF", E, R, DEV, cfg, seed=9)
    orc = DcfOracle(E, R, cfg, seed=9)
    rs = np.random.default_rng(4)
    for s in range(10):
        counts = rs.poisson(lam, size=(E, R))
        for i in range(int(counts.max(initial=0))):
            orc.submit(None, torch.from_numpy(np.where(counts > i, 1, 0).astype(np.int64)))
        eng.load_state_dict({k: v.clone() if torch.is_tensor(v) else v for k, v in orc.state().items()})
        x = rs.uniform(5, 45, size=(E, R)).astype(np.float32)
        og = eng.step(None, torch.from_numpy(x).to(DEV))
        oo = orc.step(None, torch.from_numpy(x))
        bad = compare_all(og, eng, oo, orc)
        assert not bad, (s, bad)


def test_dcf_refusals():
    with pytest.raises(P.HipUnsupported):
        P.make_engine("WIFI_DCF", 2, 4, DEV, P.NRConfig(wifi=WifiConfig(bg_stations=3)))
    with pytest.raises(P.HipUnsupported):
        P.make_engine("WIFI_DCF", 2, 4, DEV, P.NRConfig(wifi=WifiConfig(class_ac=("VO", "BE"))))


def test_config4_workload_prefix_vs_oracle():
    """The benchmarked WIFI_DCF workload itself (wifi_dcf_slots: 2048 envs x 16 stations at one AP, access category
    DCF, 802.11ax 20 MHz, stations in a 50 m disc on a 1 m/s random walk, 1500 B at Poisson 0.4, FIFO 16, 20 ms
    steps) for 60 control steps: its first 64 envs bit for bit against the oracle at every step (outputs and state,
    SNR from poses within its float32 bound), and over all 2048 envs the counter invariants: each backoff counter
    inside its retry stage's window, stages below the retry limit, queue lengths in [0, F]."""
    from isaac_net_amd import scenarios as B
    E, R, steps, E_chk = 2048, 16, 60, 64
    print(f"wifi_dcf_slots {E}x{R}, {steps} steps, oracle on {E_chk} envs", flush=True)
    wl = B.Workload(E, R, steps, seed=0, name="wifi_dcf_slots")
    cfg = wl.cfg
    eng = P.make_engine("WIFI_DCF", E, R, DEV, cfg, seed=0)
    orc = DcfOracle(E_chk, R, cfg, seed=0)
    p = eng._cdparams
    max_tx = eng.wc.max_tx
    F = cfg.frame_buffer

    def head(v):
        if not torch.is_tensor(v) or v.dim() == 0:
            return v
        if v.dim() >= 2 and v.shape[0] == 1 and v.shape[1] == E:          # radio fields [1, E, K, ...]
            return v[:, :E_chk]
        return v[:E_chk] if v.shape[0] == E else v

    class _Prefix:                                     # the engine's outputs and state of the first E_chk envs
        def __init__(self, e):
            self.e = e

        def state_dict(self):
            return {k: head(v) for k, v in self.e.state_dict().items()}

    n_del = n_att = 0
    for s in range(steps):
        c = wl.counts[s]
        eng.submit_counts(c.to(DEV))
        cn = c[:E_chk].numpy()
        for ci in range(cn.shape[-1]):                 # the calls of the counts form are global: up to the largest
            for i in range(int(c[..., ci].max())):     # count over every env
                orc.submit(None, torch.from_numpy(np.where(cn[..., ci] > i, ci + 1, 0).astype(np.int64)))
        x = wl.poses[s]
        og = eng.step(None, x.to(DEV))
        oo = orc.step(None, x[:E_chk])
        bad = compare_all({k: head(v) for k, v in og.items()}, _Prefix(eng), oo, orc)
        assert not bad, (s, bad)
        b, st = eng.dst["b"].long(), eng.dst["stage"].long()
        win = torch.clamp(p.W0 * torch.pow(2, st), max=p.Wmax)
        assert bool((b >= 0).all()) and bool((b <= win - 1).all()), s
        assert bool((st >= 0).all()) and bool((st < max_tx).all()), s
        ql = og["queue_len"]
        assert int(ql.min()) >= 0 and int(ql.max()) <= F, s
        n_del += int(og["delivered"].sum())
    n_att = int(orc.tot["att"].sum())
    print(f"config 4: {n_del} deliveries over {E} envs, {n_att} attempts and {int(orc.tot['fail'].sum())} failures "
          f"in the first {E_chk}; max |deviation| { {k: f'{v:.2e}' for k, v in MAX_DEV.items()} }", flush=True)
    MAX_DEV.clear()
    assert n_del > 0 and n_att > 0

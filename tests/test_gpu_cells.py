"""Several cells per env (inet_nr_step_cells: NRNet.step_cells with A3 association and same-slot UL interference) on
the GPU beyond the golden trajectories: the three-cell interference workload at its real shape (1024 envs x 64
robots, 14 RBGs, so each interference sum runs over 64 robots in torch's chunked order) with the oracle on its first
envs; handovers with RLC flush, HARQ-IR, round robin and an N+I EWMA against the oracle (the flush path has no
reference trajectory: there the oracle's restatement is the bar); the fused arrivals against submit_counts + step."""
import numpy as np
import pytest
import torch

import isaac_net_amd as P
from gpu_util import head, submit_oracle
from oracle import nr_oracle as O
from oracle.tolerance import FlipCounter, engine_radio, ni_rel_bound, sinr_bound

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def serving_bound(eng, n, x, serv, snr):
    """sinr_db bound of the first n envs: the shadowing-rounding bound of each robot's serving cell."""
    fi, sig, amp = engine_radio(eng)
    f = eng.st["field"][:n, :, fi].cpu().numpy()                     # [n, C, K, 3]
    b = np.stack([sinr_bound(x, f[:, c], sig, amp, snr) for c in range(f.shape[1])], -1)
    return np.take_along_axis(b, serv[..., None], -1)[..., 0]


def run_against_oracle(cfg, E, R, steps, E_chk, poses, counts, resets=(), seed=0):
    """Drive the engine (E envs) and the oracle (its first E_chk envs) with the same inputs. Returns (engine, oracle,
    flip counter, largest ratio of an N+I deviation to its bound (oracle.tolerance.ni_rel_bound, the running max over
    the steps since the EWMA carries older estimates) over the envs that never diverged). Their serving cells must be
    equal."""
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=seed)
    ora = O.OracleEngine(E_chk, R, cfg, seed=seed)
    fc = FlipCounter(E_chk, ora)
    fi, sig, amp = engine_radio(eng)
    ni_dev, nib = 0.0, np.zeros((E_chk, cfg.n_cells))
    for s in range(steps):
        ids = [e for (t, e) in resets if t == s]
        if ids:
            eng.reset(ids)
            ora.reset([e for e in ids if e < E_chk])
        c = counts[s]
        eng.submit_counts(torch.as_tensor(c).to(DEV))
        submit_oracle(ora, np.asarray(c)[:E_chk])
        x = torch.as_tensor(poses[s])
        og = eng.step(None, x.to(DEV))
        xc = x[:E_chk].cpu()
        fc.before()
        oo = ora.step(None, xc)
        serv_o = oo["serving_cell"].numpy()
        f = eng.st["field"][:E_chk, :, fi].cpu().numpy()
        nib = np.maximum(nib, ni_rel_bound(x[:E_chk].cpu().numpy(), [f[:, c] for c in range(f.shape[1])], sig, amp))
        # the reported SINR is against the serving gNB's N+I estimate, which carries its own bound (relative, so
        # 10 / ln 10 times it in dB); the UL reference and the decoding SINR of the threshold decisions carry the
        # estimate and this slot's N+I measurement
        ni_db = (10.0 / np.log(10.0)) * np.take_along_axis(nib, serv_o, 1)
        tol = serving_bound(eng, E_chk, xc.numpy(), serv_o, oo["sinr_db"].numpy()) + ni_db
        mine = eng.owner_state()
        fc.step(s, {k: v[:E_chk] for k, v in og.items() if v.dim() >= 2}, oo, tol, head(mine, E_chk),
                lambda o, xc=xc: o.step(None, xc), dec_bound=tol + ni_db)
        alive = fc.alive
        assert np.array_equal(og["serving_cell"][:E_chk].cpu().numpy()[alive], serv_o[alive]), s
        ni = mine["net.ni_ul"][:E_chk].cpu().numpy().astype(np.float64)[alive]
        ni_o = ora.ni_ul.numpy().astype(np.float64)[alive]
        if ni.size:
            ni_dev = max(ni_dev, float((np.abs(ni - ni_o) / (np.abs(ni_o) * nib[alive][..., None])).max()))
    return eng, ora, fc, ni_dev


def test_interference_workload_prefix_parity():
    """mc_interf at its real shape: 1024 envs x 64 robots, 3 cells, 106 PRBs, 100 control steps; the first 6 envs
    against the oracle, association and interference invariants over every env."""
    from isaac_net_amd import scenarios as B
    E, R, steps, E_chk = 1024, 64, 100, 6
    print(f"mc_interf {E}x{R}, {steps} steps", flush=True)
    wl = B.Workload(E, R, steps, seed=0, name="mc_interf")
    cfg = wl.cfg
    eng, ora, fc, ni_dev = run_against_oracle(cfg, E, R, steps, E_chk, wl.poses, wl.counts)
    st = eng.owner_state()
    serv = st["assoc.serv"]
    assert int(serv.min()) >= 0 and int(serv.max()) < 3 and int(st["assoc.n_ho"].sum()) == 0
    assert not bool(st["assoc.pending"].any())
    noise = 10 ** (cfg.noise_dbm_per_prb("gnb") / 10)
    ni = st["net.ni_ul"]
    assert bool((ni >= noise * (1 - 1e-6)).all()) and bool((ni > noise * 1.01).any())     # interference is there
    assert eng.counters()["ul"]["tb_new"] > 0
    print(f"prefix parity: {E_chk} envs x {steps} steps: {fc.report()}, N+I deviation / bound {ni_dev:.2f}",
          flush=True)
    assert fc.ok(E_chk * R * steps) and ni_dev <= 1.0, fc.report()


def test_handover_flush_rr_against_oracle():
    """A3 handovers under fast motion with ho_rlc="flush" (queued frames dropped at the switch), round robin, an N+I
    EWMA (li_alpha 0.3) and a partial reset, against the oracle on every env."""
    cfg = P.NRConfig(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="rr", n_harq=4,
                     max_harq_tx=3, frame_buffer=8, msg_sizes=(2500.0, 400.0), n_cells=3,
                     cell_layout="hex", cell_isd_m=120.0, cell_center_m=(60.0, 60.0), noise_model="thermal",
                     a3_ttt_ms=10.0, ho_interruption_ms=2.5, ho_rlc="flush", li_alpha=0.3, fading_rho_per_ms=0.5)
    E, R, steps = 4, 16, 30
    rs = np.random.default_rng(4)
    p = rs.uniform(0.0, 200.0, (E, R, 2))
    poses, counts = [], []
    for _ in range(steps):
        poses.append(p.astype(np.float32))
        ang = rs.uniform(0.0, 2 * np.pi, (E, R))
        p = np.clip(p + 8.0 * np.stack([np.cos(ang), np.sin(ang)], -1), 0.0, 200.0)
        counts.append(np.stack([rs.poisson(0.5, (E, R)), rs.poisson(1.0, (E, R))], -1).astype(np.uint8))
    eng, ora, fc, ni_dev = run_against_oracle(cfg, E, R, steps, E, poses, counts, resets=((12, 1), (12, 2)), seed=3)
    n_ho = int(eng.owner_state()["assoc.n_ho"].sum())
    lost = eng.counters()["ul"]["lost_frames"]
    print(f"handovers {n_ho}, lost frames {lost}: {fc.report()}, N+I deviation / bound {ni_dev:.2f}", flush=True)
    assert n_ho > 0 and lost > 0
    assert fc.ok(E * R * steps) and ni_dev <= 1.0, fc.report()


def test_cells_fused_arrivals_equal_submit_counts_then_step():
    """step(arrivals=counts) with several cells leaves every output and state tensor bitwise equal to
    submit_counts(counts) followed by step(), through handovers (RLC UM drop) and a partial reset."""
    cfg = P.NRConfig(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, n_harq=4, max_harq_tx=3,
                     harq_fail="drop", frame_buffer=8, msg_sizes=(2500.0, 400.0), n_cells=3, cell_layout="hex",
                     cell_isd_m=120.0, cell_center_m=(60.0, 60.0), noise_model="thermal", a3_ttt_ms=10.0,
                     ho_interruption_ms=5.0)
    E, R = 5, 32
    a = P.make_engine("L2", E, R, DEV, cfg, seed=5)
    b = P.make_engine("L2", E, R, DEV, cfg, seed=5)
    rs = np.random.default_rng(6)
    p = rs.uniform(0.0, 200.0, (E, R, 2))
    for s in range(14):
        if s == 6:
            a.reset([0, 3])
            b.reset([0, 3])
        counts = torch.from_numpy(np.stack([rs.poisson(0.7, (E, R)), rs.poisson(0.7, (E, R))], -1)
                                  .astype(np.uint8)).to(DEV)
        ang = rs.uniform(0.0, 2 * np.pi, (E, R))
        p = np.clip(p + 8.0 * np.stack([np.cos(ang), np.sin(ang)], -1), 0.0, 200.0)
        x = torch.from_numpy(p.astype(np.float32)).to(DEV)
        acc_a = a.submit_counts(counts)
        oa = a.step(None, x)
        ob = b.step(None, x, arrivals=counts)
        assert torch.equal(acc_a, ob["arrivals_accepted"]), s
        for k in oa:
            assert torch.equal(oa[k].nan_to_num(), ob[k].nan_to_num()), (s, k)
        sa, sb = a.owner_state(), b.owner_state()
        for k in sa:
            assert torch.equal(sa[k].nan_to_num(), sb[k].nan_to_num()), (s, k)
    assert int(a.owner_state()["assoc.n_ho"].sum()) > 0

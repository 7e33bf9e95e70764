"""Contract API of the HIP engine (isaac_net/core/engine.py NREngine): clock rules, partial reset forms, submit
acceptance and overflow, the legacy step form, output schema, and env independence (an env's trajectory does not
depend on E or on other envs' resets)."""
import numpy as np
import pytest
import torch

import isaac_net_amd as P
from gpu_util import head
from oracle import nr_oracle as O
from oracle.tolerance import FlipCounter, engine_radio, sinr_bound

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def small_cfg(**kw):
    base = dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="pf", n_harq=4, max_harq_tx=4, frame_buffer=6,
                msg_sizes=(1500.0, 300.0), channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                cell_positions_m=((50.0, 50.0),), gnb_height_m=10.0, fading_rho_per_ms=0.0)
    base.update(kw)
    return P.NRConfig(**base)


def poses(E, R, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(E, R, 2, generator=g) * 100).to(DEV)


def test_clock_and_time_rules():
    eng = P.make_engine("L2", 3, 4, DEV, small_cfg(), seed=1)
    assert eng.clock.tolist() == [0, 0, 0]
    o = eng.step(0, poses(3, 4, 0))
    assert o["t"].tolist() == [0, 0, 0] and eng.clock.tolist() == [1, 1, 1]
    with pytest.raises(ValueError):
        eng.step(5, poses(3, 4, 1))
    eng.step(None, poses(3, 4, 1))
    eng.reset([1])
    assert eng.clock.tolist() == [2, 0, 2]
    with pytest.raises(ValueError):
        eng.step(2, poses(3, 4, 2))
    o = eng.step(None, poses(3, 4, 2))
    assert o["t"].tolist() == [2, 0, 2]
    o = eng.step(torch.tensor([3, 1, 3]), poses(3, 4, 3))
    assert o["t"].tolist() == [3, 1, 3]


def test_output_schema_and_dtypes():
    eng = P.make_engine("L2", 2, 5, DEV, small_cfg(), seed=2)
    eng.submit(None, torch.ones(2, 5, dtype=torch.long, device=DEV))
    o = eng.step(None, poses(2, 5, 0))
    sch = eng.output_schema()
    assert list(o.keys()) == list(sch.keys())
    F = 6
    for k, info in sch.items():
        shape = tuple({"E": 2, "R": 5, "F": F}[c] for c in info["shape"].strip("[]").split(","))
        assert tuple(o[k].shape) == shape, k
        assert str(o[k].dtype).replace("torch.", "") == info["dtype"], k


def test_submit_accepts_until_the_buffer_is_full():
    eng = P.make_engine("L2", 2, 3, DEV, small_cfg(frame_buffer=2), seed=3)
    send = torch.tensor([[1, 0, 2], [2, 2, 0]], device=DEV)
    a1 = eng.submit(None, send)
    a2 = eng.submit(None, send)
    a3 = eng.submit(None, send)
    assert a1.tolist() == [[True, False, True], [True, True, False]]
    assert a2.tolist() == a1.tolist()
    assert not bool(a3.any())
    st = eng.owner_state()
    assert st["ul.q.enq"].tolist() == [[3000, 0, 600], [600, 600, 0]]
    assert st["ul.q.cls"][0, 0, :2].tolist() == [1, 1]


def test_reset_forms_are_equivalent():
    outs = []
    for ids in ([1, 2], torch.tensor([1, 2], device=DEV), torch.tensor([False, True, True, False], device=DEV)):
        eng = P.make_engine("L2", 4, 3, DEV, small_cfg(), seed=4)
        for s in range(3):
            eng.submit(None, torch.ones(4, 3, dtype=torch.long, device=DEV))
            eng.step(None, poses(4, 3, s))
        eng.reset(ids)
        eng.submit(None, torch.ones(4, 3, dtype=torch.long, device=DEV))
        outs.append({k: v.cpu() for k, v in eng.step(None, poses(4, 3, 9)).items()})
    for o in outs[1:]:
        for k in o:
            assert torch.equal(o[k].nan_to_num(-7), outs[0][k].nan_to_num(-7)), k


def test_legacy_step_form():
    eng = P.make_engine("L2", 2, 2, DEV, small_cfg(), seed=5)
    eng.submit(None, P.engine.Requests(send=torch.ones(2, 2, dtype=torch.long, device=DEV),
                                       det=torch.tensor([[True, False], [False, False]], device=DEV),
                                       hid=torch.tensor([7, 7], device=DEV)))
    newest, det_env = eng.step(None, poses(2, 2, 0), torch.tensor([7, 7], device=DEV))
    assert newest.shape == (2, 2) and det_env.shape == (2,)
    assert newest.dtype == torch.int64 and det_env.dtype == torch.bool


def test_env_independence():
    """Env e's results depend only on (seed, e, its episode and inputs): a 2-env engine equals the first 2 envs of
    a 6-env engine whose other envs are reset at random steps."""
    cfg = small_cfg()
    a = P.make_engine("L2", 2, 4, DEV, cfg, seed=6)
    b = P.make_engine("L2", 6, 4, DEV, cfg, seed=6)
    g = torch.Generator().manual_seed(0)
    for s in range(12):
        send = (torch.rand(6, 4, generator=g) < 0.7).long().to(DEV)
        x = poses(6, 4, 100 + s)
        a.submit(None, send[:2])
        b.submit(None, send)
        if s in (3, 8):
            b.reset([3, 5])
        oa, ob = a.step(None, x[:2]), b.step(None, x)
        for k in oa:
            if k in ("t",):
                continue
            va, vb = oa[k].cpu(), ob[k][:2].cpu()
            assert torch.equal(va.nan_to_num(-7), vb.nan_to_num(-7)), (s, k)


def test_matches_oracle_with_submit_counts():
    """submit_counts (one launch for several messages per robot, class order) equals the sequence of submit calls,
    checked against the oracle driven by those calls."""
    cfg = small_cfg(control_step_ms=25.0, n_harq=8, frame_buffer=8, fading_rician=True, rician_k_db=3.0)
    E, R = 3, 8
    eng = P.make_engine("L2", E, R, DEV, cfg, seed=11)
    ora = O.OracleEngine(E, R, cfg, seed=11)
    fc = FlipCounter(E, ora)
    rs = np.random.default_rng(1)
    for s in range(10):
        counts = np.stack([rs.poisson(0.8, (E, R)), rs.poisson(0.3, (E, R))], -1).astype(np.uint8)
        acc = eng.submit_counts(torch.from_numpy(counts).to(DEV))
        n_acc = np.zeros((E, R), np.int64)
        for ci in range(2):
            for i in range(int(counts[..., ci].max())):
                send = torch.from_numpy(np.where(counts[..., ci] > i, ci + 1, 0).astype(np.int64))
                n_acc += ora.submit(None, send).numpy()
        assert np.array_equal(acc.cpu().numpy(), n_acc)
        x = torch.from_numpy(rs.uniform(0, 100, (E, R, 2)).astype(np.float32))
        og = eng.step(None, x.to(DEV))
        fc.before()
        oo = ora.step(None, x)
        fi, sig, amp = engine_radio(eng)
        tol = sinr_bound(x.numpy(), eng.st["field"][:, 0, fi].cpu().numpy(), sig, amp, oo["sinr_db"].numpy())
        fc.step(s, og, oo, tol, head(eng.owner_state(), E), lambda o, x=x: o.step(None, x))
    print(fc.report(), flush=True)
    assert fc.ok(E * R * 10), fc.report()


@pytest.mark.parametrize("variant", ["plain", "pdcp_overhead_small_fifo"])
def test_fused_arrivals_equal_submit_counts_then_step(variant):
    """step(arrivals=counts) (inet_nr_submit_step: the enqueue inside the step's launch) leaves every output and
    every state tensor bitwise equal to submit_counts(counts) followed by step(), over steps with overflow,
    PDCP discard and per-packet overhead, and a partial reset."""
    kw = dict(control_step_ms=25.0, n_harq=8, frame_buffer=8, fading_rician=True, rician_k_db=3.0)
    if variant != "plain":
        kw.update(frame_buffer=3, discard="pdcp_arrival", timeout_steps=2, pkt_overhead_bytes=40,
                  pkt_payload_bytes=600)
    cfg = small_cfg(**kw)
    E, R = 6, 32
    a = P.make_engine("L2", E, R, DEV, cfg, seed=5)
    b = P.make_engine("L2", E, R, DEV, cfg, seed=5)
    rs = np.random.default_rng(3)
    for s in range(12):
        if s == 7:
            a.reset([1, 4])
            b.reset([1, 4])
        counts = torch.from_numpy(np.stack([rs.poisson(1.2, (E, R)), rs.poisson(0.4, (E, R))], -1)
                                  .astype(np.uint8)).to(DEV)
        x = torch.from_numpy(rs.uniform(0, 100, (E, R, 2)).astype(np.float32)).to(DEV)
        acc_a = a.submit_counts(counts)
        oa = a.step(None, x)
        ob = b.step(None, x, arrivals=counts)
        assert torch.equal(acc_a, ob["arrivals_accepted"]), s
        for k in oa:
            assert torch.equal(oa[k], ob[k]) or (oa[k].is_floating_point() and
                                                 torch.equal(oa[k].isnan(), ob[k].isnan()) and
                                                 torch.equal(oa[k].nan_to_num(), ob[k].nan_to_num())), (s, k)
        sa, sb = a.owner_state(), b.owner_state()
        for k in sa:
            va, vb = sa[k], sb[k]
            if va.is_floating_point():
                assert torch.equal(va.nan_to_num(), vb.nan_to_num()), (s, k)
            else:
                assert torch.equal(va, vb), (s, k)

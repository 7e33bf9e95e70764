"""Statistics of the HIP NR engine (log_stats, collect(), queued(), refused_env, clear_stats()) against the
reference NRNet's on the same inputs (tests/golden/stats_*.npz, written by tests/golden/make_fixtures.py from
isaac_net/core/nr_engine.py:440-497, 885-914 with log_stats on from construction).

stats_ul: poses, PF, HARQ drop, purge timeouts, a 6-frame FIFO, two classes and a partial reset; stats_dl: SNR input,
RR, PDCP discard on arrival, UL and DL traffic with small FIFOs, a partial reset and log_cap_max = 20. Every count,
env index, class, f_nact, f_own and delay is compared bit-exactly; f_snr is the previous step's SNR, which with poses
carries the radio's float32 rounding (its per-step bound is checked by the trajectory tests), so it is compared within
1e-3 dB there and exactly with SNR input."""
import json
import os

import numpy as np
import pytest
import torch

import isaac_net_amd as P
from conftest import GOLDEN
from oracle.replay import load_case

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _drive(eng, z, per_step=None):
    """The fixture's call sequence: resets, one submit() per class and message index, the DL frames, the step."""
    T, E, R = int(z["steps"]), int(z["E"]), int(z["R"])
    counts, x, resets = z["counts"], z["x"], z["reset_mask"]
    dl_counts = z["dl_counts"] if "dl_counts" in z.files else None
    for s in range(T):
        ids = np.nonzero(resets[s])[0]
        if len(ids):
            eng.reset(torch.tensor(ids, dtype=torch.long))
        for ci in range(counts.shape[-1]):
            n = torch.from_numpy(counts[s, :, :, ci]).to(DEV)
            for i in range(int(n.max())):
                eng.submit(None, P.Requests(send=torch.where(n > i, torch.full_like(n, ci + 1), torch.zeros_like(n))))
        if dl_counts is not None:
            for ci in range(dl_counts.shape[-1]):
                n = torch.from_numpy(dl_counts[s, :, :, ci]).to(DEV)
                for i in range(int(n.max())):
                    nb = torch.where(n > i, torch.full(n.shape, float(z["dl_sizes"][ci]), device=DEV),
                                     torch.zeros(n.shape, device=DEV))
                    eng.add_dl_frames(None, nb, torch.where(n > i, torch.full_like(n, ci + 1), torch.zeros_like(n)))
        eng.step(None, torch.from_numpy(x[s]).to(DEV))
        if per_step is not None:
            per_step(s)


def _load(name):
    return load_case(os.path.join(GOLDEN, f"{name}.npz"))


def _engine(z, cfgd, **kw):
    cfg = P.NRConfig(**cfgd, seed=0)
    eng = P.make_engine("L2", int(z["E"]), int(z["R"]), DEV, cfg, seed=0, **kw)
    eng.log_stats = True
    eng.log_cap_max = int(z["log_cap_max"])
    return eng


@pytest.mark.parametrize("name", ["stats_ul", "stats_dl"])
@pytest.mark.parametrize("out_format", ["reference", "compact"])
def test_statistics_match_reference(name, out_format):
    z, cfgd, kind = _load(name)
    eng = _engine(z, cfgd, out_format=out_format)
    bad = []

    def check(s):
        for key, mine in (("queued", eng.queued()), ("refused_env", eng.refused_env)):
            ref = z[f"s{s:03d}/{key}"]
            m = mine.cpu().numpy()
            if m.dtype != ref.dtype or not np.array_equal(m, ref):
                bad.append((s, key))

    _drive(eng, z, check)
    assert not bad, bad[:8]
    col = eng.collect()
    keys = json.loads(bytes(z["collect_keys"]).decode())
    assert list(col.keys()) == keys
    snr_tol = 1e-3 if kind == "pose" else 0.0
    for k in keys:
        ref = z[f"collect/{k}"]
        if ref.ndim == 0:
            assert isinstance(col[k], int) and col[k] == int(ref), (k, col[k], int(ref))
            continue
        m = col[k].numpy()
        assert m.dtype == ref.dtype and m.shape == ref.shape, (k, m.dtype, m.shape, ref.dtype, ref.shape)
        if k.endswith("f_snr") and snr_tol:
            assert np.abs(m.astype(np.float64) - ref).max(initial=0.0) <= snr_tol, k
        else:
            assert np.array_equal(m, ref), (k, np.nonzero(m != ref)[0][:8])


def test_clear_stats_and_switching_off():
    """clear_stats() empties the record and refused_env; with log_stats off nothing is recorded; queued() is the
    queue length the step reports."""
    z, cfgd, _ = _load("stats_dl")
    eng = _engine(z, cfgd)
    _drive(eng, z)
    assert eng.collect()["delay"].numel() > 0 and int(eng.refused_env.sum()) > 0
    eng.clear_stats()
    col = eng.collect()
    assert all(v.numel() == 0 for v in col.values() if torch.is_tensor(v))
    assert int(eng.refused_env.sum()) == 0 and col["overflow"] == 0 and "overflow_dl" not in col
    eng.log_stats = False
    n = torch.ones(int(z["E"]), int(z["R"]), dtype=torch.long, device=DEV)
    for _ in range(8):
        eng.submit(None, n)
    o = eng.step(None, torch.zeros(int(z["E"]), int(z["R"]), device=DEV))
    assert torch.equal(eng.queued(), o["queue_len"])
    col = eng.collect()
    assert all(v.numel() == 0 for v in col.values() if torch.is_tensor(v)) and col["overflow"] == 0
    assert int(eng.refused_env.sum()) == 0


def test_counts_form_fused_arrivals_and_graph_log_as_single_submits():
    """submit_counts, step(arrivals=) and the graph step record the statistics of the submit() calls they stand for
    (class by class, message by message): the same collect() and refused_env as the single form on the stats_ul
    inputs."""
    z, cfgd, _ = _load("stats_ul")
    single = _engine(z, cfgd)
    _drive(single, z)
    ref = single.collect()
    T, counts, x, resets = int(z["steps"]), z["counts"], z["x"], z["reset_mask"]
    for mode in ("counts", "fused", "graph"):
        eng = _engine(z, cfgd)
        g = eng.graph_step() if mode == "graph" else None
        for s in range(T):
            ids = np.nonzero(resets[s])[0]
            if len(ids):
                eng.reset(torch.tensor(ids, dtype=torch.long))
            cnt = torch.from_numpy(counts[s]).to(DEV, torch.uint8)
            xs = torch.from_numpy(x[s]).to(DEV)
            if mode == "fused":
                eng.step(None, xs, arrivals=cnt)
            elif mode == "graph":
                g(xs, cnt)
            else:
                eng.submit_counts(cnt)
                eng.step(None, xs)
        col = eng.collect()
        assert list(col) == list(ref)
        for k, v in ref.items():
            if torch.is_tensor(v):
                assert torch.equal(col[k], v), (mode, k)
            else:
                assert col[k] == v, (mode, k)
        assert torch.equal(eng.refused_env, single.refused_env), mode

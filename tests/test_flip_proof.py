"""The float-threshold flip proof of the free-running comparisons (oracle.tolerance.FlipCounter / prove_flip), on the
CPU: a copy of the oracle with one threshold decision flipped (what a GPU rounding flip looks like) must be proven a
flip at the step it diverges, naming that decision; a copy with a planted arithmetic mistake (no threshold involved)
must stay unexplained."""
import numpy as np
import torch

import isaac_net_amd as P
from oracle import nr_oracle as O
from oracle.tolerance import FlipCounter, snapshot


def _cfg():
    return P.NRConfig(mu=1, n_prb=52, control_step_ms=10.0, scheduler="pf", n_harq=4, max_harq_tx=3,
                      frame_buffer=8, msg_sizes=(2500.0, 400.0), fading_rho_per_ms=0.0)


def _inputs(E, R, steps):
    rs = np.random.default_rng(3)
    snr = [torch.from_numpy(rs.uniform(-3.0, 20.0, (E, R)).astype(np.float32)) for _ in range(steps)]
    cnt = [np.stack([rs.poisson(0.9, (E, R)), rs.poisson(0.5, (E, R))], -1) for _ in range(steps)]
    return snr, cnt


def _submit(ora, c):
    for ci in range(c.shape[-1]):
        for i in range(int(c[..., ci].max(initial=0))):
            ora.submit(None, torch.from_numpy(np.where(c[..., ci] > i, ci + 1, 0).astype(np.int64)))


def _run(mutate, limit, E=3, R=8, steps=8, at=5, env=1):
    """Oracle A (the checker) against oracle B (the 'GPU'), B mutated at step `at` by mutate(B, recorded decisions)."""
    cfg = _cfg()
    a, b = O.OracleEngine(E, R, cfg, seed=4), O.OracleEngine(E, R, cfg, seed=4)
    fc = FlipCounter(E, a, limit=limit)
    snr, cnt = _inputs(E, R, steps)
    planted = None
    for s in range(steps):
        _submit(a, cnt[s])
        _submit(b, cnt[s])
        if s == at:
            probe = snapshot(b)
            probe.dec.record = True
            probe.step(None, snr[s])
            planted = mutate(b, probe.dec.rec, env, snr[s])
        fc.before()
        oa = a.step(None, snr[s])
        ob = b.step(None, snr[s])
        b.dec.force = {}
        fc.step(s, ob, oa, None, {k: v.clone() for k, v in b.state().items()}, lambda o, x=snr[s]: o.step(None, x))
    return fc, planted


def _flip_nearest(b, rec, env, x):
    """Force B's decision of `env` nearest to its threshold (decode draws, MCS lookups, link adaptation) among those
    whose flip changes the env's results."""
    from oracle.tolerance import diverged, int_view
    cands = []
    for site, k, av, bv in rec:
        if site not in ("dec", "mcs", "la"):
            continue
        d = (av[env].double() - bv[env].double()).abs()
        d = torch.where(torch.isfinite(d), d, torch.full_like(d, float("inf")))
        for i in torch.argsort(d.reshape(-1))[:40].tolist():
            cands.append((float(d.reshape(-1)[i]), site, k, np.unravel_index(i, d.shape), av.shape))
    cands.sort(key=lambda c: c[0])
    base = snapshot(b)
    ref_out = base.step(None, x)
    ref = int_view(ref_out, base.state(), [env])
    for _, site, k, idx, shape in cands:
        f = torch.zeros(shape, dtype=torch.bool)
        f[(env,) + tuple(int(j) for j in idx)] = True
        o = snapshot(b)
        o.dec.force = {(site, k): f}
        out = o.step(None, x)
        if diverged(int_view(out, o.state(), [env]), ref, 1).any():
            b.dec.force = {(site, k): f}
            return site
    raise AssertionError("no decision of the env changes its results")


def test_a_flipped_threshold_decision_is_proven():
    fc, site = _run(_flip_nearest, limit=float("inf"))
    assert not fc.unexplained, fc.report()
    assert len(fc.flips) == 1 and fc.flips[0][:2] == (5, 1) and fc.flips[0][2][0] == site, fc.report()


def test_a_planted_arithmetic_mistake_is_unexplained():
    def olla_step(b, rec, env, x):
        b.olla_dn = b.olla_dn * 1.001                    # a wrong OLLA down-step: no threshold decision explains it
        return None
    fc, _ = _run(olla_step, limit=float("inf"))
    assert fc.unexplained and not fc.flips, fc.report()
    assert fc.unexplained[0][0] == 5

"""Comparison rules between the HIP engine and the oracle / reference vectors. Test infrastructure only.

Integer state and integer outputs must be bit-exact. Float outputs carry the rounding of the reference formulas:
  * sinr_db (the pose -> SINR link budget): the shadowing term sigma * amp * sum_k cos(k . x + phi) is evaluated in
    float32 with |k . x| up to ~1e4 rad, so one ulp of a wave vector k (the reference's CPU cos / sin differ by an ulp
    between machines) moves the phase by |x| ulp(k). The bound per robot is
        1e-5 max(|sinr|, 1) + 4 ulp(128 dB) + 2 sigma amp sum_k (|x| ulp(|kx|) + |y| ulp(|ky|) + ulp(|arg_k|)).
  * other floats: see the callers (1e-5 relative with a unit floor for dB quantities).
A free-running comparison finds the envs whose integer outputs or integer state first differ at a step and proves
each one a float-threshold flip (a decision whose inputs differ by rounding: the oracle's step replayed with that one
decision flipped gives the GPU's results) or fails; only the envs that never diverged are compared afterwards.
"""
from __future__ import annotations

import numpy as np
import torch

INT_KEYS = ("delivered", "timed_out", "dropped", "cap", "cls", "newest", "queue_len", "queue_bytes")


def _ulp(v):
    return np.spacing(np.abs(np.asarray(v, dtype=np.float32))).astype(np.float64)


def sinr_bound(pos, field, sig, amp, sinr):
    """pos [E,R,2], field [E,K,3] (kx, ky, phi of the field the radio uses), sinr [E,R] -> bound [E,R]."""
    pos = np.asarray(pos, dtype=np.float64)
    f = np.asarray(field, dtype=np.float64)
    arg = pos[..., None, 0] * f[:, None, :, 0] + pos[..., None, 1] * f[:, None, :, 1] + f[:, None, :, 2]
    d = np.abs(pos[..., None, 0]) * _ulp(f[:, None, :, 0]) + np.abs(pos[..., None, 1]) * _ulp(f[:, None, :, 1]) + \
        _ulp(arg)
    s = np.asarray(sinr, dtype=np.float64)
    return 1e-5 * np.maximum(np.abs(s), 1.0) + 4 * float(np.spacing(np.float32(128.0))) + 2 * sig * amp * d.sum(-1)


def pg_bound(pos, field, sig, amp):
    """Bound [E,R] (dB) on the path-gain difference of one cell's link between two evaluations of the radio whose
    wave vectors differ by an ulp (the shadowing term of sinr_bound) plus 4 ulp of 128 dB for the rest of the link
    budget. pos [E,R,2], field [E,K,3]."""
    pos = np.asarray(pos, dtype=np.float64)
    f = np.asarray(field, dtype=np.float64)
    arg = pos[..., None, 0] * f[:, None, :, 0] + pos[..., None, 1] * f[:, None, :, 1] + f[:, None, :, 2]
    d = np.abs(pos[..., None, 0]) * _ulp(f[:, None, :, 0]) + np.abs(pos[..., None, 1]) * _ulp(f[:, None, :, 1]) + \
        _ulp(arg)
    return 4 * float(np.spacing(np.float32(128.0))) + 2 * sig * amp * d.sum(-1)


def ni_rel_bound(pos, fields, sig, amp):
    """Relative bound [E,C] on each gNB's N+I estimate with several cells: every interference term is
    10^(x / 10) of a dB sum x carrying its robot's path-gain difference to that cell (pg_bound) and, through the
    power-control backoff (alpha <= 1 times the serving link's path gain), the difference of its serving link, so
    its relative difference is at most ln(10) / 10 times their sum; the estimate is noise plus a sum of such terms.
    5e-5 covers the float32 rounding of x (a few ulp of ~100 dB, 1.75e-6 relative each). fields: [C] of [E,K,3]."""
    b = np.stack([pg_bound(pos, f, sig, amp) for f in fields], -1)               # [E,R,C]
    serv = b.max(-1, keepdims=True)                                              # any serving cell
    return 5e-5 + (np.log(10.0) / 10.0) * (b + serv).max(1)


def engine_radio(eng):
    """(field index, sigma, amp) of a HIP engine's radio constants."""
    p = eng._cparams
    fi = 1 if (p.radio_model == 1 and p.nl_b1 != 0.0) else 0
    return fi, (p.sig if p.radio_model == 1 else 1.0), p.amp


# integer (and exactly computed float) state compared per env in free running: a difference here is a diverged
# decision of this step, even where the outputs show it only in later steps
STATE_KEYS = ("sent", "floor", "bsr", "sr_t", "last_tx", "olla", "avg", "h_state", "h_ntx", "h_mcs", "h_nsb", "h_lo",
              "h_hi", "h_ready", "h_tbs", "q.cap", "q.start", "q.end", "q.lost", "q.cls", "q.enq", "q.fin")
ASSOC_KEYS = ("assoc.serv", "assoc.a3_cand", "assoc.a3_cnt", "assoc.ho_end", "assoc.n_ho")
# how far from its threshold a decision may sit and still be a rounding flip: probabilities (BLER target, decode
# draw) relative to the larger side, the PHR cap's PRB count relative, dB quantities absolute; each widened by the
# robot's radio bound (dB) where the inputs come from poses
PROB_SITES = ("la", "dec")


def _np(v):
    return v.detach().cpu().numpy() if hasattr(v, "detach") else np.asarray(v)


def int_view(out, state, envs):
    """{key: array [len(envs), ...]} of the integer outputs, delays and integer state of the given envs (frame fields
    of empty queue slots zeroed: the layouts leave stale values there)."""
    res = {}
    for k in INT_KEYS + ("delay", "serving_cell", "dl_newest", "dl_queue_len"):
        if k in out:
            v = _np(out[k])[envs]
            res["out." + k] = np.nan_to_num(v, nan=-7.0) if k == "delay" else v
    for lk in ("ul", "dl"):
        if f"{lk}.sent" not in state:
            continue
        valid = _np(state[f"{lk}.q.cap"])[envs] >= 0
        for k in STATE_KEYS:
            key = f"{lk}.{k}"
            if key not in state or (lk == "dl" and k in ("bsr", "sr_t")):
                continue
            v = _np(state[key])[envs]
            if k.startswith("q.") and k != "q.enq":
                v = np.where(valid, v, 0)
            res[key] = v
    for k in ASSOC_KEYS:
        if k in state:
            res[k] = _np(state[k])[envs]
    return res


def diverged(a, b, E):
    """bool [E]: envs whose views differ (views over the same E envs)."""
    d = np.zeros(E, bool)
    for k, v in a.items():
        if k in b:
            d |= ~(v.reshape(E, -1) == b[k].reshape(E, -1)).all(-1)
    return d


def snapshot(ora):
    """A copy of the oracle's state (the PHY tables and the config are shared, not copied)."""
    import copy
    memo = {id(ora.cfg): ora.cfg}
    for lk in ora.links():
        memo[id(lk.phy)] = lk.phy
    return copy.deepcopy(ora, memo)


def _margins(site, a, b, bound):
    """Normalized distance |a - b| / (rounding scale) of every element of one decision record of one env."""
    a = a.double().numpy()
    b = b.double().numpy()
    bnd = 0.0
    if bound is not None:
        bd = np.asarray(bound, dtype=np.float64)
        bnd = bd.reshape(bd.shape + (1,) * (a.ndim - 1)) if a.ndim >= 1 and a.shape[0] == bd.shape[0] \
            else float(bd.max(initial=0.0))
    with np.errstate(invalid="ignore"):
        d = np.abs(a - b)
        if site in PROB_SITES:
            sc = np.maximum(np.maximum(np.abs(a), np.abs(b)), 1e-7) * (1e-4 + 10.0 * bnd)
        elif site == "phr":
            sc = np.maximum(np.abs(a), 1.0) * (1e-5 + 0.25 * bnd)
        else:
            sc = 1e-5 * np.maximum(np.maximum(np.abs(a), np.abs(b)), 1.0) + bnd
        m = d / sc
    return np.where(np.isfinite(m), m, np.inf)


def prove_flip(snap, call, e, want, bound=None, limit=1.0, n_try=24):
    """Whether env e's integer results of one step (want: int_view of env e) are the oracle's with exactly one of its
    float threshold decisions flipped, that decision lying within rounding of its threshold.

    The step is replayed on copies of the oracle's pre-step snapshot: first recording every decision, then with each of
    env e's decisions nearest to their thresholds (normalized margin <= limit, nearest first) flipped in turn. Returns
    (site, margin, a, b) of the flipped decision whose replay equals `want`, or None."""
    o = snapshot(snap)
    o.dec.record = True
    o.dec.force = {}
    call(o)
    cands = []
    for site, k, a, b in o.dec.rec:
        if a.dim() == 0 or a.shape[0] <= e:
            continue
        m = _margins(site, a[e], b[e], None if bound is None else bound[e])
        for idx in np.argwhere(m <= max(limit, 1e3)):
            idx = tuple(int(i) for i in idx)
            cands.append((float(m[idx]), site, k, idx, float(a[e][idx]), float(b[e][idx]), a.shape))
    cands.sort(key=lambda c: c[0])
    for m, site, k, idx, av, bv, shape in cands[:n_try]:
        if m > limit:
            break
        if _replays(snap, call, e, want, site, k, idx, shape):
            return (site, m, av, bv)
    # not proven: for the report, the nearest decisions beyond the limit and whether flipping one reproduces env e
    LAST_TRIED[:] = [(site, round(m, 3), _replays(snap, call, e, want, site, k, idx, shape))
                     for m, site, k, idx, av, bv, shape in cands[:6]]
    return None


LAST_TRIED = []


def _replays(snap, call, e, want, site, k, idx, shape):
    o = snapshot(snap)
    o.dec.record = False
    f = torch.zeros(shape, dtype=torch.bool)
    f[(e,) + idx] = True
    o.dec.force = {(site, k): f}
    out = call(o)
    return not diverged(int_view(out, o.state(), [e]), want, 1).any()


class FlipCounter:
    """Free-running comparison per env of the integer outputs and integer state (and exact delays).

    An env whose integer results first differ at a step is checked (with the oracle given): it is a float-threshold
    flip when replaying the step on the oracle with one decision flipped, a decision within rounding of its threshold
    (prove_flip), gives exactly the GPU's results for that env; otherwise it is unexplained (a test failure). Either
    way the env is left out of later comparisons. Usage per step: before() right before the oracle's step, then step()
    with the same call applied to the oracle (call(oracle) -> outputs)."""

    def __init__(self, E, ora=None, limit=1.0):
        self.limit = limit
        self.alive = np.ones(E, bool)
        self.E = E
        self.ora = ora
        self.snap = None
        self.flips = []            # (step, env, (site, margin, value, threshold))
        self.unexplained = []      # (step, env)
        self.float_bad = []

    def before(self):
        if self.ora is not None:
            self.snap = snapshot(self.ora)

    def step(self, s, gpu, ora, sinr_tol=None, gpu_state=None, call=None, dec_bound=None):
        """dec_bound: per-robot bound [E,R] (dB) on the inputs of the threshold decisions (default sinr_tol)."""
        E = self.E
        envs = np.arange(E)
        gv = int_view(gpu, gpu_state or {}, envs)
        ov = int_view(ora, self.ora.state() if (self.ora is not None and gpu_state) else {}, envs)
        diff = diverged(gv, ov, E)
        new = diff & self.alive
        for e in np.nonzero(new)[0]:
            proof = None
            if self.snap is not None and call is not None and gpu_state:
                want = {k: v[[e]] for k, v in gv.items()}
                proof = prove_flip(self.snap, call, int(e), want, sinr_tol if dec_bound is None else dec_bound,
                                   self.limit)
            if proof is None:
                keys = [k for k, v in gv.items() if k in ov and not np.array_equal(v[e], ov[k][e])]
                self.unexplained.append((s, int(e), keys[:6], list(LAST_TRIED)))
                LAST_TRIED.clear()
            else:
                self.flips.append((s, int(e), proof))
        self.alive &= ~diff
        if sinr_tol is not None:
            dev = np.abs(_np(gpu["sinr_db"]).astype(np.float64) - _np(ora["sinr_db"]).astype(np.float64))
            if (dev > sinr_tol)[self.alive].any():
                self.float_bad.append((s, "sinr_db", float(dev.max())))
        return new.sum()

    def ok(self, robot_steps=0):
        """No unexplained divergence, no float out of bound, and proven flips at most 1 per 10^4 robot-steps (the
        rounding of a few transcendental functions cannot flip more often)."""
        return not self.unexplained and not self.float_bad and len(self.flips) <= max(1, robot_steps // 10000)

    def report(self):
        return f"flips {self.flips}, unexplained {self.unexplained}, float issues {self.float_bad}"

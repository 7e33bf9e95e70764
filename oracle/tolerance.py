"""Comparison rules between the HIP engine and the oracle / reference vectors. Test infrastructure only.

Integer state and integer outputs must be bit-exact. Float outputs carry the rounding of the reference formulas:
  * sinr_db (the pose -> SINR link budget): the shadowing term sigma * amp * sum_k cos(k . x + phi) is evaluated in
    float32 with |k . x| up to ~1e4 rad, so one ulp of a wave vector k (the reference's CPU cos / sin differ by an ulp
    between machines) moves the phase by |x| ulp(k). The bound per robot is
        1e-5 max(|sinr|, 1) + 4 ulp(128 dB) + 2 sigma amp sum_k (|x| ulp(|kx|) + |y| ulp(|ky|) + ulp(|arg_k|)).
  * other floats: see the callers (1e-5 relative with a unit floor for dB quantities).
A free-running comparison counts the envs whose integer outputs first differ at a step (a float-threshold flip: a
decision whose inputs differ by rounding) and compares only the envs that never diverged afterwards.
"""
from __future__ import annotations

import numpy as np

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


class FlipCounter:
    """Free-running comparison of integer outputs per env; diverged envs are counted and then left out."""

    def __init__(self, E):
        self.alive = np.ones(E, bool)
        self.flips = []            # (step, env)
        self.float_bad = []

    def step(self, s, gpu, ora, sinr_tol=None):
        E = self.alive.shape[0]
        diff = np.zeros(E, bool)
        for k in INT_KEYS:
            a = gpu[k].detach().cpu().numpy().reshape(E, -1)
            b = ora[k].detach().cpu().numpy().reshape(E, -1)
            diff |= ~(a == b).all(-1)
        new = diff & self.alive
        for e in np.nonzero(new)[0]:
            self.flips.append((s, int(e)))
        self.alive &= ~diff
        d = np.nan_to_num(gpu["delay"].detach().cpu().numpy(), nan=-7.0) != \
            np.nan_to_num(ora["delay"].detach().cpu().numpy(), nan=-7.0)
        if d.reshape(E, -1)[self.alive].any():
            self.float_bad.append((s, "delay"))
        if sinr_tol is not None:
            dev = np.abs(gpu["sinr_db"].detach().cpu().numpy().astype(np.float64) -
                         ora["sinr_db"].detach().cpu().numpy().astype(np.float64))
            if (dev > sinr_tol)[self.alive].any():
                self.float_bad.append((s, "sinr_db", float(dev.max())))
        return new.sum()

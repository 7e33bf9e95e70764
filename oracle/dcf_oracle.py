"""CPU oracle of level WIFI_DCF (per-slot CSMA/CA with integer backoff counters).  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker (or as the timed CPU baseline). The product (isaac-net_amd/) never imports it.

The reference has no engine for slot-level DCF: its only integer-backoff model is the CPU event simulator
isaac_net/core/wifi/eventsim.py:56-186 (numpy PCG64 draws, validation only). Level WIFI_DCF is this build's own
engine of those semantics behind the WifiNet / LevelNet API (wifi/engine.py:100-225, levels/base.py:43-360); this
module restates it on the CPU, element for element, so the GPU kernel can be checked bit for bit. The semantics,
per env and control step [t, t + 1) of T = control_step_ms (integer nanoseconds, relative to the step start):

  stations   the R robots at one AP, all sensing each other (one collision domain), with the EDCA parameters of
             WifiConfig.access_category: W0 = CWmin + 1, Wmax = CWmax + 1, AIFSN; each has a backoff counter b and a
             retry stage (eventsim.py:62-67).
  contention the stations with queued bytes and a usable MCS contend. The next transmission slot is
             K = min over them of AIFSN_i + b_i, at t_tx = t_idle + SIFS + K slot (t_idle: end of the last busy
             period); the stations with AIFSN_i + b_i = K transmit, and every station's counter drops by the idle
             slots it counted, b_i -= max(0, K - AIFSN_i) (eventsim.py:101-139).
  outcome    one transmitter: success unless the residual-FER draw fails; the medium is busy for
             busy_succ(B) = [RTS + SIFS + CTS + SIFS] + PPDU(B) + SIFS + ACK. Two or more: a collision, busy for the
             longest busy_coll(B_i) = PPDU(B) (basic, "difs"), PPDU(B) + SIFS + ACK ("ack") or RTS + SIFS + CTS
             (eventsim.py:140-152). An access carries B = min(queued bytes, cap) application bytes (cap = floor of
             AccessTiming.cap_bytes); PPDU(B) = preamble + T_sym ceil((22 + 8 B + 8 o ceil(B / P)) / N_DBPS) with
             the per-MSDU overhead o and payload P and the integer data bits per symbol N_DBPS.
  backoff    after a success the station serves B bytes FIFO, returns to stage 0 and draws b ~ U{0..W0-1}; after a
             failure its stage rises and it draws b ~ U{0..min(W0 2^stage, Wmax) - 1}; at max_tx attempts the
             access's bytes are dropped, the messages they touch are lost (discarded whole, their remaining bytes
             too) and the stage returns to 0 (eventsim.py:156-179).
  arrivals   messages arrive at the step start (submit); queued sizes count in whole bytes (rounded up). A
             station that was not contending at the end of the last step (empty queue or no usable MCS) and now
             is, whose counter has already run out, transmits at the next slot boundary if the medium has been idle
             for its AIFS, else it draws a counter first (eventsim.py:113-123).
  step end   an exchange starts only if it ends within the step; otherwise the medium stays idle and the countdown
             carries into the next step (t_idle -= T). When nobody is left contending, the idle anchor is re-based
             to AIFS slots before the step end and the extra idle slots m are counted off every counter
             (b = max(0, b - m)): every later transmission time and counter is unchanged by it, and the integers stay
             bounded over any number of idle steps. Messages finish at the end of the exchange that carried their
             last byte: fin = t + t_end / T (double, then float32).
Draws come from the engine's counter RNG (proto/rng.py keys): channel STEP, stream 2 element (n_event R + r) for
the counters drawn after an exchange, stream 3 element r for the counters of arriving stations, stream 4 element
n_event for the FER draw; reset draws channel RESET stream 5 element r for the initial counters. A draw from
U{0..W-1} is ((h >> 8) W) >> 24 of the element hash h.

Outputs: the LevelNet dict (delivered, timed_out, cap, cls, delay, newest, det_env, queue_len, queue_bytes, sinr_db,
t) plus serving_cell, wifi_mcs, wifi_rate_mbps, wifi_access_ms (mean over the step's successes of the time from the
station's previous exchange end, or the step start, to the success end; NaN without success), wifi_p_fail (failed
attempts / attempts in the step; NaN without attempts), wifi_busy (busy share of the step, per env).

Parity status: the GPU kernel is checked against this module bit for bit (tests/test_gpu_dcf.py); this module's
contention statistics are checked against Bianchi's saturation model and against the validation figures of the
reference's event simulator (tests/test_dcf_oracle.py). Being this build's own model, its per-draw behaviour has no
reference vector: "parity unpinned" against the reference beyond those statistics.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from .nr_oracle import M32, STEP, SUBMIT, CounterRNG, Radio, base_key, elem_hash, mix32, salt
from .wifi_oracle import INF, WifiOracle

RESET = 3
S_POST, S_ARRIVE, S_FER, S_INIT = 2, 3, 4, 5


def _elem(base, i):
    return mix32(mix32((base + (i * 0x9E3779B9)) & M32) ^ base)


def _key(s0, env, ep, channel, ctr, stream):
    h = mix32(s0 ^ salt(env & M32))
    h = mix32(h ^ salt(ep & M32))
    h = mix32(h ^ salt(channel))
    h = mix32(h ^ salt(ctr & M32))
    return mix32(h ^ salt(stream))


def draw_int(h, W):
    """U{0..W-1} from a 32-bit hash: ((h >> 8) W) >> 24."""
    return ((h >> 8) * W) >> 24


def dcf_constants(cfg, wc):
    """Integer-nanosecond timing and the per-MCS data bits per symbol of the DCF level."""
    from isaac_net_amd.wifi_config import (AC_NAMES, ACK_BYTES, BLOCK_ACK_BYTES, CTS_BYTES, DATA_SUBCARRIERS, EDCA,
                                           MODULATION, NON_HT_RATES, RTS_BYTES, mcs_numbers, preamble_us, symbol_us)
    ns = lambda us: int(round(us * 1000.0))  # noqa: E731
    ids = mcs_numbers(wc.standard, wc.bandwidth_mhz, wc.n_ss)
    if wc.standard == "a":
        ndbps = [int(r * 4) for r in NON_HT_RATES]
    else:
        nsd = DATA_SUBCARRIERS[wc.standard][wc.bandwidth_mhz]
        ndbps = []
        for m in ids:
            bits, code = MODULATION[m]
            v = nsd * bits * code * wc.n_ss
            assert abs(v - round(v)) < 1e-9
            ndbps.append(int(round(v)))

    def ctrl_ns(nbytes):
        return ns(20.0 + 4.0 * math.ceil((22 + 8 * nbytes) / (wc.ctrl_rate_mbps * 4.0)))
    agg = wc.max_ampdu_bytes > 0
    cw = EDCA[wc.access_category]
    T = cfg.control_step_ms * 1e6
    assert abs(T - round(T)) < 1e-6
    return dict(ndbps=ndbps, tsym=ns(symbol_us(wc.standard, wc.gi_us)), pre=ns(preamble_us(wc.standard, wc.n_ss)),
                sifs=ns(wc.sifs_us), slot=ns(wc.slot_us), t_ack=ctrl_ns(BLOCK_ACK_BYTES if agg else ACK_BYTES),
                t_rts=ctrl_ns(RTS_BYTES), t_cts=ctrl_ns(CTS_BYTES), W0=cw[0] + 1, Wmax=cw[1] + 1, aifsn=int(cw[2]),
                T=int(round(T)), ovh=int(wc.msdu_overhead_bytes), payload=int(wc.msdu_payload_bytes),
                ac=AC_NAMES.index(wc.access_category))


class DcfOracle(WifiOracle):
    """WIFI_DCF on the CPU: the WifiOracle FIFO, radio and outputs with the event loop above as _serve."""

    rebase = True       # False: keep the unbounded idle anchor (Python integers), to show the re-base changes nothing

    def __init__(self, E, R, cfg, seed=0):
        from isaac_net_amd.wifi_config import WifiConfig
        wc = cfg.wifi if cfg.wifi is not None else WifiConfig()
        assert wc.bg_stations == 0 and wc.class_ac is None, "one access category, no background stations"
        self.k = None
        super().__init__(E, R, cfg, seed)
        self.k = dcf_constants(cfg, wc)
        self.b = np.zeros((E, R), np.int64)
        self.stage = np.zeros((E, R), np.int64)
        self.had = np.zeros((E, R), bool)
        self.t_idle = np.zeros(E, np.int64)
        self.tot = {"att": np.zeros(E, np.int64), "fail": np.zeros(E, np.int64), "succ": np.zeros(E, np.int64),
                    "busy_ns": np.zeros(E, np.int64)}       # statistics since construction (tests)
        self._reset_dcf(np.ones(E, bool))

    def reset(self, env_ids=None):
        super().reset(env_ids)
        if getattr(self, "k", None) is None:
            return
        m = np.ones(self.E, bool)
        if env_ids is not None:
            m = np.zeros(self.E, bool)
            m[np.asarray(env_ids, dtype=np.int64)] = True
        self._reset_dcf(m)

    def _reset_dcf(self, m):
        k = self.k
        for e in np.nonzero(m)[0]:
            base = _key(self.rng.s0, int(self.rng.env[e]), int(self.rng.episode[e]), RESET, 0, S_INIT)
            for r in range(self.R):
                self.b[e, r] = draw_int(_elem(base, r), k["W0"])
        self.stage[m] = 0
        self.had[m] = False
        self.t_idle[m] = 0

    # ------------------------------------------------------------------ integer timing
    def cap_int(self, rate):
        """floor(AccessTiming.cap_bytes) of the float32 cap, per station [E,R] int64."""
        d = self.d
        txop = torch.full_like(rate, float(self.ac_txop[self.k["ac"]]))
        return torch.floor(self._cap_bytes(rate, txop)).to(torch.int64).numpy()

    def ppdu_ns(self, B, ndbps):
        k = self.k
        bits = 22 + 8 * B + 8 * k["ovh"] * ((B + k["payload"] - 1) // k["payload"])
        return k["pre"] + k["tsym"] * ((bits + ndbps - 1) // ndbps)

    def busy(self, B, ndbps):
        """(busy_succ, busy_coll) in ns of an access of B bytes."""
        k, wc = self.k, self.wc
        tdata = self.ppdu_ns(B, ndbps)
        if wc.rts_cts:
            hs = k["t_rts"] + k["sifs"] + k["t_cts"] + k["sifs"]
            return hs + tdata + k["sifs"] + k["t_ack"], k["t_rts"] + k["sifs"] + k["t_cts"]
        succ = tdata + k["sifs"] + k["t_ack"]
        return succ, (succ if wc.collision_time == "ack" else tdata)

    # ------------------------------------------------------------------ the control step
    def _serve(self, t, snr):
        wc, k, E, R, F = self.wc, self.k, self.E, self.R, self.F
        nm = (snr[..., None] >= self.thr).sum(-1)
        link = (nm > 0).numpy()
        mcs = (nm - 1).clamp(min=0)
        rate = self.rates[mcs]
        cap = self.cap_int(rate)
        ndbps = np.array(k["ndbps"], np.int64)[mcs.numpy()]
        rem = np.ceil(self.rem.numpy()).astype(np.int64)        # whole bytes
        fin = np.full((E, R, F), np.inf)
        acc_sum = np.zeros((E, R)); n_succ = np.zeros((E, R), np.int64)
        n_att = np.zeros((E, R), np.int64); n_fail = np.zeros((E, R), np.int64)
        busy_tot = np.zeros(E, np.int64)
        T, slot, sifs, aif = k["T"], k["slot"], k["sifs"], k["aifsn"]
        W0, Wmax, L = k["W0"], k["Wmax"], wc.max_tx
        fer_thr = np.float32(wc.frame_error_rate)
        for e in range(E):
            env, ep, ctr = int(self.rng.env[e]), int(self.rng.episode[e]), int(self.rng.ctr[STEP][e])
            kpost = _key(self.rng.s0, env, ep, STEP, ctr, S_POST)
            karr = _key(self.rng.s0, env, ep, STEP, ctr, S_ARRIVE)
            kfer = _key(self.rng.s0, env, ep, STEP, ctr, S_FER)
            b, stage, ti = self.b[e], self.stage[e], int(self.t_idle[e])
            q = rem[e].sum(-1)
            # arrivals at the step start to stations that were not contending
            for r in range(R):
                if q[r] > 0 and link[e, r] and not self.had[e, r]:
                    el = -ti - sifs
                    ka = el // slot if el >= 0 else -1
                    if max(0, b[r] - max(0, ka - aif)) == 0:
                        b[r] = ka + 1 - aif if ka >= aif else draw_int(_elem(karr, r), W0)
            prev_end = np.zeros(R, np.int64)
            n_ev = 0
            idle_end = False
            while True:
                q = rem[e].sum(-1)
                cand = (q > 0) & link[e]
                if not cand.any():
                    idle_end = True
                    break
                Kc = int((aif + b)[cand].min())
                t_tx = ti + sifs + Kc * slot
                tx = cand & ((aif + b) == Kc)
                Bv = np.minimum(q, cap[e])
                n_tx = int(tx.sum())
                if n_tx == 1:
                    r0 = int(np.nonzero(tx)[0][0])
                    dur = self.busy(int(Bv[r0]), int(ndbps[e, r0]))[0]
                else:
                    dur = max(self.busy(int(Bv[r]), int(ndbps[e, r]))[1] for r in np.nonzero(tx)[0])
                t_end = t_tx + dur
                if t_end > T:
                    break
                b -= np.maximum(0, Kc - aif)
                np.maximum(b, 0, out=b)
                ok = False
                if n_tx == 1:
                    u = np.float32((_elem(kfer, n_ev) >> 8) * (1.0 / 16777216.0))
                    ok = not (u < fer_thr)
                busy_tot[e] += dur
                for r in np.nonzero(tx)[0]:
                    n_att[e, r] += 1
                    if ok:
                        self._consume(e, r, int(Bv[r]), rem, fin, t, t_end, lost=False)
                        acc_sum[e, r] += (t_end - prev_end[r]) * 1e-6
                        n_succ[e, r] += 1
                        stage[r] = 0
                        W = W0
                    else:
                        n_fail[e, r] += 1
                        stage[r] += 1
                        if stage[r] >= L:
                            self._consume(e, r, int(Bv[r]), rem, fin, t, t_end, lost=True)
                            stage[r] = 0
                        W = min(W0 << int(stage[r]), Wmax)
                    b[r] = draw_int(_elem(kpost, n_ev * R + int(r)), W)
                    prev_end[r] = t_end
                ti = t_end
                n_ev += 1
            ti -= T
            if self.rebase and idle_end and -ti - sifs >= 0:
                # nobody contends: re-base the idle anchor to AIFS slots before the step end, counting the
                # extra idle slots off every counter (exact: same transmission times and counters afterwards)
                m = (-ti - sifs) // slot - aif
                if m > 0:
                    ti += m * slot
                    np.maximum(b - m, 0, out=b)
            self.t_idle[e] = ti
            self.had[e] = (rem[e].sum(-1) > 0) & link[e]
            self.tot["att"][e] += n_att[e].sum()
            self.tot["fail"][e] += n_fail[e].sum()
            self.tot["succ"][e] += n_succ[e].sum()
            self.tot["busy_ns"][e] += busy_tot[e]
        self.rem = torch.from_numpy(rem.astype(np.float32))
        fin_t = torch.from_numpy(fin.astype(np.float32))
        nan = float("nan")
        self.o_access = torch.from_numpy(np.where(n_succ > 0, acc_sum / np.maximum(n_succ, 1), nan).astype(np.float32))
        self.o_pfail = torch.from_numpy(np.where(n_att > 0, n_fail / np.maximum(n_att, 1), nan).astype(np.float32))
        self.o_busy = torch.from_numpy(np.repeat((busy_tot / T)[:, None], R, 1).astype(np.float32))
        self.o_mcs = torch.where(torch.from_numpy(link), self.mcs_ids[mcs], torch.full_like(mcs, -1))
        self.o_rate = torch.where(torch.from_numpy(link), rate, torch.zeros_like(rate))
        return fin_t

    def _consume(self, e, r, B, rem, fin, t, t_end, lost):
        """Serve (lost=False) or drop (lost=True) B bytes from the head of station r's FIFO. Served messages whose
        last byte leaves finish at t_end; a message with a dropped byte is discarded whole (never finishes)."""
        tf = float(t[e]) + t_end / self.k["T"]
        for f in range(self.F):
            if B <= 0:
                break
            if rem[e, r, f] <= 0:
                continue
            take = min(B, int(rem[e, r, f]))
            B -= take
            if lost:
                rem[e, r, f] = 0
            else:
                rem[e, r, f] -= take
                if rem[e, r, f] == 0:
                    fin[e, r, f] = tf

    def state(self):
        sd = super().state()
        sd["dcf.b"] = torch.from_numpy(self.b.copy())
        sd["dcf.stage"] = torch.from_numpy(self.stage.copy())
        sd["dcf.had"] = torch.from_numpy(self.had.copy())
        sd["dcf.t_idle"] = torch.from_numpy(self.t_idle.copy())
        return sd

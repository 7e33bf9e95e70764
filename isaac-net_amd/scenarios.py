"""Synthetic workloads of the NR uplink engine: the configurations it is benchmarked and tested on, as NRConfig
objects, and their per-step inputs (robot poses and message arrivals).

Mapping to NRConfig (TDD "DDDSU" at mu = 1: one UL data slot and one SR opportunity per 2.5 ms, so K UL slots per
control step need control_step_ms = 2.5 K; "52 PRBs" needs n_prb = 52 since the 38.101 value at 30 kHz is 51):
  plumbing    64 envs x 8 robots, K = 4, round robin, 4 HARQ x 4 transmissions, 1500 B at Poisson 0.5, FIFO 16,
              UMi LOS around a gNB at the centre of a 100 m square, i.i.d. Rayleigh block fading per slot.
  rl_scale    4096 envs x 32 robots, K = 10, PF with EWMA 0.01, 8 HARQ x 5 transmissions, Rician K = 3 dB, 200 B at
              Poisson 0.8 + 4000 B at Poisson 0.1, FIFO 32, random walk at 1 m/s in a 200 m square, UMi LOS.
  wifi_dcf    level WIFI: 2048 envs x 16 stations at one AP, legacy DCF parameters (CWmin 15, CWmax 1023, binary
              exponential backoff over 7 attempts), 802.11ax 20 MHz with its 12-entry MCS table, 20 sub-steps of 1 ms
              per control step, 1500 B at Poisson 0.4, FIFO 16, stations uniform in a 50 m disc around the AP with a
              1 m/s random walk kept inside the disc, log-distance path loss with plane-wave shadowing.
  wifi_dcf_slots  the same inputs on level WIFI_DCF (per-slot CSMA/CA with integer backoff counters).
  rl_scale_dl  rl_scale with the downlink on (dl=True: 40 DL data slots and 5 CQI reports per step) and 2000 B DL
              messages at Poisson 0.5 per robot-step (at most 2).
  mc_interf   1024 envs x 64 robots, 3 cells on a hexagonal grid 150 m apart (centroid at the centre of a 200 m square),
              max-RSRP association without handover (a3_offset_db = inf), thermal noise with the same-slot UL
              interference of the other cells' scheduled robots, open-loop fractional power control (on by default
              with several cells), PF over 106 PRBs (14 RBGs), K = 10, 1200 B at Poisson 0.3, UMi LOS, correlated
              Rayleigh fading on every robot-cell link, 1 m/s random walk in the square.
  freq_sel    16384 envs x 128 robots (two wavefronts per env), one cell, 273 PRBs (100 MHz at 30 kHz) in 8 RBGs of
              35 PRBs, i.i.d. Rayleigh fading per subband and slot, PF, K = 20 (DDDSU at 50 ms), 8 HARQ x 4
              transmissions, 800 B at Poisson 0.2, FIFO 16, UMi LOS around the centre of a 200 m square.
Inputs come from numpy's PCG64 seeded by the workload seed (poses uniform at the start, then a random walk clamped to
the square or disc; arrival counts per class), identical for the GPU engine and the CPU oracle.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from .config import NRConfig


def plumbing_config(**kw):
    base = dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="rr", n_harq=4, max_harq_tx=4,
                frame_buffer=16, msg_sizes=(1500.0,), fading_rho_per_ms=0.0, channel="tr38901",
                tr38901_scenario="UMi", tr38901_los="los", cell_positions_m=((50.0, 50.0),), gnb_height_m=10.0,
                seed=0)
    base.update(kw)
    return NRConfig(**base)


def rl_scale_config(**kw):
    base = dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=25.0, scheduler="pf", pf_window=100.0,
                n_harq=8, max_harq_tx=5, frame_buffer=32, msg_sizes=(200.0, 4000.0), fading_rho_per_ms=0.0,
                fading_rician=True, rician_k_db=3.0, channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0, seed=0)
    base.update(kw)
    return NRConfig(**base)


def mc_interf_config(**kw):
    base = dict(mu=1, n_prb=106, tdd_pattern="DDDSU", control_step_ms=25.0, scheduler="pf", pf_window=100.0,
                n_harq=8, max_harq_tx=5, frame_buffer=16, msg_sizes=(1200.0,), n_cells=3, cell_layout="hex",
                cell_isd_m=150.0, cell_center_m=(100.0, 100.0), noise_model="thermal", a3_offset_db=float("inf"),
                channel="tr38901", tr38901_scenario="UMi", tr38901_los="los", gnb_height_m=10.0, seed=0)
    base.update(kw)
    return NRConfig(**base)


def freq_sel_config(**kw):
    base = dict(mu=1, n_prb=273, rbg_size=35, tdd_pattern="DDDSU", control_step_ms=50.0, scheduler="pf",
                pf_window=100.0, n_harq=8, max_harq_tx=4, frame_buffer=16, msg_sizes=(800.0,), fading_rho_per_ms=0.0,
                channel="tr38901", tr38901_scenario="UMi", tr38901_los="los", cell_positions_m=((100.0, 100.0),),
                gnb_height_m=10.0, seed=0)
    base.update(kw)
    return NRConfig(**base)


def wifi_dcf_config(**kw):
    from .wifi_config import WifiConfig
    base = dict(control_step_ms=20.0, frame_buffer=16, msg_sizes=(1500.0,), cell_positions_m=((0.0, 0.0),),
                wifi=WifiConfig(access_category="DCF", standard="ax", bandwidth_mhz=20), seed=0)
    base.update(kw)
    return NRConfig(**base)


WORKLOADS = {
    "plumbing": dict(cfg=plumbing_config, E=64, R=8, arena=100.0, speed=0.0, rates=(0.5,), steps=1000),
    "rl_scale": dict(cfg=rl_scale_config, E=4096, R=32, arena=200.0, speed=1.0, rates=(0.8, 0.1), steps=500),
    "rl_scale_dl": dict(cfg=lambda **kw: rl_scale_config(dl=True, **kw), E=4096, R=32, arena=200.0, speed=1.0,
                        rates=(0.8, 0.1), steps=500, dl_rates=(0.5,), dl_size=2000.0),
    "mc_interf": dict(cfg=mc_interf_config, E=1024, R=64, arena=200.0, speed=1.0, rates=(0.3,), steps=300),
    "freq_sel": dict(cfg=freq_sel_config, E=16384, R=128, arena=200.0, speed=1.0, rates=(0.2,), steps=100),
    "wifi_dcf": dict(cfg=wifi_dcf_config, E=2048, R=16, radius=50.0, speed=1.0, rates=(0.4,), steps=500,
                     level="WIFI"),
    "wifi_dcf_slots": dict(cfg=wifi_dcf_config, E=2048, R=16, radius=50.0, speed=1.0, rates=(0.4,), steps=500,
                           level="WIFI_DCF"),
}


class Workload:
    """Per-step inputs of a workload: poses [steps, E, R, 2] float32 and arrival counts [steps, E, R, NC] uint8,
    generated on the host and moved to `device` (resident before any timed region)."""

    def __init__(self, E, R, steps, seed=0, device="cpu", name="rl_scale"):
        w = WORKLOADS[name]
        self.cfg = w["cfg"]()
        self.level = w.get("level", "L2")
        rs = np.random.default_rng(seed)
        step_m = w["speed"] * self.cfg.control_step_ms * 1e-3
        poses = np.empty((steps, E, R, 2), np.float32)
        if "radius" in w:                                   # uniform in a disc around the AP at the origin
            rad = w["radius"]
            r0, a0 = rad * np.sqrt(rs.uniform(size=(E, R))), rs.uniform(0.0, 2 * math.pi, size=(E, R))
            p = np.stack([r0 * np.cos(a0), r0 * np.sin(a0)], -1)
        else:
            a = w["arena"]
            p = rs.uniform(0.0, a, size=(E, R, 2))
        for s in range(steps):
            poses[s] = p
            ang = rs.uniform(0.0, 2 * math.pi, size=(E, R))
            p = p + step_m * np.stack([np.cos(ang), np.sin(ang)], -1)
            if "radius" in w:
                n = np.linalg.norm(p, axis=-1, keepdims=True)
                p = np.where(n > rad, p * (rad / np.maximum(n, 1e-9)), p)
            else:
                p = np.clip(p, 0.0, a)
        counts = np.stack([rs.poisson(lam, size=(steps, E, R)) for lam in w["rates"]], -1)
        self.poses = torch.from_numpy(poses).to(device)
        self.counts = torch.from_numpy(np.minimum(counts, 255).astype(np.uint8)).to(device)
        self.dl_bytes = None
        if "dl_rates" in w:
            # DL messages per robot-step (Poisson, at most 2): the bytes of the add_dl_frames calls of each step
            n = np.minimum(rs.poisson(w["dl_rates"][0], size=(steps, E, R)), 2)
            self.dl_bytes = torch.from_numpy(np.stack([np.where(n > i, w["dl_size"], 0.0) for i in range(2)], 1)
                                             .astype(np.float32)).to(device)             # [steps, 2, E, R]
        self.E, self.R, self.steps = E, R, steps

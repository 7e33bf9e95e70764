"""make_engine / HipNREngine: the contract API of isaac-net's NR engine over the HIP kernels of libinet_nr.so.

Mirrors isaac_net/core/engine.py (make_engine :230-316, NREngine :319-960) for level "L2" with backend="hip":
reset(env_ids) / submit(t, requests) / step(t, poses_or_snr) -> dict / clock / output_schema / counters, with the same
inputs, output keys, dtypes and shapes, the same per-env clock rules (t=None uses the engine clock; an explicit t must
equal it) and the same error behaviour for inputs the engine cannot take. What the kernels do not implement is refused
at construction with HipUnsupported (a NotImplementedError and a ValueError, like the reference's TritonUnsupported,
nr_fast.py:104-111, 538-563).

All per-env state lives in device tensors that torch allocates; every call hands the library plain pointers. The host
keeps only the control-step counter T, the per-env epoch used by `clock`, and the slot of the last fading update.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib
from .channels import (RICIAN_K_DB, delay_spread_grid, lg_ds_params, scenario_name, subband_fading_sqrt,
                       sum_of_cosines_cdf_table)
from .config import NRConfig
from .phy import PhyTables, cqi_tables

BIG_SLOT = 0x7FFFFFFF
FADING, BLER_UL, BLER_DL = 1, 2, 3
NCTR = 13
CTR_NAMES = ("tb_new", "tb_retx", "tb_ok", "tb_fail", "exhaust", "bytes_ok", "bytes_new", "lost_frames",
             "new_while_pending", "prb_used")
# the 5G-LENA grant accounting (mac.py:119-122), counters 10..12, reported when a LENA MAC switch is on
LENA_CTR_NAMES = ("tb_bytes", "tb_empty", "retx_block")


class HipUnsupported(NotImplementedError, ValueError):
    """A config feature the HIP backend does not implement (refused before anything is built)."""


@dataclass
class Requests:
    """Messages each robot enqueues in one control step (isaac_net/core/proto/netsim.py:163-172).
    send [E,R] long (0 = none, c >= 1 = one message of class c), det [E,R] bool, hid [E] long (optional)."""
    send: torch.Tensor
    det: Optional[torch.Tensor] = None
    hid: Optional[torch.Tensor] = None


# ---------------------------------------------------------------------------------------------- counter hash (host)
M32 = 0xFFFFFFFF


def mix32(x):
    x ^= x >> 16
    x = (x * 0x21F0AAAD) & M32
    x ^= x >> 15
    x = (x * 0x735A2D97) & M32
    return x ^ (x >> 15)


def salt(v):
    return (mix32(v & M32) + 0x9E3779B9) & M32


def seed_key(seed):
    return mix32(mix32(seed & M32) ^ salt((seed >> 32) & M32))


# RBG counts of the one-cell step builds (nr_step_s*.hip): 8 (273 PRB in RBGs of 35) and the RBG-configuration-1 counts
# of the standard carriers at 30 kHz
ONE_CELL_RBGS = (8, 10, 11, 12, 13, 14, 16, 17, 18)


def refusals(cfg: NRConfig):
    """[(feature, why)] of the config's features the HIP step kernel does not implement (empty: it runs)."""
    out = []

    def no(cond, what, why):
        if cond:
            out.append((what, why))
    mc = cfg.n_cells > 1
    no(mc and cfg.n_cells > 7, f"n_cells={cfg.n_cells}", "one to seven cells per env (the reference's 1..7)")
    no(mc and cfg.dl, "the downlink with several cells", "the multi-cell step runs the uplink")
    no(mc and cfg.harq_combining == "ir_lena", "HARQ-IR (harq_combining='ir_lena') with several cells",
       "chase combining or none with several cells (IR's integer state differed from the reference's on 2 of 6 "
       "seeded 3- and 4-cell trajectories)")
    no(cfg.rlf and cfg.rach, "re-establishment through RACH (rlf with rach)", "a fixed re-establishment delay")
    no(mc and cfg.frame_buffer > 64, "frame_buffer > 64 with several cells", "a 64-bit handover loss mask")
    no(not cfg.ul, "ul=False (a downlink-only engine)", "the UL link runs every step")
    no(cfg.dl and cfg.duplex != "tdd", "the FDD downlink carrier", "TDD (one carrier)")
    no(cfg.ul_grant_model != "lumped", "ul_grant_model='bsr'", "lumped SR grants only")
    no(cfg.n_layers_max != 1, "rank-2 MIMO", "single-layer TBs")
    no(cfg.ul_mini_slot_symbols is not None, "mini-slot grants", "one scheduling occasion per slot")
    no(cfg.scheduler not in ("pf", "pf_wideband", "maxci", "rr"), f"scheduler={cfg.scheduler!r}",
       "pf, pf_wideband, maxci and rr")
    no(cfg.pf_update == "rbg" and cfg.scheduler not in ("pf", "pf_wideband"),
       "pf_update='rbg' without a PF scheduler", "the per-RBG PF update of the pf schedulers")
    no(cfg.ul_tpc, "closed-loop TPC (ul_tpc)", "open-loop fractional power control")
    no(cfg.freq_corr_mode == "los" and (cfg.channel != "tr38901" or
                                        scenario_name(cfg.tr38901_scenario) not in ("UMi", "UMa", "InH")),
       "per-link delay spreads (fading_delay_spread_ns=None) outside TR 38.901 or on RMa / InF",
       "per-link delay spreads on UMi, UMa and InH, or one fixed delay spread")
    no(cfg.traffic is not None, "traffic models (NRConfig.traffic)", "messages through submit()")
    no(cfg.rach or cfg.drx, "RACH / DRX access", "always connected")
    no(cfg.tbs_mode != "38214" or cfg.bler_source != "pdsch", "tbs_mode / bler_source", "38.214 TBS, Sionna PDSCH")
    no(cfg.rng != "engine", "rng='global'", "counter-based engine RNG")
    no(cfg.edge is not None or cfg.background is not None or cfg.energy is not None, "edge / background / energy",
       "no wrapper stages")
    no(cfg.blockage or cfg.los_source != "stochastic" or cfg.gnb_antenna != "isotropic" or cfg.o2i_indoor_frac > 0
       or cfg.shadow_white_frac > 0, "obstacle stack, sector antennas, O2I or white shadowing",
       "plain path loss + plane-wave shadowing")
    no(cfg.channel not in ("log_distance", "tr38901"), f"channel={cfg.channel!r}", "log_distance and tr38901")
    if cfg.channel == "tr38901":
        no(cfg.tr38901_los == "stochastic" and (cfg.tr38901_scenario.startswith("InF") or
                                                (cfg.tr38901_scenario == "UMa" and cfg.ue_height_m > 13.0)),
           "the stochastic LOS state of InF or of UMa above 13 m", "the stochastic LOS state of UMi, UMa and InH")
        no(cfg.los_soft, "the soft LOS state (los_soft)", "a hard LOS state")
        no(cfg.tr38901_scenario == "RMa", "the RMa scenario", "UMa, UMi, InH, InF")
        no(cfg.tr38901_scenario.startswith("InF") and cfg.tr38901_los == "nlos", "InF NLOS", "InF LOS")
    no(cfg.n_subbands not in ((8, 13, 14) if mc else ONE_CELL_RBGS), f"{cfg.n_subbands} subbands",
       f"{', '.join(map(str, ONE_CELL_RBGS))} RBGs (several cells: 8, 13 or 14) in this build")
    no(cfg.n_harq not in (2, 4, 8, 16), f"n_harq={cfg.n_harq}", "2, 4, 8 or 16 HARQ processes in this build")
    no(cfg.max_harq_tx > 16, "max_harq_tx > 16", "up to 16 transmissions")
    no(cfg.shadow_modes > 16, "shadow_modes > 16", "up to 16 plane waves")
    no(cfg.frame_buffer > 255, "frame_buffer > 255", "8-bit class field, int32 offsets")
    air = [m + (math.ceil(m / cfg.pkt_payload_bytes) * cfg.pkt_overhead_bytes if cfg.pkt_overhead_bytes else 0)
           for m in cfg.msg_sizes]
    no(max(air, default=0) > 1 << 22, "messages above 2^22 bytes", "a full queue inside the int32 byte offsets")
    no(len(cfg.msg_sizes) > 255, "more than 255 message classes", "8-bit class field")
    return out


def split_offsets(floor, sent, enq, rebase_at):
    """int64 byte offsets [E,R] -> (base [E,R] int64, rel(x) -> x - base as int32-range int64): the base is the
    floor where the floor has reached rebase_at (else 0), as the step kernel rebases; raises if the queued bytes
    (enq - floor) or the unsent ones do not fit in int32 above the base."""
    base = torch.where(floor >= rebase_at, floor, torch.zeros_like(floor)) if rebase_at > 0 else \
        torch.zeros_like(floor)
    lim = (1 << 31) - 1
    if bool(((enq - base) > lim).any()) or bool(((sent - base) < -(1 << 30)).any()) or \
            bool(((floor - base) > lim).any()):
        raise ValueError("byte offsets beyond 2^31 above the robot's floor: not representable")
    return base, (lambda x: x.long() - base)


class HipNREngine:
    """NR engine (level "L2": one cell with the uplink, and the downlink with NRConfig(dl=True); or several cells
    with the uplink, NRNet.step_cells) on MI355X. API of isaac_net.core.engine.NREngine."""

    level = "L2"
    backend = "hip"
    # the floor (bytes) from which a step moves a robot's int32 byte offsets down into its 64-bit base
    REBASE_AT = 1 << 30

    def __init__(self, E, R, device="cuda", cfg: NRConfig | None = None, seed=None, out_format="reference"):
        cfg = cfg if cfg is not None else NRConfig()
        no = refusals(cfg)
        if no:
            raise HipUnsupported("the hip backend of the NR engine does not implement "
                                 + "; ".join(f"{f} ({why})" for f, why in no))
        dev = torch.device(device)
        if dev.type != "cuda":
            raise ValueError("the hip backend needs a GPU device (cuda:N on ROCm)")
        if not 1 <= R <= 256:
            raise HipUnsupported(f"R={R}: the hip backend holds one env's robots in one 64-lane wavefront segment, "
                                 "or in two or four wavefronts (1 <= R <= 256)")
        if R > 64 and cfg.n_cells > 1:
            raise HipUnsupported(f"R={R} with several cells: envs of more than 64 robots (two or four wavefronts) run "
                                 "one cell")
        if R > 128 and cfg.dl:
            raise HipUnsupported(f"R={R} with the downlink: envs of up to 128 robots (two wavefronts) run the DL")
        self._lib = _lib.load()
        self.E, self.R, self.dev, self.config = E, R, dev, cfg
        if seed is None:
            seed = cfg.seed if cfg.seed is not None else int(torch.randint(0, 2 ** 62, ()).item())
        self.seed = int(seed)
        self.S, self.P, self.F = cfg.n_subbands, cfg.n_harq, cfg.frame_buffer
        self.C = cfg.n_cells
        self.N = cfg.slots_per_step
        self.out_format = out_format
        self.tabs = PhyTables(cfg.mcs_table, cfg.bler_target, max(cfg.max_harq_tx, 2), cfg.ul_mcs_max)
        self.dl = bool(cfg.dl)
        # the DL PHY differs from the UL's only by its MCS cap (dl_mcs_max), mac.py:97-99
        self.tabs_dl = PhyTables(cfg.mcs_table, cfg.bler_target, max(cfg.max_harq_tx, 2), cfg.dl_mcs_max) \
            if self.dl else None
        self._alloc_state()
        self._upload_tables()
        self._build_params()
        self.T = 0
        self._uniform_epoch = 0
        self.last_g = None
        self._last_hid = torch.zeros(E, dtype=torch.long, device=dev)
        self._rows = {}
        self._log_stats, self._feat, self._dl_delay = False, None, None
        self.log_cap_max = 10 ** 9       # only frames captured at or before this step (global clock) are logged
        self.clear_stats()
        self.reset(None)

    # ------------------------------------------------------------------ buffers
    def _alloc_state(self):
        E, R, S, P, F, d = self.E, self.R, self.S, self.P, self.F, self.dev
        i32, f32 = torch.int32, torch.float32
        z = lambda *shape, dt=i32, v=0: torch.full(shape, v, dtype=dt, device=d)  # noqa: E731
        cfg = self.config
        nf = 0 if cfg.channel not in ("log_distance", "tr38901") else (3 if cfg.channel == "tr38901" else 1)
        self.st = {
            "sent": z(E, R), "floor_": z(E, R), "bsr": z(E, R), "sr_t": z(E, R, v=-1), "last_tx": z(E, R, v=-1),
            "olla": z(E, R, dt=f32), "avg": z(E, R, dt=f32, v=100.0), "enq": z(E, R), "qlen": z(E, R),
            "csi": z(E, S, R, dt=f32), "h_re": z(E, self.C * S, R, dt=f32), "h_im": z(E, self.C * S, R, dt=f32),
            "h_meta": z(E, P, R), "h_lo": z(E, P, R), "h_hi": z(E, P, R), "h_ready": z(E, P, R), "h_tbs": z(E, P, R),
            "h_comb": z(E, P, R, dt=f32), "h_lexp": z(E, P, R, dt=f32, v=-math.inf), "h_nrb": z(E, P, R, dt=f32),
            "q_cap": z(E, F, R, v=-1), "q_start": z(E, F, R), "q_end": z(E, F, R), "q_fin": z(E, F, R, v=BIG_SLOT),
            "q_meta": z(E, F, R), "q_hid": z(E, F, R),
            # Rician state per robot-cell link [E][C][R]: phasor, K target, the LOS K draw (K from the LOS state),
            # its ramp start and slot; per env: waiting for the first LOS state
            "spec_re": z(E, self.C, R, dt=f32), "spec_im": z(E, self.C, R, dt=f32), "k_lin": z(E, self.C, R, dt=f32),
            "k_los": z(E, self.C, R, dt=f32), "k_from": z(E, self.C, R, dt=f32), "k_g0": z(E, self.C, R),
            "k_fresh": z(E),
            # per-link delay spreads: grid indices of every robot-cell link [E][C][R]
            "fc_idx": z(E, self.C, R), "fc_idl": z(E, self.C, R), "fc_idn": z(E, self.C, R),
            "env_id": torch.arange(E, dtype=i32, device=d), "episode": z(E, v=-1), "ctr_step": z(E),
            "ctr_submit": z(E), "epoch": z(E),
            "field": z(E, self.C, max(nf, 1), max(cfg.shadow_modes, 1), 3, dt=f32),
            "ctr": z(E, NCTR, dt=torch.int64), "hist": z(E, 3, cfg.max_harq_tx + 1, dt=torch.int64),
            "clock": z(1, dt=torch.int64),
            "base": z(E, R, dt=torch.int64),           # byte-stream base of every robot's UL offsets
            "last_nprb": z(E, R, dt=f32),               # PRBs of the last PUSCH (ul_amc_alloc "previous")
            # per-robot Doppler: the last pose, whether it is set, the AR(1) correlation per ms (the global one
            # until a pose step sets it: channels/doppler.py:32-37)
            "prev_pos": z(E, R, 2, dt=f32), "has_prev": z(E, R),
            "rho_ms": z(E, R, dt=f32, v=float(cfg.fading_rho_per_ms)),
        }
        self._n_fields = nf
        self._last_snr = torch.zeros(E, R, device=d)
        s = _lib.InetNrState()
        for name, _ in _lib.InetNrState._fields_:
            setattr(s, name, self.st[name].data_ptr())
        self._cstate = s
        self._ccells = None
        if self.C > 1:                       # association and N+I estimates (NRNet._init_cells, nr_engine.py:216-230)
            C_ = self.C
            self.cst = {"serv": z(E, R), "a3_cand": z(E, R, v=-1), "a3_cnt": z(E, R), "ho_end": z(E, R),
                        "n_ho": z(E, R), "pending": z(E, v=1), "ni_ul": z(E, C_, S, dt=f32), "ion": z(E, dt=f32)}
            if cfg.rlf:                      # radio link failure (CellAssociation.RLF_INIT, radio.py:340-342)
                self.cst.update({"rlf_active": z(E, R), "oos_cnt": z(E, R), "is_cnt": z(E, R),
                                 "t310_end": z(E, R, v=-1), "t311_end": z(E, R, v=-1), "reest_end": z(E, R, v=-1),
                                 "reest_cell": z(E, R), "n_rlf": z(E, R), "rlf_ctr": z(E, 5, dt=torch.int64)})
            c = _lib.InetNrCells()
            for name, t_ in self.cst.items():
                setattr(c, name, t_.data_ptr())
            if cfg.rlf:
                ms = lambda v: int(round(v / cfg.slot_ms))  # noqa: E731
                c.rlf, c.rlf_flush = 1, int(cfg.rlf_flush)
                c.n310, c.n311 = cfg.n310, cfg.n311
                c.t310, c.t311, c.reest = ms(cfg.t310_ms), ms(cfg.t311_ms), ms(cfg.reest_delay_ms)
                c.qout, c.qin = cfg.rlf_qout_db, cfg.rlf_qin_db
            xy = [v for p_ in cfg.gnb_xy() for v in p_]
            c.gnb_xy[:len(xy)] = xy
            c.C = C_
            c.ttt = int(round(cfg.a3_ttt_ms / cfg.slot_ms))
            c.ho_int = int(round(cfg.ho_interruption_ms / cfg.slot_ms))
            c.ho_flush = int(cfg.ho_rlc == "flush")
            c.use_int = int(cfg.noise_model == "thermal" and cfg.ul_interference)
            c.pc_on = int(cfg.ul_pc_on)
            c.has_floor = int(cfg.a3_min_target_rsrp_dbm is not None)
            c.a3_off, c.a3_hyst = cfg.a3_offset_db, cfg.a3_hyst_db
            if c.has_floor:
                c.floor_rx = cfg.a3_min_target_rsrp_dbm - (cfg.gnb_tx_dbm - 10 * math.log10(12 * cfg.nprb)
                                                           - cfg.ue_tx_dbm)
            c.noise_mw = 10 ** (cfg.noise_dbm_per_prb("gnb") / 10)
            c.ref_db = 10 * math.log10(cfg.snr_ref_prbs)
            c.li_a, c.li_b = cfg.li_alpha, 1 - cfg.li_alpha
            c.pc_p0, c.pc_alpha = cfg.ul_pc_p0_dbm, cfg.ul_pc_alpha
            self._ccells = c
        if self.dl:
            self.dst = {
                "sent": z(E, R), "floor_": z(E, R), "last_tx": z(E, R, v=-1), "olla": z(E, R, dt=f32),
                "avg": z(E, R, dt=f32, v=100.0), "enq": z(E, R), "qlen": z(E, R), "csi": z(E, S, R, dt=f32),
                "h_meta": z(E, P, R), "h_lo": z(E, P, R), "h_hi": z(E, P, R), "h_ready": z(E, P, R),
                "h_tbs": z(E, P, R), "h_comb": z(E, P, R, dt=f32), "h_lexp": z(E, P, R, dt=f32, v=-math.inf),
                "h_nrb": z(E, P, R, dt=f32), "q_cap": z(E, F, R, v=-1), "q_start": z(E, F, R), "q_end": z(E, F, R),
                "q_fin": z(E, F, R, v=BIG_SLOT), "q_meta": z(E, F, R), "newest": z(E, R, v=-1),
                "ctr": z(E, NCTR, dt=torch.int64), "hist": z(E, 3, cfg.max_harq_tx + 1, dt=torch.int64),
                "base": z(E, R, dt=torch.int64),
            }
            ds = _lib.InetNrDlState()
            for name, t_ in self.dst.items():
                setattr(ds, name, t_.data_ptr())
            if cfg.cqi_table == "38214":
                thr, cm = cqi_tables(self.tabs_dl, cfg.mcs_table)
                self._cqi = (torch.from_numpy(thr).to(d), torch.from_numpy(cm.astype(np.int32)).to(d))
                ds.cqi_thr, ds.cqi_mcs = self._cqi[0].data_ptr(), self._cqi[1].data_ptr()
            ds.gnb_proc = cfg.gnb_proc_slots
            ds.ref_off = cfg.gnb_tx_dbm - 10 * math.log10(cfg.nprb)
            ds.noise_prb = cfg.noise_dbm_per_prb("ue")
            ds.snr_off = cfg.dl_snr_offset_db
            self._cdl = ds

    def _upload_tables(self):
        cfg, t, d = self.config, self.tabs, self.dev
        nsyms = sorted({cfg.slot_symbols(p)[1] for p in range(len(cfg.tdd_pattern))} - {0}) or [cfg.ul_data_symbols]
        if self.dl:
            nsyms = sorted(set(nsyms) | ({cfg.slot_symbols(p)[0] for p in range(len(cfg.tdd_pattern))} - {0}))
        self._nsym_idx = {ns: i for i, ns in enumerate(nsyms)}
        la = [t.la_tables(cfg.nprb, ns, cfg.dmrs_re_per_prb, cfg.overhead_re_per_prb) for ns in nsyms]
        w = torch.tensor(cfg.subband_prbs, dtype=torch.float32)
        host = {
            "bler": torch.from_numpy(t.bler.reshape(-1)), "thr_ref": torch.from_numpy(t.thr_ref),
            "se": torch.from_numpy(t.se), "beta": torch.from_numpy(t.beta), "rate": torch.from_numpy(t.r),
            "mcs_eq": torch.from_numpy(t.mcs_eq.astype(np.int32)).reshape(-1),
            "la_tbs": torch.from_numpy(np.stack([x[0] for x in la])).reshape(-1),
            "la_ci0": torch.from_numpy(np.stack([x[1] for x in la]).astype(np.int32)).reshape(-1),
            "la_cwi": torch.from_numpy(np.stack([x[2] for x in la])).reshape(-1),
            "la_ncb": torch.from_numpy(np.stack([x[3] for x in la])).reshape(-1),
            "w": w, "logw": torch.log(w.float()), "wdb": 10 * torch.log10(w / cfg.snr_ref_prbs),
        }
        self.tab = {k: v.contiguous().to(d) for k, v in host.items()}
        c = _lib.InetNrTables()
        for k, v in self.tab.items():
            setattr(c, k, v.data_ptr())
        c.s0, c.ds, c.c0, c.dc = t.s0, t.ds, t.c0, t.dc
        c.M, c.C, c.G, c.NPRB, c.EQW, c.mcs_max = t.M, t.C, t.G, cfg.nprb, t.mcs_eq.shape[1], t.mcs_max
        c.thr_monotone = int(bool(np.all(np.diff(t.thr_ref[:t.mcs_max + 1]) >= 0)))
        self._ctab = c
        if self.dl:                                   # the same tables with the DL MCS cap
            cd = _lib.InetNrTables()
            C.memmove(C.addressof(cd), C.addressof(c), C.sizeof(c))
            mx = self.tabs_dl.mcs_max
            cd.mcs_max = mx
            cd.thr_monotone = int(bool(np.all(np.diff(t.thr_ref[:mx + 1]) >= 0)))
            self._ctab_dl = cd
        self._sizes = torch.tensor(cfg.msg_sizes, dtype=torch.float32, device=d)

    def _build_params(self):
        from .channels import SCENARIOS, SIGMA_SF, breakpoint_m
        cfg = self.config
        p = _lib.InetNrParams()
        p.E, p.R, p.S, p.P, p.F, p.N = self.E, self.R, self.S, self.P, self.F, self.N
        p.sched = {"pf": 0, "pf_wideband": 0, "maxci": 1, "rr": 2}[cfg.scheduler]
        p.pf_wb = int(cfg.pf_metric == "wideband" or cfg.scheduler == "pf_wideband")   # (mac.py:259)
        p.comb = {"none": 0, "cc": 1, "ir_lena": 2}[cfg.harq_combining]
        p.eesm = int(cfg.eff_sinr == "eesm")
        p.harq_drop = int(cfg.harq_fail == "drop")
        p.olla, p.phr_cap, p.retx_prio = int(cfg.olla), int(cfg.phr_cap), int(cfg.retx_priority)
        p.rician, p.fading = int(cfg.rician_mode in ("fixed", "los")), int(cfg.fading)
        p.k_from_los = int(cfg.rician_mode == "los")
        if p.k_from_los:                              # (mu_K, sigma_K) of the scenario (nr_engine.py:67-77)
            p.k_mu, p.k_sigma = RICIAN_K_DB[scenario_name(cfg.tr38901_scenario)]
            p.k_ramp = int(cfg.rician_k_ramp_slots)   # K ramps to a new target over k_ramp slots
            p.k_rinv = 1.0 / p.k_ramp if p.k_ramp else 0.0
        p.purge = int(cfg.discard == "purge")
        # per-robot Doppler (engine.py:862-864, channels/doppler.py:23-29): the float32 scalars of the reference's
        # tensor-scalar operations (f_c / c, 2 pi 2.5 ms evaluated left to right in double, the control step in s)
        p.doppler = int(cfg.fading_doppler == "per_robot")
        p.dop_floor = cfg.doppler_min_speed_mps
        p.dop_kf = cfg.carrier_ghz * 1e9 / 299_792_458.0
        p.dop_kx = 2 * math.pi * 2.5 * 1e-3
        p.dop_dt = cfg.control_step_ms * 1e-3
        p.out_ref = int(self.out_format == "reference")
        p.max_tx, p.sr_delay, p.ul_rtt, p.rlc_retx = cfg.max_harq_tx, cfg.sr_delay, cfg.ul_rtt, cfg.rlc_retx_slots
        p.timeout, p.tb_oh = cfg.timeout_steps, cfg.tb_overhead_bytes
        p.n_fields, p.n_modes = self._n_fields, cfg.shadow_modes
        p.n_cells = self.C
        p.rebase_at = self.REBASE_AT
        p.seed_key = C.c_int32(seed_key(self.seed) - (1 << 32) if seed_key(self.seed) >= 1 << 31
                               else seed_key(self.seed)).value
        p.olla_up = cfg.olla_up_db
        p.olla_dn = cfg.olla_up_db * (1 - cfg.bler_target) / cfg.bler_target
        p.pf_a, p.pf_b = 1 - 1 / cfg.pf_window, 1 / cfg.pf_window
        # 5G-LENA MAC switches and UL power control at one cell (mac.py:26-31, mac_ul.py:154-180, nr_engine.py:649-675)
        p.pf_rbg, p.pf_freeze = int(cfg.pf_update == "rbg"), int(cfg.pf_avg_idle == "freeze")
        p.whole_band = int(cfg.ul_power == "whole_band")
        p.wb_db = 10 * math.log10(cfg.nprb / cfg.snr_ref_prbs)
        p.pc1_on = int(cfg.ul_pc_on and cfg.n_cells == 1)
        p.retx_tdma, p.amc_prev = int(cfg.ul_retx_sched == "tdma"), int(cfg.ul_amc_alloc == "previous")
        # frequency-correlated fading: the square root of the subband correlation (nr_engine.py:320-330)
        L = subband_fading_sqrt(cfg)
        self._fc_L = None if L is None else L.to(self.dev)
        p.fc_on = int(L is not None)
        p.fc_L = self._fc_L.data_ptr() if L is not None else None
        if cfg.freq_corr_mode == "los":    # per-link delay spreads: L on the log grid, lgDS per state (:330-340)
            _, tab = delay_spread_grid(cfg)
            self._fc_tab = tab.to(self.dev).contiguous()
            lo, hi, G = cfg.fading_ds_grid
            scn = scenario_name(cfg.tr38901_scenario)
            p.fc_on, p.fc_G, p.fc_tab = 2, int(G), self._fc_tab.data_ptr()
            (p.ds_mu_n, p.ds_sig_n), (p.ds_mu_l, p.ds_sig_l) = (lg_ds_params(scn, cfg.carrier_ghz, los)
                                                                for los in (False, True))
            p.ds_c1 = math.log10(lo)
            p.ds_c2 = (int(G) - 1) / (math.log10(hi) - math.log10(lo))
        p.pc_p0, p.pc_alpha = cfg.ul_pc_p0_dbm, cfg.ul_pc_alpha
        p.target, p.phr_min, p.snr_ref_prbs = cfg.bler_target, cfg.phr_min_db, float(cfg.snr_ref_prbs)
        p.w0 = float(cfg.subband_prbs[0])
        p.ref_off = cfg.ue_tx_dbm - 10 * math.log10(cfg.snr_ref_prbs)
        p.noise_prb, p.ue_tx, p.subband_noise = cfg.noise_dbm_per_prb("gnb"), cfg.ue_tx_dbm, cfg.subband_noise_dbm
        gx, gy = cfg.gnb_xy()[0]
        p.gnb_x, p.gnb_y = gx, gy
        po = cfg.proc_offset_ms / cfg.control_step_ms
        p.proc_off_hi = po
        p.proc_off_lo = po - float(np.float32(po))
        K = cfg.shadow_modes
        self._spectrum, self._dcorr = 0, (cfg.shadow_dcorr_m, 0.0, 0.0)
        if cfg.channel == "tr38901":
            sc = SCENARIOS[cfg.tr38901_scenario]
            scn = cfg.tr38901_scenario
            h_bs = float(cfg.gnb_height_m) if cfg.gnb_height_m is not None else sc.h_bs
            h_ut, fc = float(cfg.ue_height_m), cfg.carrier_ghz
            dbp = breakpoint_m(scn, fc, h_bs, h_ut)
            p.radio_model = 1
            p.hh2 = (h_bs - h_ut) ** 2
            p.dbp = dbp if math.isfinite(dbp) else float("inf")
            if scn in ("UMa", "UMi"):
                a, n1, b = (28.0, 22.0, 9.0) if scn == "UMa" else (32.4, 21.0, 9.5)
                p.pl_a, p.pl_n1, p.pl_c20 = a, n1, 20 * math.log10(fc)
                p.pl_c2 = b * math.log10(dbp ** 2 + (h_bs - h_ut) ** 2)
            elif scn == "InH":
                p.pl_a, p.pl_n1, p.pl_c20, p.pl_c2 = 32.4, 17.3, 20 * math.log10(fc), 0.0
            else:                                                   # InF (LOS)
                p.pl_a, p.pl_n1, p.pl_c20, p.pl_c2 = 31.84, 21.50, 19.00 * math.log10(fc), 0.0
            los = cfg.tr38901_los == "los"
            sto = cfg.tr38901_los == "stochastic"
            if sto:              # the stochastic LOS state: LOS and NLOS parameters, the CDF of the LOS-state field
                self._los_cdf = sum_of_cosines_cdf_table(K).to(self.dev)
                p.los_sto, p.los_cdf = 1, self._los_cdf.data_ptr()
                p.plos_scn = {"UMi": 0, "UMa": 1, "InH": 2}[scn]
                p.sig_nlos = SIGMA_SF[scn][1]
            if not los:
                if scn == "UMi":
                    p.nl_b1, p.nl_b0, p.nl_c, p.nl_d = 35.3, 22.4, 21.3 * math.log10(fc), 0.3 * (h_ut - 1.5)
                elif scn == "UMa":
                    p.nl_b1, p.nl_b0, p.nl_c, p.nl_d = 39.08, 13.54, 20 * math.log10(fc), 0.6 * (h_ut - 1.5)
                else:                                               # InH
                    p.nl_b1, p.nl_b0, p.nl_c, p.nl_d = 38.3, 17.30, 24.9 * math.log10(fc), 0.0
            p.sig = SIGMA_SF[scn][0 if (los or sto) else 1]
            p.amp = 1.0 * math.sqrt(2 / K)
            self._spectrum, self._dcorr = 1, (sc.sf_corr_los_m, sc.sf_corr_nlos_m, sc.los_corr_m)
        else:
            p.radio_model = 0
            p.amp = cfg.shadow_sigma_db * math.sqrt(2 / K)
            p.pl_const, p.pl_exp10 = cfg.pl_const_db, 10 * cfg.pathloss_exp
            self._spectrum = 0 if cfg.shadow_acf == "sos" else 1
        self._cparams = p
        self._dcorr_c = (C.c_float * 3)(*self._dcorr)

    # ------------------------------------------------------------------ schedule rows (nr_engine.py:506-523)
    def _rows_for(self, g0, dt0):
        cfg = self.config
        P_ = len(cfg.tdd_pattern)
        key = (g0 % math.lcm(P_, cfg.sr_period_slots, cfg.cqi_period_slots), dt0)
        hit = self._rows.get(key)
        if hit is not None:
            return hit
        sched = cfg.schedule(g0)
        pg_pos = next(p for p in range(P_) if cfg.slot_symbols(p)[1] > 0)
        rows, prev = [], None
        evol, rhos = [], []
        for rel, _dls, uls, sr, _cqi, _ack in sched:
            dt = dt0 if prev is None else rel - prev
            prev = rel
            rho = self._row_rho(dt)[0]
            evol.append(cfg.fading and dt > 0)
            rhos.append(float(np.float32(rho)))
        n = len(sched)
        for k, (rel, _dls, uls, sr, _cqi, _ack) in enumerate(sched):
            dt = dt0 if k == 0 else rel - sched[k - 1][0]
            rho, c1 = self._row_rho(dt)
            need_h = evol[k] and (uls > 0 or k == n - 1 or not (evol[k + 1] and rhos[k + 1] == 0.0))
            pg = cfg.proactive_grant == "every_ul_slot" or (cfg.proactive_grant == "per_period"
                                                            and (g0 + rel) % P_ == pg_pos)
            flags = (1 if sr else 0) | (2 if uls else 0) | (4 if evol[k] else 0) | (8 if need_h else 0) | \
                (16 if pg else 0)
            re = float(min(12 * uls - cfg.dmrs_re_per_prb - cfg.overhead_re_per_prb, 156)) if uls else 0.0
            rows.append((rel, self._nsym_idx.get(uls, -1), flags, re, rho, c1, salt((FADING << 16) | rel),
                         salt((BLER_UL << 16) | rel)))
        if n > 64:
            raise HipUnsupported("more than 64 scheduled slots (SR / UL / fading) per control step")
        res = (self._rows_to_device(rows), n, sched[-1][0] if sched else None, sum(1 for r in rows if r[2] & 2))
        if self.dl:
            res = res + (self._rows_to_device(self._dl_rows(sched, evol, rhos, dt0)),)
        self._rows[key] = res
        return res

    def _row_rho(self, dt):
        """(rho, c1) of a fading row dt slots after the previous one: rho^(dt slot_ms) and sqrt(1 - rho^2) of the
        global rho (nr_engine.py:583-585); with per-robot Doppler the exponent dt slot_ms (the kernels raise each
        robot's rho_ms to it, nr_engine.py:586-589) and 0."""
        cfg = self.config
        if cfg.fading_doppler == "per_robot":
            return (dt * cfg.slot_ms if dt > 0 else 1.0), 0.0
        rho = cfg.fading_rho_per_ms ** (dt * cfg.slot_ms) if dt > 0 else 1.0
        return rho, math.sqrt(1 - rho ** 2)

    def _dl_rows(self, sched, evol, rhos, dt0):
        """The DL rows of a step (the rows of the UL kernel with the DL meaning): flags 1 CQI report, 2 DL data slot,
        4 / 8 fading evolves / its gain is needed (at DL data and CQI rows, and wherever a later row's evolution
        depends on it), bits 8..23 the HARQ-ACK slot relative to the step's first slot; the DL decode stream."""
        cfg = self.config
        n = len(sched)
        rows = []
        for k, (rel, dls, _uls, _sr, cqi, ack) in enumerate(sched):
            dt = dt0 if k == 0 else rel - sched[k - 1][0]
            rho, c1 = self._row_rho(dt)
            need_h = evol[k] and (dls > 0 or cqi or (k < n - 1 and not (evol[k + 1] and rhos[k + 1] == 0.0)))
            if not 0 <= ack < 1 << 16:
                raise HipUnsupported("a HARQ-ACK slot more than 65535 slots after the step start")
            flags = (1 if cqi else 0) | (2 if dls else 0) | (4 if evol[k] else 0) | (8 if need_h else 0) | (ack << 8)
            re = float(min(12 * dls - cfg.dmrs_re_per_prb - cfg.overhead_re_per_prb, 156)) if dls else 0.0
            rows.append((rel, self._nsym_idx.get(dls, -1), flags, re, rho, c1, salt((FADING << 16) | rel),
                         salt((BLER_DL << 16) | rel)))
        return rows

    def _rows_to_device(self, rows):
        buf = np.zeros((max(len(rows), 1), 8), dtype=np.int32)
        for k, r in enumerate(rows):
            buf[k, 0:3] = r[0:3]
            buf[k, 3:6] = np.array(r[3:6], dtype=np.float32).view(np.int32)
            buf[k, 6:8] = np.array(r[6:8], dtype=np.uint32).view(np.int32)
        return torch.from_numpy(buf).to(self.dev)

    # ------------------------------------------------------------------ contract API
    @property
    def clock(self):
        return self.T - self.st["epoch"].long()

    def output_schema(self):
        keys = [("newest", "[E,R]", "int64"), ("det_env", "[E]", "bool"), ("delivered", "[E,R,F]", "bool"),
                ("timed_out", "[E,R,F]", "bool"), ("dropped", "[E,R,F]", "bool"), ("cap", "[E,R,F]", "int64"),
                ("cls", "[E,R,F]", "int64"), ("delay", "[E,R,F]", "float32"), ("queue_len", "[E,R]", "int64"),
                ("queue_bytes", "[E,R]", "float32"), ("sinr_db", "[E,R]", "float32"),
                ("serving_cell", "[E,R]", "int64"), ("t", "[E]", "int64")]
        out = {k: {"shape": s, "dtype": dt, "when": "always"} for k, s, dt in keys}
        if self.dl:
            for k in ("dl_newest", "dl_queue_len"):
                out[k] = {"shape": "[E,R]", "dtype": "int64", "when": "dl"}
        return out

    def _now(self, t):
        """engine.py:738-755."""
        if t is None:
            return self.T
        if isinstance(t, torch.Tensor):
            if t.dim() == 0:
                t = int(t)
            else:
                if not torch.equal(t.to(self.dev, torch.long), self.clock):
                    raise ValueError("t must equal the engine clock (the NR engine cannot jump in time); pass t=None")
                return self.T
        t = int(t)
        if self._uniform_epoch is None:
            raise ValueError("after a partial reset the envs have different clocks: pass t=None")
        if t + self._uniform_epoch != self.T:
            raise ValueError(f"t={t} but the engine clock is {self.T - self._uniform_epoch}: the NR engine cannot "
                             "jump in time; pass t=None")
        return self.T

    def _stream(self):
        return torch.cuda.current_stream(self.dev).cuda_stream

    def reset(self, env_ids=None):
        """Re-initialize env_ids (None = all; index tensor, list or bool mask [E])."""
        if env_ids is not None and isinstance(env_ids, slice) and env_ids == slice(None):
            env_ids = None
        lib = self._lib
        if env_ids is None:
            self.T = 0
            self._ul_slots_run = 0
            self._dl_slots_run = 0
            self._uniform_epoch = 0
            self.last_g = None
            self._last_snr = torch.zeros_like(self._last_snr)
            self._last_hid = torch.zeros_like(self._last_hid)
            _lib.check(lib.inet_nr_reset(C.byref(self._cstate), C.byref(self._cparams), None, 0,
                                         self._k_lin0(), self._dcorr_c, self._spectrum, self._stream()), "reset")
            if self._ccells is not None:
                _lib.check(lib.inet_nr_cells_reset(C.byref(self._ccells), C.byref(self._cparams), None,
                                                   self._stream()), "cells reset")
            if self.dl:
                _lib.check(lib.inet_nr_dl_reset(C.byref(self._cdl), C.byref(self._cparams), None, self._stream()),
                           "dl reset")
            return
        if isinstance(env_ids, torch.Tensor) and env_ids.dtype == torch.bool:
            mask = env_ids.to(self.dev)
        else:
            ids = torch.as_tensor(env_ids if isinstance(env_ids, torch.Tensor) else list(env_ids), dtype=torch.long,
                                  device=self.dev).reshape(-1)
            if ids.numel() == 0:
                return
            mask = torch.zeros(self.E, dtype=torch.bool, device=self.dev)
            mask[ids] = True
        rows = mask.nonzero(as_tuple=True)[0].cpu()
        if rows.numel() == 0:
            return
        m8 = mask.to(torch.uint8).contiguous()
        _lib.check(lib.inet_nr_reset(C.byref(self._cstate), C.byref(self._cparams), m8.data_ptr(), self.T,
                                     self._k_lin0(), self._dcorr_c, self._spectrum, self._stream()), "reset")
        if self._ccells is not None:
            _lib.check(lib.inet_nr_cells_reset(C.byref(self._ccells), C.byref(self._cparams), m8.data_ptr(),
                                               self._stream()), "cells reset")
        if self.dl:
            _lib.check(lib.inet_nr_dl_reset(C.byref(self._cdl), C.byref(self._cparams), m8.data_ptr(),
                                            self._stream()), "dl reset")

        self._uniform_epoch = None
        mk = mask[:, None]
        self._last_snr = torch.where(mk, torch.zeros_like(self._last_snr), self._last_snr)
        self._last_hid = torch.where(mask, torch.zeros_like(self._last_hid), self._last_hid)

    env_offset = 0

    def set_env_offset(self, offset):
        """Key env row i by the global env id offset + i (a shard of a larger batch, isaac_net/core/sharded.py:61-78,
        CounterRNG.set_env_offset, proto/rng.py:103-109): the env ids move in place, the episode counters are rewound
        by one and every env is reset again, so the envs redraw their initial state under the global ids and stay in
        their first episode. An env then draws the same numbers whichever shard holds it."""
        offset = int(offset)
        if offset == self.env_offset:
            return
        self.st["env_id"].add_(offset - self.env_offset)
        self.env_offset = offset
        self.st["episode"].sub_(1)
        self.reset(None)

    def _k_lin0(self):
        cfg = self.config
        return float(10 ** (cfg.rician_k_db / 10)) if cfg.rician_mode == "fixed" else 0.0

    def submit(self, t, requests, snr_db=None, *, tag=None, priority=None, deadline_ms=None):
        """Enqueue one message per robot (Requests or send [E,R]); returns accepted [E,R] bool (engine.py:796-819)."""
        if tag is not None or priority is not None or deadline_ms is not None:
            raise HipUnsupported("per-message extras (tag / priority / deadline_ms) are not implemented")
        T = self._now(t)
        req = requests if isinstance(requests, Requests) or hasattr(requests, "send") else Requests(send=requests)
        send = req.send.to(self.dev, torch.long).contiguous()
        if tuple(send.shape) != (self.E, self.R):
            raise ValueError(f"send must be [E,R] = [{self.E},{self.R}], got {tuple(send.shape)}")
        det = None if req.det is None else req.det.to(self.dev, torch.uint8).contiguous()
        hid = torch.zeros(self.E, dtype=torch.long, device=self.dev) if req.hid is None else \
            req.hid.to(self.dev, torch.long).contiguous()
        self._last_hid = hid.clone()
        acc = torch.empty(self.E, self.R, dtype=torch.bool, device=self.dev)
        cfg = self.config
        pre = self._stats_pre_submit(T) if self._log_stats else None
        _lib.check(self._lib.inet_nr_submit(
            C.byref(self._cstate), C.byref(self._cparams), T, send.data_ptr(), None if det is None else det.data_ptr(),
            hid.data_ptr(), None, 0, self._sizes.data_ptr(), int(cfg.discard == "pdcp_arrival"),
            cfg.pkt_payload_bytes, cfg.pkt_overhead_bytes, acc.data_ptr(), self._stream()), "submit")
        if pre is not None:
            snr = self._last_snr if snr_db is None else snr_db.to(self.dev, torch.float32)
            self._stats_enqueue(send > 0, *pre, snr if snr.dim() == 2 else snr.mean(-1), acc=acc)
        return acc

    def submit_counts(self, counts, t=None):
        """Enqueue counts [E,R,NC] messages per class in one launch: equivalent to the submit() calls of class 1
        first, one call per message index. Returns accepted messages [E,R] int32."""
        T = self._now(t)
        cnt = counts.to(self.dev, torch.uint8).contiguous()
        nc = cnt.shape[-1]
        if tuple(cnt.shape[:2]) != (self.E, self.R) or nc > len(self.config.msg_sizes):
            raise ValueError("counts must be [E,R,n_classes] with n_classes <= len(msg_sizes)")
        if self._log_stats:
            self._stats_counts(T, cnt)
        return self._launch_submit_counts(T, cnt)

    def _launch_submit_counts(self, T, cnt):
        self._last_hid = torch.zeros_like(self._last_hid)
        acc = torch.empty(self.E, self.R, dtype=torch.int32, device=self.dev)
        cfg = self.config
        _lib.check(self._lib.inet_nr_submit(
            C.byref(self._cstate), C.byref(self._cparams), T, None, None, None, cnt.data_ptr(), cnt.shape[-1],
            self._sizes.data_ptr(), int(cfg.discard == "pdcp_arrival"), cfg.pkt_payload_bytes,
            cfg.pkt_overhead_bytes, acc.data_ptr(), self._stream()), "submit")
        return acc

    def add_frames(self, t, send, det, hid, snr_db=None):
        """Legacy wrapper (NetSlot API)."""
        self.submit(t, Requests(send, det, hid), snr_db)

    def add_dl_frames(self, t, nbytes, cls=None):
        """Downlink messages of nbytes [E,R] application bytes (0 = none) at t, with classes cls [E,R] (0..255) or
        None (NREngine.add_dl_frames, engine.py:825-827; needs config.dl). Returns accepted [E,R] bool."""
        if not self.dl:
            raise ValueError("add_dl_frames needs NRConfig(dl=True)")
        T = self._now(t)
        nb = torch.as_tensor(nbytes).to(self.dev, torch.float32).contiguous()
        if tuple(nb.shape) != (self.E, self.R):
            raise ValueError(f"nbytes must be [E,R] = [{self.E},{self.R}], got {tuple(nb.shape)}")
        cl = None
        if cls is not None:
            cl = torch.as_tensor(cls).to(self.dev, torch.long).contiguous()
            if tuple(cl.shape) != (self.E, self.R):
                raise ValueError("cls must be [E,R]")
            if bool(((cl < 0) | (cl > 255)).any()):
                raise HipUnsupported("DL message classes outside 0..255 (8-bit class field)")
        acc = torch.empty(self.E, self.R, dtype=torch.bool, device=self.dev)
        cfg = self.config
        _lib.check(self._lib.inet_nr_dl_submit(
            C.byref(self._cstate), C.byref(self._cdl), C.byref(self._cparams), T, nb.data_ptr(),
            None if cl is None else cl.data_ptr(), int(cfg.discard == "pdcp_arrival"), cfg.pkt_payload_bytes,
            cfg.pkt_overhead_bytes, acc.data_ptr(), self._stream()), "dl submit")
        if self._log_stats:                         # every refused DL frame (nr_engine.py:496-497)
            self.stats["overflow_dl"] = self.stats.get("overflow_dl", 0) + int(((nb > 0) & ~acc).sum())
        return acc

    def _alloc_out(self):
        E, R, F, d = self.E, self.R, self.F, self.dev
        e = lambda *s, dt: torch.empty(*s, dtype=dt, device=d)  # noqa: E731
        if self.out_format == "reference":
            o = {"newest": e(E, R, dt=torch.int64), "det_env": e(E, dt=torch.bool),
                 "delivered": e(E, R, F, dt=torch.bool), "timed_out": e(E, R, F, dt=torch.bool),
                 "dropped": e(E, R, F, dt=torch.bool), "cap": e(E, R, F, dt=torch.int64),
                 "cls": e(E, R, F, dt=torch.int64), "delay": e(E, R, F, dt=torch.float32),
                 "queue_len": e(E, R, dt=torch.int64), "queue_bytes": e(E, R, dt=torch.float32),
                 "sinr_db": e(E, R, dt=torch.float32), "serving_cell": e(E, R, dt=torch.int64),
                 "t": e(E, dt=torch.int64)}
        else:
            o = {"newest": e(E, R, dt=torch.int64), "det_env": e(E, dt=torch.bool), "flags": e(E, R, F, dt=torch.uint8),
                 "cap32": e(E, R, F, dt=torch.int32), "cls8": e(E, R, F, dt=torch.uint8),
                 "delay": e(E, R, F, dt=torch.float32), "queue_len": e(E, R, dt=torch.int64),
                 "queue_bytes": e(E, R, dt=torch.float32), "sinr_db": e(E, R, dt=torch.float32),
                 "t": e(E, dt=torch.int64)}
        c = _lib.InetNrOutputs()
        ptr = lambda k: o[k].data_ptr() if k in o else None  # noqa: E731
        c.delivered = ptr("delivered") or ptr("flags")
        c.timed_out, c.dropped, c.cap, c.cls = ptr("timed_out"), ptr("dropped"), ptr("cap"), ptr("cls")
        c.cap32, c.cls8, c.delay = ptr("cap32"), ptr("cls8"), ptr("delay")
        c.newest, c.queue_len, c.serving_cell = ptr("newest"), ptr("queue_len"), ptr("serving_cell")
        c.queue_bytes, c.sinr_db, c.det_env, c.t = ptr("queue_bytes"), ptr("sinr_db"), ptr("det_env"), ptr("t")
        if self._ccells is not None and self.config.rlf:      # robots in radio link failure after the step
            o["rlf"] = e(E, R, dt=torch.bool)
            self._ccells.out_rlf = o["rlf"].data_ptr()
        return o, c

    def step(self, t=None, x=None, cur_hid=None, *, snr_db=None, dl_snr_db=None, pathgain_db=None, vel=None,
             triggers=None, blockers=None, arrivals=None):
        """Advance [t, t+1). x: poses [E,R,2|3] (through the radio) or SNR [E,R] dB; snr_db=: [E,R,S] or [E,R].
        Returns the reference's output dict; with cur_hid (legacy form) returns (newest, det_env).
        arrivals= (extension): counts [E,R,NC] uint8 of this step's messages, enqueued inside the step's launch as
        submit_counts(counts) would do before it; the dict then also holds arrivals_accepted [E,R] int32."""
        if pathgain_db is not None and self.C == 1:
            raise ValueError("pathgain_db= needs config.n_cells > 1; use x (poses or SNR) with one cell")
        if (dl_snr_db is not None and not self.dl) or triggers is not None or blockers is not None:
            raise HipUnsupported("dl_snr_db (without dl=True) / triggers / blockers need features the hip backend "
                                 "does not implement (traffic models, blockage)")
        T = self._now(t)
        legacy = cur_hid is not None
        hid = (cur_hid if legacy else self._last_hid).to(self.dev, torch.long).contiguous()
        kind, xin = self._input(x, snr_db, pathgain_db)
        self._check_kind(kind)
        vin = self._vel_input(vel, kind)
        plan = self._plan(T, kind)
        dl = None
        if self.dl:
            # DL reference (NREngine.step -> NRNet.step_rx / step, nr_engine.py:624-631, 651-653): from the poses'
            # path gain; or the UL SNR plus dl_snr_offset_db; or dl_snr_db as given (SNR input only)
            if kind != 0 and dl_snr_db is not None:
                dxin = dl_snr_db.to(self.dev, torch.float32).contiguous()
                dkind = 2 if dxin.dim() == 3 else 1
                if tuple(dxin.shape) != {1: (self.E, self.R), 2: (self.E, self.R, self.S)}[dkind]:
                    raise ValueError(f"dl_snr_db must be [E,R] or [E,R,S], got {tuple(dxin.shape)}")
                dl = (dkind, dxin, 0)
            else:
                dl = (kind, xin, 1)
        arr = None
        if arrivals is not None:
            cnt = arrivals.to(self.dev, torch.uint8).contiguous()
            if tuple(cnt.shape[:2]) != (self.E, self.R) or cnt.dim() != 3 or cnt.shape[-1] > len(self.config.msg_sizes):
                raise ValueError("arrivals must be [E,R,n_classes] with n_classes <= len(msg_sizes)")
            arr = cnt
            if not legacy:
                self._last_hid = torch.zeros_like(self._last_hid)
                hid = self._last_hid
        if arr is not None and self._log_stats:
            self._stats_counts(T, arr)
        self._cparams.vel = None if vin is None else vin.data_ptr()
        try:
            o = self._launch_step(T, plan, xin, hid, dl, arrivals=arr)
        finally:
            self._cparams.vel = None
        if self._log_stats:
            self._stats_step(o)
        self._commit(T, plan, o)
        if legacy:
            return o["newest"], o["det_env"]
        return o

    def _input(self, x, snr_db, pathgain_db=None):
        E, R, S = self.E, self.R, self.S
        if pathgain_db is not None:                  # several cells: the path gain of every link as given (kind 3)
            xin = pathgain_db.to(self.dev, torch.float32).contiguous()
            if tuple(xin.shape) != (E, R, self.C):
                raise ValueError(f"pathgain_db must be [E,R,C] = {(E, R, self.C)}, got {tuple(xin.shape)}")
            return 3, xin
        if snr_db is None:
            if x is None:
                raise ValueError("step needs poses [E,R,2|3] or an SNR [E,R]")
            if x.dim() == 3:
                kind, xin = 0, x[..., :2].to(self.dev, torch.float32).contiguous()
            else:
                kind, xin = 1, x.to(self.dev, torch.float32).contiguous()
        else:
            xin = snr_db.to(self.dev, torch.float32).contiguous()
            kind = 2 if xin.dim() == 3 else 1
        want = {0: (E, R, 2), 1: (E, R), 2: (E, R, S)}[kind]
        if tuple(xin.shape) != want:
            raise ValueError(f"input must have shape {want}, got {tuple(xin.shape)}")
        return kind, xin

    def _vel_input(self, vel, kind):
        """The velocity input [E,R,2|3] (m/s) of a pose step with per-robot Doppler as a contiguous [E,R,2] float32
        device tensor (the speed is |vel[..., :2]|, radio.py:292-293); None without one. Like the reference it is
        ignored with SNR input or without per-robot Doppler."""
        if vel is None or kind != 0 or self.config.fading_doppler != "per_robot":
            return None
        v = vel[..., :2].to(self.dev, torch.float32).contiguous()
        if tuple(v.shape) != (self.E, self.R, 2):
            raise ValueError(f"vel must be [E,R,2|3], got {tuple(vel.shape)}")
        return v

    def _check_kind(self, kind):
        if self.R > 64 and kind == 2:
            raise HipUnsupported("per-subband SNR input with more than 64 robots per env")
        if self.C > 1 and kind not in (0, 3):
            raise ValueError("several cells: pass poses [E,R,2|3] or pathgain_db=[E,R,C]")

    def _schedule(self, g0):
        """cfg.schedule(g0), cached by g0 modulo the period of the TDD pattern, SR and CQI occasions."""
        cfg = self.config
        k = g0 % math.lcm(len(cfg.tdd_pattern), cfg.sr_period_slots, cfg.cqi_period_slots)
        sc = self.__dict__.setdefault("_sched_cache", {})
        if k not in sc:
            sc[k] = cfg.schedule(g0)
        return sc[k]

    def _plan(self, T, kind):
        """The host side of step T: its slot rows (device), their count, the last fading slot and the UL slots."""
        cfg = self.config
        g0 = T * self.N
        sched = self._schedule(g0)
        fad = cfg.fading and len(sched) > 0
        dt0 = (1 if self.last_g is None else g0 + sched[0][0] - self.last_g) if fad else 0
        rows, n_rows, last_rel, n_ul, *dl_rows = self._rows_for(g0, dt0)
        key = (g0 % math.lcm(len(cfg.tdd_pattern), cfg.sr_period_slots, cfg.cqi_period_slots), dt0, kind)
        n_dl = sum(1 for r in sched if r[1]) if self.dl else 0
        return dict(rows=rows, n_rows=n_rows, last_rel=last_rel, n_ul=n_ul, fad=fad, kind=kind, key=key,
                    dl_rows=dl_rows[0] if dl_rows else None, n_dl=n_dl)

    def _launch_step(self, T, plan, xin, hid, dl=None, arrivals=None):
        """Launch the step kernel (T < 0: the kernel reads the device clock) and return the output dict. With the
        downlink, dl = (input kind, input, add dl_snr_offset_db) of the DL step, launched first: it reads the fading
        state and RNG words of the step start, which the UL step then advances."""
        o, co = self._alloc_out()
        if self.dl:
            dkind, dxin, add_off = dl
            E, R, d = self.E, self.R, self.dev
            o["dl_newest"] = torch.empty(E, R, dtype=torch.int64, device=d)
            o["dl_queue_len"] = torch.empty(E, R, dtype=torch.int64, device=d)
            cd = self._cdl
            cd.out_newest, cd.out_queue_len = o["dl_newest"].data_ptr(), o["dl_queue_len"].data_ptr()
            cd.out_delay = None if self._dl_delay is None else self._dl_delay.data_ptr()
            cd.snr_offset = add_off
            self._cparams.input_kind = dkind
            self._cparams.n_data = plan["n_dl"]
            dev_ = self.dl_kernel_events
            if dev_ is not None:
                dev_.begin(torch.cuda.current_stream(self.dev))
            _lib.check(self._lib.inet_nr_dl_step(C.byref(self._cstate), C.byref(cd), C.byref(self._ctab_dl),
                                                 C.byref(self._cparams), plan["dl_rows"].data_ptr(), plan["n_rows"], T,
                                                 dxin.data_ptr(), self._stream()), "dl step")
            if dev_ is not None:
                dev_.end(torch.cuda.current_stream(self.dev))
        self._cparams.input_kind = plan["kind"]
        self._cparams.n_data = plan["n_ul"]
        ev = self.kernel_events
        if ev is not None:
            ev.begin(torch.cuda.current_stream(self.dev))
        if self._ccells is not None:                  # NRNet.step_cells (inet_nr_step_cells), arrivals fused or not
            a = None
            if arrivals is not None:
                cfg = self.config
                o["arrivals_accepted"] = torch.empty(self.E, self.R, dtype=torch.int32, device=self.dev)
                a = _lib.InetNrArrivals(arrivals.data_ptr(), self._sizes.data_ptr(), o["arrivals_accepted"].data_ptr(),
                                        arrivals.shape[-1], int(cfg.discard == "pdcp_arrival"), cfg.pkt_payload_bytes,
                                        cfg.pkt_overhead_bytes)
            _lib.check(self._lib.inet_nr_step_cells(
                C.byref(self._cstate), C.byref(self._ccells), C.byref(self._ctab), C.byref(self._cparams),
                plan["rows"].data_ptr(), plan["n_rows"], T, xin.data_ptr(), hid.data_ptr(), C.byref(co),
                None if a is None else C.byref(a), self._stream()), "step")
        elif arrivals is None:
            _lib.check(self._lib.inet_nr_step(C.byref(self._cstate), C.byref(self._ctab), C.byref(self._cparams),
                                              plan["rows"].data_ptr(), plan["n_rows"], T, xin.data_ptr(),
                                              hid.data_ptr(), C.byref(co), self._stream()), "step")
        else:
            cfg = self.config
            o["arrivals_accepted"] = torch.empty(self.E, self.R, dtype=torch.int32, device=self.dev)
            a = _lib.InetNrArrivals(arrivals.data_ptr(), self._sizes.data_ptr(), o["arrivals_accepted"].data_ptr(),
                                    arrivals.shape[-1], int(cfg.discard == "pdcp_arrival"), cfg.pkt_payload_bytes,
                                    cfg.pkt_overhead_bytes)
            _lib.check(self._lib.inet_nr_submit_step(
                C.byref(self._cstate), C.byref(self._ctab), C.byref(self._cparams), plan["rows"].data_ptr(),
                plan["n_rows"], T, xin.data_ptr(), hid.data_ptr(), C.byref(co), C.byref(a), self._stream()), "step")
        if ev is not None:
            ev.end(torch.cuda.current_stream(self.dev))
        return o

    def _commit(self, T, plan, o):
        """Host bookkeeping after step T: fading slot, UL slot count, clock, last SINR."""
        if plan["fad"]:
            self.last_g = T * self.N + plan["last_rel"]
        self._ul_slots_run += plan["n_ul"]
        if self.dl:
            self._dl_slots_run += plan["n_dl"]
        self.T = T + 1
        self._last_snr = o["sinr_db"]

    def graph_step(self, n_cls=None):
        """The control step (submit_counts of per-class arrival counts, then step) as HIP graph replays: returns a
        GraphStep, called as g(x, counts) or g(counts=..., snr_db=...) in place of submit_counts + step. A graph is
        recorded for every new slot schedule (TDD / SR / CQI phase, fading slot spacing) and input kind, then
        replayed; the downlink and several cells run inside the step graph."""
        return GraphStep(self, len(self.config.msg_sizes) if n_cls is None else n_cls)

    # ------------------------------------------------------------------ statistics
    FEATS = ("cls", "f_nact", "f_snr", "f_own")

    @property
    def log_stats(self):
        """Record per-frame statistics (NRNet.log_stats, nr_engine.py:440-446, 466-497, 885-914): per step the delay,
        env and features of the UL frames delivered, and of those timed out or dropped, captured at or before
        log_cap_max; the DL delays; the UL overflow, PDCP-discard, HARQ-drop and late counts, the refused DL
        frames and refused_env. The queue features f_nact (robots of the env with a queued frame when the frame
        arrived), f_snr (the SNR given to submit, else the previous step's) and f_own (its queue position) are kept
        while statistics are on: frames submitted while they were off carry 0."""
        return self._log_stats

    @log_stats.setter
    def log_stats(self, on):
        on = bool(on)
        if on and self._feat is None:
            E, R, F, d = self.E, self.R, self.F, self.dev
            self._feat = {"f_nact": torch.zeros(E, R, F, dtype=torch.long, device=d),
                          "f_snr": torch.zeros(E, R, F, dtype=torch.float32, device=d),
                          "f_own": torch.zeros(E, R, F, dtype=torch.long, device=d)}
            if self.dl:
                self._dl_delay = torch.empty(E, R, F, dtype=torch.float32, device=d)
        elif not on:
            self._feat, self._dl_delay = None, None
        self._log_stats = on

    def clear_stats(self):
        """Empty the statistics record and refused_env (NRNet.clear_stats)."""
        self.stats = {"delay": [], "overflow": 0, "dl_delay": [], "dropped": 0, "late": 0, "discarded": 0,
                      "d_env": [], "x_env": []}
        self.refused_env = torch.zeros(self.E, dtype=torch.long, device=self.dev)   # overflow + PDCP discard
        for f in self.FEATS:
            self.stats["d_" + f] = []
            self.stats["x_" + f] = []

    def queued(self):
        """Queued UL frames per robot [E,R] int64 (NRNet.queued)."""
        return self.st["qlen"].long()

    def collect(self):
        """The statistics since the last clear_stats() (NRNet.collect): every per-step list concatenated into one
        CPU tensor (an empty float32 tensor if nothing was logged), then the counts."""
        st = self.stats
        out = {k: (torch.cat(v) if v else torch.zeros(0)) for k, v in st.items() if isinstance(v, list)}
        out.update({k: v for k, v in st.items() if not isinstance(v, list)})
        return out

    def _stats_pre_submit(self, T):
        """(queued frames [E,R], head frame stale under discard="pdcp_arrival" [E,R]) before an enqueue at step T."""
        count = self.st["qlen"].long()
        if self.config.discard != "pdcp_arrival":
            return count, torch.zeros_like(count, dtype=torch.bool)
        head = self.st["q_cap"][:, 0, :].long()
        return count, (head >= 0) & ((T - head) >= self.config.timeout_steps)

    def _stats_enqueue(self, want, count, stale, snr, acc=None):
        """The statistics of one enqueue call (NRNet.add_frames, nr_engine.py:466-487): want [E,R] messages, count /
        stale as _stats_pre_submit's; acc: the accepted mask the launch returned (None: admission replayed here,
        PDCP refusal then the full queue). Records the accepted frames' features; returns (acc, queued after)."""
        st, F = self.stats, self.F
        adm = want & ~stale
        full = count >= F
        if acc is None:
            acc = adm & ~full
        st["overflow"] += int((adm & full).sum())
        st["discarded"] += int((want & ~adm).sum())
        self.refused_env += (want & ~acc).sum(-1)
        at = (torch.arange(F, device=self.dev) == count[..., None]) & acc[..., None]
        ft = self._feat
        nact = (count > 0).sum(-1)
        ft["f_nact"] = torch.where(at, nact[:, None, None], ft["f_nact"])
        ft["f_snr"] = torch.where(at, snr[..., None], ft["f_snr"])
        ft["f_own"] = torch.where(at, count[..., None], ft["f_own"])
        return acc, count + acc.long()

    def _stats_counts(self, T, cnt):
        """The statistics of a counts-form enqueue (submit_counts, or arrivals fused into the step launch): its
        submit() calls replayed one at a time, class by class and message by message, as the kernel enqueues them."""
        count, stale0 = self._stats_pre_submit(T)
        had = count > 0
        c = cnt.long()
        for ci in range(c.shape[-1]):
            for i in range(int(c[..., ci].max())):
                # the head frame is the one queued before the call, or this step's first (never stale)
                stale = torch.where(had, stale0, (count > 0) & (self.config.timeout_steps <= 0))
                _, count = self._stats_enqueue(c[..., ci] > i, count, stale, self._last_snr)

    def _stats_step(self, o):
        """Log the frames the step resolved (NRNet._log_ul / _log_dl, nr_engine.py:890-907) from its outputs (the
        queue layout before compaction), then compact the feature record as the queue was (queues.py:105-110)."""
        st, cfg, E = self.stats, self.config, self.E
        if "flags" in o:
            fl = o["flags"]
            delivered, timed, dropped = (fl & 1) != 0, (fl & 2) != 0, (fl & 4) != 0
            cap, cls = o["cap32"].long(), o["cls8"].long()
        else:
            delivered, timed, dropped, cap, cls = o["delivered"], o["timed_out"], o["dropped"], o["cap"], o["cls"]
        keep = cap + self.st["epoch"].long()[:, None, None] <= self.log_cap_max     # capture step, global clock
        dk, tk = delivered & keep, (timed | dropped) & keep
        delay = o["delay"]
        st["delay"].append(delay[dk].cpu())
        eidx = torch.arange(E, device=self.dev)[:, None, None].expand_as(cap)
        st["d_env"].append(eidx[dk].cpu())
        st["x_env"].append(eidx[tk].cpu())
        st["dropped"] += int(dropped.sum())
        st["late"] += int((dk & (delay >= cfg.timeout_steps)).sum())
        feats = {"cls": cls, **self._feat}
        for f in self.FEATS:
            st["d_" + f].append(feats[f][dk].cpu())
            st["x_" + f].append(feats[f][tk].cpu())
        order = torch.argsort((delivered | timed | dropped).to(torch.uint8), dim=-1, stable=True)
        for k, v in self._feat.items():
            self._feat[k] = torch.gather(v, -1, order)
        if self._dl_delay is not None:
            dd = self._dl_delay
            st["dl_delay"].append(dd[~torch.isnan(dd)].cpu())

    def counters(self):
        """{"ul": {counter: value, ntx_hist, rv_tx, rv_fail}} (and "dl" with the downlink) since the last full reset
        (NRNet.counters)."""
        cfg = self.config

        def link(st, n_slots):
            c = st["ctr"].sum(0).tolist()
            h = st["hist"]
            res = {k: float(c[i]) for i, k in enumerate(CTR_NAMES)}
            res["ntx_hist"] = h[:, 0].sum(0).double().tolist()
            res["rv_tx"] = h[:, 1].sum(0).double().tolist()
            res["rv_fail"] = h[:, 2].sum(0).double().tolist()
            res["prb_avail"] = float(sum(cfg.subband_prbs)) * self.E * self.C * n_slots
            if cfg.lena_mac_switches():
                res.update({k: float(c[10 + i]) for i, k in enumerate(LENA_CTR_NAMES)})
            return res
        out = {"ul": link(self.st, self._ul_slots_run)}
        if self.dl:
            out["dl"] = link(self.dst, self._dl_slots_run)
        return out

    _ul_slots_run = 0
    _dl_slots_run = 0
    # set to a KernelTimer to record HIP events around every (UL / DL) step-kernel launch, on the launch stream
    kernel_events = None
    dl_kernel_events = None

    # ------------------------------------------------------------------ state in the reference's layout
    def _link_sd(self, pre, st):
        """The MacLink / FrameQueue keys of one link ("ul" or "dl") in the reference's names and layouts."""
        cfg, N = self.config, self.N
        L = lambda x: x.long()  # noqa: E731
        rs = lambda x: x.permute(0, 2, 1)  # noqa: E731
        meta = st["h_meta"]
        po = cfg.proc_offset_ms / cfg.control_step_ms
        fin_slot = st["q_fin"].long()
        tf = torch.div(fin_slot, N, rounding_mode="floor")
        fin = (tf.double() + (fin_slot - tf * N + 1).double() / N) + po
        fin = torch.where(fin_slot == BIG_SLOT, torch.full_like(fin, math.inf), fin)
        qm = st["q_meta"]
        b = st["base"]                                # the int64 offsets are base + the int32 values
        bq = b[:, :, None]
        out = {
            "sent": L(st["sent"]) + b, "floor": L(st["floor_"]) + b, "olla": st["olla"], "avg": st["avg"],
            "csi": rs(st["csi"]),
            "h_state": rs(L(meta & 0xFF)), "h_ntx": rs(L((meta >> 8) & 0xFF)), "h_mcs": rs(L((meta >> 16) & 0xFF)),
            "h_nsb": rs(L((meta >> 24) & 0xFF)), "h_lo": rs(L(st["h_lo"])) + bq, "h_hi": rs(L(st["h_hi"])) + bq,
            "h_ready": rs(L(st["h_ready"])), "h_tbs": rs(L(st["h_tbs"])), "h_comb": rs(st["h_comb"]),
            "h_lexp": rs(st["h_lexp"]), "h_nrb": rs(st["h_nrb"]), "last_tx": L(st["last_tx"]),
            "q.cap": rs(L(st["q_cap"])), "q.start": rs(L(st["q_start"])) + bq, "q.end": rs(L(st["q_end"])) + bq,
            "q.lost": rs((qm & 1) != 0), "q.fin": rs(fin), "q.cls": rs(L((qm >> 8) & 0xFF)),
            "q.enq": L(st["enq"]) + b,
        }
        if pre == "ul":
            out.update({"bsr": L(st["bsr"]), "sr_t": L(st["sr_t"]), "q.det": rs((qm & 2) != 0),
                        "q.hid": rs(L(st["q_hid"]))})
            if cfg.ul_amc_alloc == "previous":        # UlMac AMC_STATE (mac_ul.py:51)
                out["last_nprb"] = st["last_nprb"]
        else:                                         # the DL link holds no BSR / SR state (constant initial values)
            out.update({"bsr": torch.zeros_like(out["sent"]), "sr_t": torch.full_like(out["sent"], -1)})
        return {f"{pre}.{k}": v for k, v in out.items()}

    def owner_state(self):
        """Every state tensor under the reference's owner keys ("ul.sent", "net.h", "eng.epoch", "rng.ctr[2]": the
        equivalence-test form of isaac_net/core/nr_fast.py:41-75, state_dict(eng)), reference shapes and dtypes, on
        the engine's device. Frame fields of empty queue slots are unspecified (the reference leaves stale values)."""
        st, cfg = self.st, self.config
        L = lambda x: x.long()  # noqa: E731
        rs = lambda x: x.permute(0, 2, 1)  # noqa: E731
        out = self._link_sd("ul", st)
        E, R, S = self.E, self.R, self.S
        hh = lambda x: rs(x).reshape(E, R, self.C, S) if self.C > 1 else rs(x)  # noqa: E731
        out.update({
            "net.h": torch.stack([hh(st["h_re"]), hh(st["h_im"])], -1), "eng.epoch": L(st["epoch"]),
            "eng._last_snr": self._last_snr, "eng._last_hid": self._last_hid,
            "rng.episode": L(st["episode"]), "rng.ctr[1]": L(st["ctr_submit"]), "rng.ctr[2]": L(st["ctr_step"]),
        })
        if self.dl:
            out.update(self._link_sd("dl", self.dst))
            out["net.dl_newest"] = L(self.dst["newest"])
        if self.C > 1:                                # CellAssociation and NRNet._reset_cells state
            c = self.cst
            out.update({"assoc." + n: L(c[n]) for n in ("serv", "a3_cand", "a3_cnt", "ho_end", "n_ho")})
            out["assoc.pending"] = c["pending"] != 0
            if cfg.rlf:
                out.update({"assoc." + n: L(c[n]) for n in RLF_KEYS})
                out["assoc.rlf_active"] = c["rlf_active"] != 0
                out.update({f"assoc.ctr[{k}]": c["rlf_ctr"][:, i].sum() for i, k in enumerate(RLF_CTR)})
            out["net.ni_ul"] = c["ni_ul"]
            out["net.ioN[ul]"] = c["ion"]
        if cfg.rician_mode in ("fixed", "los"):
            # (between steps the input K is the target; a fixed K never ramps: ramp start = target, k_g0 0)
            rv = (lambda x: x[:, 0]) if self.C == 1 else (lambda x: x.permute(0, 2, 1))   # [E,R] / [E,R,C]
            k = rv(st["k_lin"])
            out.update({"net.spec": torch.stack([rv(st["spec_re"]), rv(st["spec_im"])], -1), "net.k_in": k,
                        "net.k_lin": k})
            if cfg.rician_mode == "los":
                out.update({"net.k_los": rv(st["k_los"]), "net.k_from": rv(st["k_from"]), "net.k_g0": L(rv(st["k_g0"])),
                            "net.k_fresh": st["k_fresh"] != 0})
            else:
                out.update({"net.k_los": k, "net.k_from": k, "net.k_g0": torch.zeros_like(L(k))})
        if cfg.freq_corr_mode == "los":
            rv = (lambda x: x[:, 0]) if self.C == 1 else (lambda x: x.permute(0, 2, 1))   # [E,R] / [E,R,C]
            out.update({"net.fc_idx": L(rv(st["fc_idx"])), "net.fc_idx_los": L(rv(st["fc_idl"])),
                        "net.fc_idx_nlos": L(rv(st["fc_idn"]))})
        if cfg.fading_doppler == "per_robot":
            out["net.fading_rho_ms"] = st["rho_ms"]
        return out

    def _link_load(self, pre, st, sd):
        """Load one link's keys of a reference-layout state dict into its device buffers."""
        cfg, N, d = self.config, self.N, self.dev
        g = lambda k: torch.as_tensor(sd[f"{pre}.{k}"]).to(d)  # noqa: E731
        rs = lambda x: x.permute(0, 2, 1).contiguous()  # noqa: E731
        I = lambda x: x.to(torch.int32)  # noqa: E731
        # the int64 byte offsets as base + int32 values: the base is the floor once that reaches REBASE_AT
        base, rel = split_offsets(g("floor").long(), g("sent").long(), g("q.enq").long(), self.REBASE_AT)
        st["base"].copy_(base)
        bq = base[:, :, None]
        st["floor_"].copy_(I(rel(g("floor"))))
        st["sent"].copy_(I(rel(g("sent"))))
        st["enq"].copy_(I(rel(g("q.enq"))))
        pairs = (("last_tx", "last_tx"),)
        if pre == "ul":
            pairs += (("bsr", "bsr"), ("sr_t", "sr_t"))
        for a, b in pairs:
            st[a].copy_(I(g(b)))
        if pre == "ul" and cfg.ul_amc_alloc == "previous" and f"{pre}.last_nprb" in sd:
            st["last_nprb"].copy_(g("last_nprb").float())
        st["olla"].copy_(g("olla"))
        st["avg"].copy_(g("avg"))
        st["csi"].copy_(rs(g("csi")))
        meta = (g("h_state") | (g("h_ntx") << 8) | (g("h_mcs") << 16) | (g("h_nsb") << 24))
        st["h_meta"].copy_(rs(I(meta)))
        for a in ("h_lo", "h_hi"):                  # (a free process's stale range: at most 2^30 below the base)
            st[a].copy_(rs(I((g(a).long() - bq).clamp(-(1 << 30), (1 << 31) - 1))))
        for a in ("h_ready", "h_tbs"):
            st[a].copy_(rs(I(g(a))))
        for a in ("h_comb", "h_lexp", "h_nrb"):
            st[a].copy_(rs(g(a).float()))
        cap = g("q.cap")
        valid = cap >= 0
        st["qlen"].copy_(I(valid.sum(-1)))
        st["q_cap"].copy_(rs(I(torch.where(valid, cap, torch.full_like(cap, -1)))))
        for a, k in (("q_start", "q.start"), ("q_end", "q.end")):      # (empty slots keep their stale values)
            st[a].copy_(rs(I((g(k).long() - bq).clamp(-(1 << 30), (1 << 31) - 1))))
        po = cfg.proc_offset_ms / cfg.control_step_ms
        fin = g("q.fin").double()
        slot = torch.round((fin - po) * N).long() - 1
        slot = torch.where(torch.isinf(fin) | ~valid, torch.full_like(slot, BIG_SLOT), slot)
        st["q_fin"].copy_(rs(I(slot)))
        qm = g("q.lost").long() | (g("q.cls").long() << 8)
        if pre == "ul":
            qm = qm | (g("q.det").long() << 1)
            st["q_hid"].copy_(rs(I(g("q.hid"))))
        st["q_meta"].copy_(rs(I(qm)))

    def load_owner_state(self, sd, T=None, last_g=None):
        """Load owner-key state (the keys of owner_state(); tensors on any device) into the device buffers; T / last_g
        set the host clock and the last fading slot (teacher forcing)."""
        st, cfg, d = self.st, self.config, self.dev
        g = lambda k: torch.as_tensor(sd[k]).to(d)  # noqa: E731
        rs = lambda x: x.permute(0, 2, 1).contiguous()  # noqa: E731
        I = lambda x: x.to(torch.int32)  # noqa: E731
        self._link_load("ul", st, sd)
        if self.dl:
            self._link_load("dl", self.dst, sd)
            self.dst["newest"].copy_(I(g("net.dl_newest")))
        h = g("net.h")
        if self.C > 1:                                # [E,R,C,S,2] -> [E][C S][R]
            h = h.reshape(self.E, self.R, self.C * self.S, 2)
        st["h_re"].copy_(rs(h[..., 0]))
        st["h_im"].copy_(rs(h[..., 1]))
        if self.C > 1:
            c = self.cst
            for n in ("serv", "a3_cand", "a3_cnt", "ho_end", "n_ho") + (("rlf_active",) + RLF_KEYS if cfg.rlf else ()):
                c[n].copy_(I(g("assoc." + n)))
            if cfg.rlf:                               # the counters: totals on env 0
                rc = torch.zeros_like(c["rlf_ctr"])
                for i, k in enumerate(RLF_CTR):
                    if f"assoc.ctr[{k}]" in sd:
                        rc[0, i] = int(torch.as_tensor(sd[f"assoc.ctr[{k}]"]))
                c["rlf_ctr"].copy_(rc)
            c["pending"].copy_(I(g("assoc.pending")))
            c["ni_ul"].copy_(g("net.ni_ul").float())
            c["ion"].copy_(g("net.ioN[ul]").float())
        st["epoch"].copy_(I(g("eng.epoch")))
        st["episode"].copy_(I(g("rng.episode")))
        st["ctr_submit"].copy_(I(g("rng.ctr[1]")))
        st["ctr_step"].copy_(I(g("rng.ctr[2]")))
        if cfg.rician_mode in ("fixed", "los"):
            sp = g("net.spec")
            lv = (lambda v: v[:, None]) if self.C == 1 else (lambda v: v.permute(0, 2, 1))   # -> [E,C,R]
            st["spec_re"].copy_(lv(sp[..., 0]))
            st["spec_im"].copy_(lv(sp[..., 1]))
            st["k_lin"].copy_(lv(g("net.k_lin")))
            if cfg.rician_mode == "los":
                st["k_los"].copy_(lv(g("net.k_los")))
                st["k_from"].copy_(lv(g("net.k_from")))
                st["k_g0"].copy_(lv(I(g("net.k_g0"))))
                fr = sd.get("net.k_fresh")
                st["k_fresh"].copy_(I(torch.as_tensor(fr).to(self.dev)) if fr is not None else 0)
        if cfg.freq_corr_mode == "los":
            G = int(cfg.fading_ds_grid[2])
            lv = (lambda v: v[:, None]) if self.C == 1 else (lambda v: v.permute(0, 2, 1))   # -> [E,C,R]
            for n, k in (("fc_idx", "net.fc_idx"), ("fc_idl", "net.fc_idx_los"), ("fc_idn", "net.fc_idx_nlos")):
                v = g(k)
                if bool(((v < 0) | (v >= G)).any()):
                    raise ValueError(f"{k}: grid indices outside [0, {G})")
                st[n].copy_(lv(I(v)))
        if cfg.fading_doppler == "per_robot" and "net.fading_rho_ms" in sd:
            st["rho_ms"].copy_(g("net.fading_rho_ms").float())
        self._last_snr = g("eng._last_snr").float().clone()
        self._last_hid = g("eng._last_hid").long().clone()
        if T is not None:
            self.T = int(T)
            ep = st["epoch"]
            self._uniform_epoch = int(ep[0]) if bool((ep == ep[0]).all()) else None
        self.last_g = last_g


    # ------------------------------------------------------------------ checkpoints (core/checkpoint.py:103-143)
    _CK_ENG = {"eng.epoch": "epoch", "eng._last_snr": "_last_snr", "eng._last_hid": "_last_hid",
               "rng.episode": "net.rng.episode", "rng.ctr[1]": "net.rng.ctr[1]", "rng.ctr[2]": "net.rng.ctr[2]"}

    def _ck_key(self, k):
        """Owner key -> the key of the reference's checkpoint (the attribute path from NREngine)."""
        if k.startswith(("ul.", "dl.", "assoc.")):
            return "net." + k
        return self._CK_ENG.get(k, k)

    def _field_keys(self):
        """[(checkpoint key prefix, field index)] of the radio's shadowing fields (RadioMC / TR38901Channel)."""
        if self._n_fields == 3:
            return [("radio.ch.sf_los", 0), ("radio.ch.sf_nlos", 1), ("radio.ch.los_field", 2)]
        return [("radio", 0)] if self._n_fields == 1 else []

    def state_dict(self):
        """The engine's checkpoint: a flat {key: tensor | host value} under the keys of the reference engine's
        state_dict (core/checkpoint.py collect on NREngine: "net.ul.sent", "net.rng.ctr[2]", "radio.ch.sf_los.k",
        "T", ...) for the state this engine keeps; counters as the reference keeps them (totals, per-env PRBs and
        HARQ histograms). Tensors are snapshots (clones) on the engine's device."""
        cfg, st, E = self.config, self.st, self.E
        out = {self._ck_key(k): v.clone() for k, v in self.owner_state().items()}
        out["net.rng.env"] = st["env_id"].long().clone()
        if self._feat is not None:                 # the queued frames' features, kept while log_stats is on
            out.update({f"net.ul.q.{k}": v.clone() for k, v in self._feat.items()})
        for pre, fi in self._field_keys():
            f = st["field"][:, :, fi].permute(1, 0, 2, 3)          # [C, E, K, 3]
            out[pre + ".k"] = f[..., :2].clone()
            out[pre + ".phi"] = f[..., 2].clone()
        links = [("ul", st, self._ul_slots_run)] + ([("dl", self.dst, self._dl_slots_run)] if self.dl else [])
        for name, ls, n_slots in links:
            c = ls["ctr"]
            for i, k in enumerate(CTR_NAMES):
                out[f"net.{name}.ctr[{k}]"] = c[:, i].sum().float()
            if cfg.lena_mac_switches():
                for i, k in enumerate(LENA_CTR_NAMES):
                    out[f"net.{name}.ctr[{k}]"] = c[:, 10 + i].sum().float()
            out[f"net.{name}.ctr[prb_avail]"] = torch.tensor(float(sum(cfg.subband_prbs)) * E * self.C * n_slots,
                                                             device=self.dev)
            h = ls["hist"].float()
            out[f"net.{name}.ntx_hist"] = h[:, 0].sum(0)
            out[f"net.{name}.rv_tx"] = h[:, 1].clone()
            out[f"net.{name}.rv_fail"] = h[:, 2].clone()
            out[f"net.{name}.prb_used_env"] = c[:, 9].float()
        if cfg.fading_doppler == "per_robot":          # the radio's last poses (radio.py:194-195)
            out["radio.prev_pos"] = st["prev_pos"].clone()
            out["radio.has_prev"] = st["has_prev"] != 0
            out["per_robot_doppler"] = True
        out.update({"T": int(self.T), "net.last_g": self.last_g, "_uniform_epoch": self._uniform_epoch,
                    "E": E, "R": self.R, "F": self.F, "seed": self.seed,
                    "net.rng.s0": int(self._cparams.seed_key) & M32})
        return out

    # Reference checkpoint keys that hold no state here: torch generators (the engine's draws are counter based),
    # values derived from the config, the reference's per-step caches (recomputed every step) and statistics buffers.
    _CK_SKIP = {"gen", "net.gen", "radio.gen", "net.rng._zero", "net.sizes", "radio._sizes", "radio.gnb", "radio.gnb3",
                "radio.ch.gnb", "radio.ch.los", "radio.has_prev", "radio.prev_pos", "radio.speed", "net.refused_env",
                "net._gain_c", "net._ni_la_ul", "net._pg", "net.ul.member", "net.ul.pc_backoff", "net.ul.phr_snr",
                "net.ul.sched_ok", "net.ioN[dl]", "net.ni_dl", "net.ul.sb_prb", "net.dl.sb_prb", "net.ul.q.f_nact",
                "net.ul.q.f_snr", "net.ul.q.f_own", "net.dl.q.f_nact", "net.dl.q.f_snr", "net.dl.q.f_own",
                "net.dl.q.det", "net.dl.q.hid", "net.dl_newest",
                "net.fc_L", "net.fc_tab", "net.fc_grid_ns"}   # (the subband correlations' square roots: config)
    # Reference host values that switch on what this engine does not run (traffic models, access procedures, hooks
    # and traces, frequency-correlated or per-robot fading, blockage, O2I, radio link failure, TPC, BSR grants,
    # MIMO, QoS): a checkpoint holding another value was written with that feature on. (_lena_mac, the LENA grant
    # counters' switch, must equal this config's: _ck_expected.)
    _CK_OFF = {"_gate": None, "_dl_gate": None, "_los_fn": None, "access": None, "_extras": False, "traffic": None,
               "traffic_dl": None, "per_robot_doppler": False, "net.fc_mode": None, "net.trace_frames": None,
               "net.trace_frames_dl": None, "net._user_hook[ul]": None, "net._user_hook[dl]": None,
               "net.assoc.rlf": False, "radio._blocked": None, "radio.blk_a": None, "radio.obstacle_outputs": False,
               "radio.white": None, "radio.ch.o2i": False, "radio.ch.soft": False,
               **{f"net.{lk}.{k}": v for lk in ("ul", "dl") for k, v in (
                   ("slot_hook", None), ("sinr_hook", None), ("trace", None), ("mimo", False), ("qos", False),
                   ("_tpc", False), ("_bsr_model", False), ("_lena_mac", False), ("_occ", None))}}

    def _ck_expected(self, k):
        """The value host switch k must hold in a checkpoint this engine loads."""
        cfg = getattr(self, "config", None)
        if k.endswith("._lena_mac"):
            return bool(cfg.lena_mac_switches()) if cfg is not None else False
        if k == "net.fc_mode":
            return cfg.freq_corr_mode if cfg is not None else None
        if k == "per_robot_doppler":
            return cfg is not None and cfg.fading_doppler == "per_robot"
        if k == "net.assoc.rlf":
            return cfg is not None and bool(cfg.rlf) and cfg.n_cells > 1
        return self._CK_OFF[k]

    def _strict_extra_keys(self, sd, used):
        """strict loading: the state keys of sd that are neither restored (used) nor known to hold no state here,
        and the host switches that are on."""
        bad = []
        for k, v in sd.items():
            if k in used or k in self._CK_SKIP or k.endswith(".gen"):
                continue
            if torch.is_tensor(v) or isinstance(v, np.ndarray):
                bad.append(k)
            elif k in self._CK_OFF:
                want = HipNREngine._ck_expected(self, k)
                if v != want and not (v is None and want is False):
                    bad.append(f"{k}={v!r}")
        return bad

    def load_state_dict(self, sd, strict=True, T=None, last_g=None):
        """Restore a checkpoint in place: this engine's state_dict(), or the reference engine's (the same keys;
        keys of the reference that hold no state here are skipped: torch generators, trace hooks, statistics, the
        queue's f_nact / f_snr / f_own fields unless log_stats is on, host configuration values). Per-env counters come back as the
        reference keeps them: totals (on env 0) and per-env PRBs and HARQ histograms. strict: raise if state this
        engine keeps is missing or has another shape. The owner-key form of owner_state() is accepted too (with
        T / last_g as in load_owner_state). Returns self."""
        if "ul.sent" in sd and "net.ul.sent" not in sd:
            self.load_owner_state(sd, T=T, last_g=last_g)
            return self
        cfg, st, d = self.config, self.st, self.dev
        mine = self.owner_state()
        owner, missing = {}, []
        used = {"net.rng.env", "net.rng.s0", "T", "net.last_g", "_uniform_epoch"}
        for k, v in mine.items():
            ck = self._ck_key(k)
            used.add(ck)
            if ck in sd:
                val = torch.as_tensor(sd[ck])
                if strict and tuple(val.shape) != tuple(v.shape):
                    raise KeyError(f"load_state_dict: {ck} has shape {tuple(val.shape)}, the engine {tuple(v.shape)}")
                owner[k] = val
            elif k.endswith((".bsr", ".sr_t")) and k.startswith("dl."):
                owner[k] = v                                 # constant in the DL link
            else:
                missing.append(ck)
        if missing:
            if strict:
                raise KeyError("load_state_dict: missing from the state dict: " + ", ".join(missing))
            for k, v in mine.items():
                owner.setdefault(k, v)
        g = lambda k: torch.as_tensor(sd[k]).to(d)  # noqa: E731
        for pre, _ in self._field_keys():
            used.update((pre + ".k", pre + ".phi"))
        for name in ("ul", "dl"):
            used.update(f"net.{name}.{k}" for k in ("ntx_hist", "rv_tx", "rv_fail", "prb_used_env"))
            used.update(f"net.{name}.ctr[{k}]" for k in CTR_NAMES + ("prb_avail",) +
                        (LENA_CTR_NAMES if cfg.lena_mac_switches() else ()))
        if strict:
            bad = self._strict_extra_keys(sd, used)
            if bad:
                raise KeyError("load_state_dict: state this engine does not run (strict): " + ", ".join(bad[:12]))
        if "net.rng.env" in sd:
            st["env_id"].copy_(g("net.rng.env").to(torch.int32))
        if cfg.fading_doppler == "per_robot" and "radio.prev_pos" in sd and "radio.has_prev" in sd:
            st["prev_pos"].copy_(g("radio.prev_pos").float())
            st["has_prev"].copy_(g("radio.has_prev").to(torch.int32))
        for pre, fi in self._field_keys():
            if pre + ".k" in sd:
                st["field"][:, :, fi, :, :2].copy_(g(pre + ".k").permute(1, 0, 2, 3))
                st["field"][:, :, fi, :, 2].copy_(g(pre + ".phi").permute(1, 0, 2))
            elif strict:
                raise KeyError(f"load_state_dict: missing from the state dict: {pre}.k")
        if "net.rng.s0" in sd:
            s0 = int(sd["net.rng.s0"])
            self._cparams.seed_key = C.c_int32(s0 - (1 << 32) if s0 >= 1 << 31 else s0).value
        links = [("ul", st)] + ([("dl", self.dst)] if self.dl else [])
        for name, ls in links:
            if f"net.{name}.ctr[tb_new]" not in sd:
                continue
            c = torch.zeros_like(ls["ctr"])
            for i, k in enumerate(CTR_NAMES):
                c[0, i] = int(round(float(sd[f"net.{name}.ctr[{k}]"])))
            for i, k in enumerate(LENA_CTR_NAMES):
                if f"net.{name}.ctr[{k}]" in sd:
                    c[0, 10 + i] = int(round(float(sd[f"net.{name}.ctr[{k}]"])))
            if f"net.{name}.prb_used_env" in sd:
                c[:, 9] = g(f"net.{name}.prb_used_env").round().long()
            ls["ctr"].copy_(c)
            h = torch.zeros_like(ls["hist"])
            h[0, 0] = g(f"net.{name}.ntx_hist").round().long()
            h[:, 1] = g(f"net.{name}.rv_tx").round().long()
            h[:, 2] = g(f"net.{name}.rv_fail").round().long()
            ls["hist"].copy_(h)
            w = float(sum(cfg.subband_prbs)) * self.E * self.C
            n_slots = int(round(float(sd[f"net.{name}.ctr[prb_avail]"]) / w))
            if name == "ul":
                self._ul_slots_run = n_slots
            else:
                self._dl_slots_run = n_slots
        if "T" in sd:
            T = int(sd["T"])
        elif strict:
            raise KeyError("load_state_dict: missing from the state dict: T")
        self.load_owner_state(owner, T=T, last_g=sd.get("net.last_g", last_g))
        if "_uniform_epoch" in sd:
            self._uniform_epoch = sd["_uniform_epoch"]
        if self._feat is not None:                 # with log_stats on: the queued frames' features
            for k, v in self._feat.items():
                if f"net.ul.q.{k}" in sd:
                    self._feat[k] = g(f"net.ul.q.{k}").to(v.dtype).reshape(v.shape).clone()
        return self


def set_env_offset(engine, offset):
    """The engine's env rows keyed by global env id offset + local id (sharded.set_env_offset,
    isaac_net/core/sharded.py:61-78): HipNREngine / HipWifiEngine.set_env_offset."""
    engine.set_env_offset(offset)


def state_dict(eng):
    """{owner key: tensor} of every state tensor of a hip NR engine: the form of the reference's
    nr_fast.state_dict(eng) (isaac_net/core/nr_fast.py:61-67), used by the equivalence tests."""
    return eng.owner_state()


# the radio link failure state of CellAssociation kept per robot (radio.py:340-342; rlf_active is a bool) and its
# counters (radio.py:342)
RLF_KEYS = ("oos_cnt", "is_cnt", "t310_end", "t311_end", "reest_end", "reest_cell", "n_rlf")
RLF_CTR = ("rlf", "reest", "rlf_idle", "t310_start", "t310_stop")


class GraphStep:
    """submit_counts + step of a HipNREngine as HIP graphs (torch.cuda.CUDAGraph), recorded on first use and replayed
    at every control step: one graph for the enqueue, and one step graph per slot schedule (TDD / SR / CQI phase and
    fading slot spacing) and input kind, as the reference's graph backend keeps one captured step per key
    (isaac_net/core/nr_fast.py:435-489). The step graph holds the downlink step before the uplink one with
    NRConfig(dl=True) (DL frames are enqueued eagerly with add_dl_frames, as the reference's fast engine enqueues them
    outside its graph) and the several-cells step with n_cells > 1.

    The recorded launches read the control step from the engine's device clock (InetNrState.clock), which the
    replay sets to the engine's T; the inputs are copied into static buffers; the returned dict is the step graph's
    static output buffers, overwritten by its next replay. The graphs hold kernel nodes only (no memset node).
    With log_stats on, the statistics of the enqueue and of the resolved frames are taken around the replays."""

    def __init__(self, eng, n_cls):
        E, R, dev = eng.E, eng.R, eng.dev
        self.eng = eng
        self.counts = torch.zeros(E, R, n_cls, dtype=torch.uint8, device=dev)
        self.inputs = {}                      # input kind -> static input buffer
        self.vel = None                       # per-robot Doppler: the static velocity input [E,R,2]
        self.steps = {}                       # (schedule key incl. the kind, DL delay buffer, vel) -> (graph, outputs)
        eng.st["clock"].fill_(eng.T)
        torch.cuda.synchronize(dev)
        self.g_submit = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.g_submit):
            eng._launch_submit_counts(-1, self.counts)
        self.hid = eng._last_hid              # the submit graph's hazard ids (zeros), read by the step graphs
        torch.cuda.synchronize(dev)

    def _record(self, plan, kind, use_vel):
        eng = self.eng
        x = self.inputs[kind]
        torch.cuda.synchronize(eng.dev)
        g = torch.cuda.CUDAGraph()
        ev, dev_ = eng.kernel_events, eng.dl_kernel_events
        eng.kernel_events = eng.dl_kernel_events = None
        eng._cparams.vel = self.vel.data_ptr() if use_vel else None
        try:
            with torch.cuda.graph(g):
                out = eng._launch_step(-1, plan, x, self.hid, (kind, x, 1) if eng.dl else None)
        finally:
            eng.kernel_events, eng.dl_kernel_events = ev, dev_
            eng._cparams.vel = None
        torch.cuda.synchronize(eng.dev)
        return g, out

    def __call__(self, x=None, counts=None, *, snr_db=None, vel=None, pathgain_db=None):
        """One control step: counts [E,R,NC] uint8 messages per class (as submit_counts), then the step on poses
        x [E,R,2|3], SNR x [E,R] or snr_db= [E,R,S] (with the downlink: its reference from the same input), or with
        several cells pathgain_db= [E,R,C]; vel= [E,R,2|3] the velocity input of per-robot Doppler (as step)."""
        eng = self.eng
        T = eng.T
        if pathgain_db is not None and eng.C == 1:
            raise ValueError("pathgain_db= needs config.n_cells > 1")
        kind, xin = eng._input(x, snr_db, pathgain_db)
        eng._check_kind(kind)
        vin = eng._vel_input(vel, kind)
        if vin is not None:
            if self.vel is None:
                self.vel = torch.empty_like(vin)
            self.vel.copy_(vin)
        if counts is None or tuple(counts.shape) != tuple(self.counts.shape):
            raise ValueError(f"counts must be {tuple(self.counts.shape)}")
        if kind not in self.inputs:
            self.inputs[kind] = torch.empty_like(xin)
        self.inputs[kind].copy_(xin)
        plan = eng._plan(T, kind)
        key = (plan["key"], 0 if eng._dl_delay is None else eng._dl_delay.data_ptr(), vin is not None)
        hit = self.steps.get(key)
        if hit is None:
            hit = self.steps[key] = self._record(plan, kind, vin is not None)
        g, out = hit
        self.counts.copy_(counts)
        eng.st["clock"].fill_(T)
        if eng._log_stats:
            eng._stats_counts(T, self.counts)
        self.g_submit.replay()
        eng._last_hid = self.hid
        ev = eng.kernel_events
        if ev is not None:
            ev.begin(torch.cuda.current_stream(eng.dev))
        g.replay()
        if ev is not None:
            ev.end(torch.cuda.current_stream(eng.dev))
        if eng._log_stats:
            eng._stats_step(out)
        eng._commit(T, plan, out)
        return out


class KernelTimer:
    """Timing events recorded around each step-kernel launch on the launch stream (an engine's kernel_events hook).
    The n event pairs are created and recorded once here: a HIP event is created on its first record, which can
    cost more than the launch it brackets, so none is created inside a timed loop."""

    def __init__(self, n, device="cuda"):
        self.pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        stream = torch.cuda.current_stream(device)
        for a, b in self.pairs:
            a.record(stream)
            b.record(stream)
        torch.cuda.synchronize(device)
        self.n = 0

    def begin(self, stream):
        if self.n >= len(self.pairs):
            raise RuntimeError(f"KernelTimer: more than {len(self.pairs)} timed launches")
        self.pairs[self.n][0].record(stream)

    def end(self, stream):
        self.pairs[self.n][1].record(stream)
        self.n += 1

    def ms(self):
        """Duration of every timed launch in ms (after the stream has been synchronized)."""
        return [a.elapsed_time(b) for a, b in self.pairs[:self.n]]


def make_engine(level, E, R, device="cuda", config: NRConfig | None = None, backend="hip", *, sizes=None,
                params=None, seed=None, inject=False, strict=False, out_format="reference"):
    """Factory with the signature of isaac_net.core.engine.make_engine (engine.py:230-255) for level "L2" (the NR
    engine) and level "WIFI" (isaac_net/core/wifi/engine.py:436-444), backend "hip" (also "auto", which resolves to
    "hip" on a GPU device)."""
    if level not in ("L2", "WIFI", "WIFI_DCF"):
        raise HipUnsupported(f"level {level!r}: the hip backend implements levels 'L2' (NR), 'WIFI' and "
                             "'WIFI_DCF'")
    if backend not in ("hip", "auto"):
        raise ValueError(f"unknown backend {backend!r} for this package; use 'hip'")
    if inject:
        raise HipUnsupported("inject=True (externally fed draws) is not implemented; the engine RNG is used")
    cfg = config if config is not None else NRConfig()
    if sizes is not None:
        cfg = cfg.with_(msg_sizes=tuple(float(s) for s in sizes))
    if seed is None:
        seed = cfg.seed
    if level == "WIFI":
        from .wifi_engine import HipWifiEngine
        return HipWifiEngine(E, R, device, cfg, seed=seed)
    if level == "WIFI_DCF":
        from .wifi_engine import HipWifiDcfEngine
        return HipWifiDcfEngine(E, R, device, cfg, seed=seed)
    return HipNREngine(E, R, device, cfg, seed=seed, out_format=out_format)

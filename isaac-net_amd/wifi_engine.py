"""HipWifiEngine: level "WIFI" (the mean-field 802.11 uplink at one or several access points on one channel) over the
HIP kernels of libinet_nr.so (include/inet_wifi.h).

Mirrors isaac_net/core/wifi/engine.py (WifiNet, :100-403) on the LevelNet contract (isaac_net/core/levels/base.py:43-360):
reset(env_ids) / submit(t, requests, snr_db) / step(t, poses_or_snr, cur_hid, *, rx_dbm) -> dict / clock /
state_dict, with the same inputs, output keys, dtypes and shapes and the same per-env clock rules (t=None uses the
engine clock; an int or an [E] tensor sets each env's step). What the kernels do not implement is refused at
construction with HipUnsupported: more than 8 APs, APs on several channels when R + A > 64 or (R + A) x channels
>= 400, AIFS zones (access categories of different AIFSN in one env) when R + A > 64, hidden nodes when
(R + A)^2 >= 400, rng="global", and the radio features the NR engine refuses. Several APs run with association and
roaming, on one channel or several (one collision domain per channel), with or without AIFS zones and hidden
nodes.

All state lives in device tensors that torch allocates; every call hands the library plain pointers.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import torch

from . import _lib
from .config import NRConfig
from .engine import HipUnsupported, Requests, seed_key
from .wifi_config import PPDU_MAX_US, WifiConfig, derive, radio_config

OUT_KEYS = ("newest", "det_env", "delivered", "timed_out", "cap", "cls", "delay", "queue_len", "queue_bytes",
            "sinr_db", "t", "serving_cell", "wifi_mcs", "wifi_rate_mbps", "wifi_access_ms", "wifi_p_fail",
            "wifi_busy")


def wifi_refusals(cfg: NRConfig):
    """[(feature, why)] of the config's features the HIP Wi-Fi kernels do not implement (empty: it runs)."""
    wc = cfg.wifi if cfg.wifi is not None else WifiConfig()
    out = []

    def no(cond, what, why):
        if cond:
            out.append((what, why))
    n_ap = len(wc.ap_xy(cfg))
    no(n_ap > 8, f"{n_ap} access points", "up to 8 APs per env")
    d = derive(cfg, wc)
    no(d.Z > 6, f"{d.Z} AIFS zones", "AIFSN differences up to 5 (six zones)")
    no(cfg.rng != "engine", "rng='global'", "counter-based engine RNG")
    no(cfg.traffic is not None, "traffic models (NRConfig.traffic)", "messages through submit()")
    no(cfg.frame_buffer > 64, "frame_buffer > 64", "FIFO columns of up to 64 slots in LDS")
    no(wc.max_tx > 16, "max_tx > 16", "up to 16 backoff stages")
    no(len(cfg.msg_sizes) > 16, "more than 16 message classes", "16 classes")
    no(d.n_acc_max > 128, "a Poisson support above 128 accesses per sub-step", "substep_ms too long for the table")
    no(len(d.rates) > 16, "more than 16 MCS", "16 table entries")
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
    no(cfg.shadow_modes > 16, "shadow_modes > 16", "up to 16 plane waves")
    return out


class HipWifiEngine:
    """Level WIFI on MI355X. API of isaac_net.core.wifi.engine.WifiNet (levels/base.LevelNet)."""

    level = "WIFI"
    backend = "hip"

    def __init__(self, E, R, device="cuda", cfg: NRConfig | None = None, seed=None, envs_per_wave=None):
        cfg = cfg if cfg is not None else NRConfig()
        if cfg.wifi is not None and not isinstance(cfg.wifi, WifiConfig):
            raise TypeError("NRConfig.wifi must be a WifiConfig")
        no = wifi_refusals(cfg)
        if no:
            raise HipUnsupported("the hip backend of level WIFI does not implement "
                                 + "; ".join(f"{f} ({why})" for f, why in no))
        dev = torch.device(device)
        if dev.type != "cuda":
            raise ValueError("the hip backend needs a GPU device (cuda:N on ROCm)")
        if not 1 <= R <= 64:
            raise HipUnsupported(f"R={R}: one env's robots share one 64-lane wavefront segment (1 <= R <= 64)")
        self._lib = _lib.load()
        self.E, self.R, self.dev, self.config = E, R, dev, cfg
        self.wc = cfg.wifi if cfg.wifi is not None else WifiConfig()
        if seed is None:
            seed = cfg.seed if cfg.seed is not None else int(torch.randint(0, 2 ** 62, ()).item())
        self.seed = int(seed)
        self.F, self.TIMEOUT = cfg.frame_buffer, cfg.timeout_steps
        self.d = derive(cfg, self.wc)
        self.K = self.Ksub = self.d.K
        self.n_acc_max = self.d.n_acc_max
        self.A = len(self.wc.ap_xy(cfg))                 # access points, one background station each
        chans = self.wc.channels(self.A)
        uniq = sorted(set(chans))
        self._ap_dom = [uniq.index(c) for c in chans]     # each AP's collision domain (wifi/engine.py:119-122)
        self.D = len(uniq)
        if self.D > 1 and (R + self.A > 64 or (R + self.A) * self.D >= 400):
            raise HipUnsupported(f"APs on {self.D} channels with R + A = {R + self.A}: several collision domains "
                                 "need R + A <= 64 and (R + A) x channels < 400")
        if self.d.Z > 1 and R + self.A > 64:
            raise HipUnsupported(f"AIFS zones with R + A = {R + self.A}: every station needs a lane of its own "
                                 "(R + A <= 64)")
        if self.wc.hidden_nodes and (R + self.A) ** 2 >= 400:
            raise HipUnsupported(f"hidden nodes with R + A = {R + self.A}: (R + A)^2 < 400, the size up to which the "
                                 "reference's sensing-matrix products add in index order")
        rb = 1 << max(0, (R - 1).bit_length())
        self.envs_per_wave = int(envs_per_wave) if envs_per_wave is not None else 1
        if self.envs_per_wave < 1 or self.envs_per_wave * rb > 64:
            raise ValueError(f"envs_per_wave must be in 1..{64 // rb} for R={R}")
        self._alloc_state()
        self._build_params()
        self.reset(None)

    # ------------------------------------------------------------------ buffers and constants
    def _alloc_state(self):
        E, R, F, d = self.E, self.R, self.F, self.dev
        i32, f32 = torch.int32, torch.float32
        z = lambda *shape, dt=i32, v=0: torch.full(shape, v, dtype=dt, device=d)  # noqa: E731
        cfg = self.config
        nf = 3 if cfg.channel == "tr38901" else 1
        self._n_fields = nf
        self.st = {
            "cap": z(E, F, R, v=-1), "cls": z(E, F, R), "det": z(E, F, R, dt=torch.uint8), "hid": z(E, F, R, v=-1),
            "rem": z(E, F, R, dt=f32), "f_nact": z(E, F, R), "f_snr": z(E, F, R, dt=f32), "f_own": z(E, F, R),
            "qlen": z(E, R), "last_snr": z(E, R, dt=f32), "roam_left": z(E, R), "serv": z(E, R),
            "att_n": z(E, R, dt=f32), "att_logp": z(E, R, dt=f32), "credit": z(E, R, dt=f32),
            "tau": z(E, R + self.A, dt=f32), "clock": z(E, dt=torch.int64), "last_hid": z(E, dt=torch.int64),
            "pending": z(E, dt=torch.uint8, v=1), "env_id": torch.arange(E, dtype=i32, device=d),
            "episode": z(E, v=-1), "ctr_step": z(E), "ctr_submit": z(E),
            "field": z(E, self.A, nf, max(cfg.shadow_modes, 1), 3, dt=f32), "calls": z(1),
        }
        s = _lib.InetWifiState()
        for name, _ in _lib.InetWifiState._fields_:
            setattr(s, name, self.st[name].data_ptr())
        self._cstate = s

    def _build_params(self):
        from .channels import SCENARIOS, SIGMA_SF, breakpoint_m, sum_of_cosines_cdf_table
        cfg, wc, dd = self.config, self.wc, self.d
        p = _lib.InetWifiParams()
        p.E, p.R, p.F, p.K, p.M, p.L = self.E, self.R, self.F, dd.K, len(dd.rates), wc.max_tx
        p.n_cls, p.n_acc_max, p.fp_iters, p.timeout = len(cfg.msg_sizes), dd.n_acc_max, wc.fp_iters, self.TIMEOUT
        p.access_noise = 0 if wc.access_noise == "poisson" else 1
        p.rts_cts, p.coll_ack = int(wc.rts_cts), int(wc.collision_time == "ack")
        p.per_class_ac, p.no_aggr = int(dd.per_class_ac), int(wc.max_ampdu_bytes == 0)
        p.seed_key = C.c_int32(seed_key(self.seed) - (1 << 32) if seed_key(self.seed) >= 1 << 31
                               else seed_key(self.seed)).value
        p.roam_sub = int(round(wc.roam_ms / wc.substep_ms))
        p.bg_ac, p.envs_per_wave = dd.bg_ac, self.envs_per_wave
        f = np.float32
        p.noise_dbm, p.roam_hyst, p.damp = dd.noise_dbm, wc.roam_hyst_db, wc.fp_damping
        p.fer1 = float(f(1.0 - wc.frame_error_rate))
        p.dt_us, p.tau0, p.slot_us, p.sifs_us = dd.dt_us, dd.tau0, wc.slot_us, wc.sifs_us
        p.pre, p.tsym, p.ovh1, p.t_ack, p.t_rts, p.t_cts = dd.pre, dd.tsym, dd.ovh1, dd.t_ack, dd.t_rts, dd.t_cts
        p.hs = dd.t_rts + wc.sifs_us + dd.t_cts + wc.sifs_us
        p.ampdu_lim, p.msdu_payload, p.ppdu_max = dd.ampdu_lim, float(wc.msdu_payload_bytes), PPDU_MAX_US
        p.bg_w, p.bg_rate, p.bg_B = float(wc.bg_stations), dd.bg_rate, float(wc.bg_frame_bytes)
        for i, v in enumerate(dd.rates):
            p.rates[i], p.thr[i], p.mcs_ids[i] = float(v), float(dd.thr[i]), int(dd.mcs_ids[i])
        for a in range(5):
            p.ac_W0[a], p.ac_Wmax[a] = float(dd.ac_W0[a]), float(dd.ac_Wmax[a])
            p.ac_aifsn[a], p.ac_txop[a] = float(dd.ac_aifsn[a]), float(dd.ac_txop[a])
        for c, a in enumerate(dd.cls_ac):
            p.cls_ac[c] = int(a)
        for c, v in enumerate(cfg.msg_sizes):
            p.sizes[c] = float(v)
        for k, v in enumerate(dd.lgamma):
            p.lgamma[k] = float(v)
        # the AP's radio: the NRConfig of RadioMC for the APs (wifi/engine.py:82-97)
        rc = radio_config(cfg, wc)
        K = rc.shadow_modes
        p.n_fields, p.n_modes = self._n_fields, K
        xy = rc.gnb_xy()
        gx, gy = xy[0]
        p.gnb_x, p.gnb_y, p.ue_tx = gx, gy, rc.ue_tx_dbm
        p.A = len(xy)
        for a, (x_, y_) in enumerate(xy):
            p.ap_xy[2 * a], p.ap_xy[2 * a + 1] = x_, y_
        p.n_dom = self.D
        for a, dom in enumerate(self._ap_dom):
            p.ap_dom[a] = dom
        p.Z = dd.Z
        # hidden nodes: the robot-robot power sta_c0 - sta_c1 log10(d) against the CCA threshold (wifi/engine.py:268-271)
        p.hidden = int(bool(wc.hidden_nodes))
        p.cca_dbm = wc.cca_dbm
        p.sta_c0 = float(np.float32(wc.sta_tx_dbm - wc.sta_pl_1m()))
        p.sta_c1 = float(np.float32(10 * wc.sta_pl_exp))
        dc = (rc.shadow_dcorr_m, 0.0, 0.0)
        p.spectrum = 0 if rc.shadow_acf == "sos" else 1
        if rc.channel == "tr38901":
            sc = SCENARIOS[rc.tr38901_scenario]
            scn = rc.tr38901_scenario
            h_bs = float(rc.gnb_height_m) if rc.gnb_height_m is not None else sc.h_bs
            h_ut, fc = float(rc.ue_height_m), rc.carrier_ghz
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
            else:
                p.pl_a, p.pl_n1, p.pl_c20, p.pl_c2 = 31.84, 21.50, 19.00 * math.log10(fc), 0.0
            los = rc.tr38901_los == "los"
            if rc.tr38901_los == "stochastic":   # LOS and NLOS parameters, the CDF of the LOS-state field
                self._los_cdf = sum_of_cosines_cdf_table(K).to(self.dev)
                p.los_sto, p.los_cdf = 1, self._los_cdf.data_ptr()
                p.plos_scn = {"UMi": 0, "UMa": 1, "InH": 2}[scn]
                p.sig_nlos = SIGMA_SF[scn][1]
            if not los:
                if scn == "UMi":
                    p.nl_b1, p.nl_b0, p.nl_c, p.nl_d = 35.3, 22.4, 21.3 * math.log10(fc), 0.3 * (h_ut - 1.5)
                elif scn == "UMa":
                    p.nl_b1, p.nl_b0, p.nl_c, p.nl_d = 39.08, 13.54, 20 * math.log10(fc), 0.6 * (h_ut - 1.5)
                else:
                    p.nl_b1, p.nl_b0, p.nl_c, p.nl_d = 38.3, 17.30, 24.9 * math.log10(fc), 0.0
            p.sig = SIGMA_SF[scn][0 if rc.tr38901_los in ("los", "stochastic") else 1]
            p.amp = 1.0 * math.sqrt(2 / K)
            p.spectrum = 1
            dc = (sc.sf_corr_los_m, sc.sf_corr_nlos_m, sc.los_corr_m)
        else:
            p.radio_model = 0
            p.amp = rc.shadow_sigma_db * math.sqrt(2 / K)
            p.pl_const, p.pl_exp10 = rc.pl_const_db, 10 * rc.pathloss_exp
        for i in range(3):
            p.dcorr[i] = dc[i]
        self._cparams = p

    def _stream(self):
        return torch.cuda.current_stream(self.dev).cuda_stream

    # ------------------------------------------------------------------ API
    @property
    def clock(self):
        return self.st["clock"].clone()

    def output_schema(self):
        E, R, F = "E", "R", "F"
        shapes = {"newest": ("[E,R]", "int64"), "det_env": ("[E]", "bool"), "delivered": ("[E,R,F]", "bool"),
                  "timed_out": ("[E,R,F]", "bool"), "cap": ("[E,R,F]", "int64"), "cls": ("[E,R,F]", "int64"),
                  "delay": ("[E,R,F]", "float32"), "queue_len": ("[E,R]", "int64"),
                  "queue_bytes": ("[E,R]", "float32"), "sinr_db": ("[E,R]", "float32"), "t": ("[E]", "int64"),
                  "serving_cell": ("[E,R]", "int64"), "wifi_mcs": ("[E,R]", "int64"),
                  "wifi_rate_mbps": ("[E,R]", "float32"), "wifi_access_ms": ("[E,R]", "float32"),
                  "wifi_p_fail": ("[E,R]", "float32"), "wifi_busy": ("[E,R]", "float32")}
        del E, R, F
        return {k: {"shape": s, "dtype": dt, "when": "always"} for k, (s, dt) in shapes.items()}

    def _tvec(self, t):
        """Per-env step [E] int64 on the device (None: the engine clock)."""
        if t is None:
            return None
        if isinstance(t, torch.Tensor):
            t = t.to(self.dev, torch.long)
            return t.expand(self.E).contiguous() if t.dim() == 0 else t.contiguous()
        return torch.full((self.E,), int(t), dtype=torch.long, device=self.dev)

    def reset(self, env_ids=None):
        """Re-initialize env_ids (None = all; index tensor, list or bool mask [E]) (levels/base.py:142-157)."""
        if isinstance(env_ids, slice) and env_ids == slice(None):
            env_ids = None
        m8 = None
        if env_ids is not None:
            if isinstance(env_ids, torch.Tensor) and env_ids.dtype == torch.bool:
                mask = env_ids.to(self.dev)
            else:
                ids = torch.as_tensor(env_ids if isinstance(env_ids, torch.Tensor) else list(env_ids),
                                      dtype=torch.long, device=self.dev).reshape(-1)
                if ids.numel() == 0:
                    return
                mask = torch.zeros(self.E, dtype=torch.bool, device=self.dev)
                mask[ids] = True
            m8 = mask.to(torch.uint8).contiguous()
        self._reset_launch(m8)

    env_offset = 0

    def set_env_offset(self, offset):
        """Key env row i by the global env id offset + i (isaac_net/core/sharded.py:61-78): the env ids move in
        place, the episode counters are rewound by one and every env is reset again under the global ids."""
        offset = int(offset)
        if offset == self.env_offset:
            return
        self.st["env_id"].add_(offset - self.env_offset)
        self.env_offset = offset
        self.st["episode"].sub_(1)
        self.reset(None)

    def _reset_launch(self, m8):
        _lib.check(self._lib.inet_wifi_reset(C.byref(self._cstate), C.byref(self._cparams),
                                             None if m8 is None else m8.data_ptr(), self._stream()), "wifi reset")

    def submit(self, t, requests, snr_db=None):
        """Enqueue one message per robot (Requests or send [E,R]); returns accepted [E,R] bool
        (levels/base.py:223-246)."""
        tv = self._tvec(t)
        req = requests if isinstance(requests, Requests) or hasattr(requests, "send") else Requests(send=requests)
        send = req.send.to(self.dev, torch.long).contiguous()
        if tuple(send.shape) != (self.E, self.R):
            raise ValueError(f"send must be [E,R] = [{self.E},{self.R}], got {tuple(send.shape)}")
        det = None if req.det is None else req.det.to(self.dev, torch.uint8).contiguous()
        hid = None if req.hid is None else req.hid.to(self.dev, torch.long).contiguous()
        snr = None if snr_db is None else snr_db.to(self.dev, torch.float32).contiguous()
        acc = torch.empty(self.E, self.R, dtype=torch.bool, device=self.dev)
        ptr = lambda x: None if x is None else x.data_ptr()  # noqa: E731
        _lib.check(self._lib.inet_wifi_submit(
            C.byref(self._cstate), C.byref(self._cparams), ptr(tv), send.data_ptr(), ptr(det), ptr(hid), ptr(snr),
            None, 0, acc.data_ptr(), self._stream()), "wifi submit")
        return acc

    def _counts(self, counts):
        cnt = counts.to(self.dev, torch.uint8).contiguous()
        if cnt.dim() != 3 or tuple(cnt.shape[:2]) != (self.E, self.R) or not 0 < cnt.shape[-1] <= len(
                self.config.msg_sizes):
            raise ValueError("counts must be [E,R,n_classes] with n_classes <= len(msg_sizes)")
        return cnt

    def submit_counts(self, counts, t=None):
        """Enqueue counts [E,R,NC] messages per class in one launch: the submit() calls of class 1 first, one call per
        message index. Returns accepted messages [E,R] int32."""
        tv = self._tvec(t)
        cnt = self._counts(counts)
        acc = torch.empty(self.E, self.R, dtype=torch.int32, device=self.dev)
        _lib.check(self._lib.inet_wifi_submit(
            C.byref(self._cstate), C.byref(self._cparams), None if tv is None else tv.data_ptr(), None, None, None,
            None, cnt.data_ptr(), cnt.shape[-1], acc.data_ptr(), self._stream()), "wifi submit")
        return acc

    def add_frames(self, t, send, det, hid, snr_db=None):
        """Legacy wrapper (NetSlot API)."""
        self.submit(t, Requests(send, det, hid), snr_db)

    def _alloc_out(self):
        E, R, F, d = self.E, self.R, self.F, self.dev
        e = lambda *s, dt: torch.empty(*s, dtype=dt, device=d)  # noqa: E731
        o = {"newest": e(E, R, dt=torch.int64), "det_env": e(E, dt=torch.bool),
             "delivered": e(E, R, F, dt=torch.bool), "timed_out": e(E, R, F, dt=torch.bool),
             "cap": e(E, R, F, dt=torch.int64), "cls": e(E, R, F, dt=torch.int64), "delay": e(E, R, F, dt=torch.float32),
             "queue_len": e(E, R, dt=torch.int64), "queue_bytes": e(E, R, dt=torch.float32),
             "sinr_db": e(E, R, dt=torch.float32), "t": e(E, dt=torch.int64), "serving_cell": e(E, R, dt=torch.int64),
             "wifi_mcs": e(E, R, dt=torch.int64), "wifi_rate_mbps": e(E, R, dt=torch.float32),
             "wifi_access_ms": e(E, R, dt=torch.float32), "wifi_p_fail": e(E, R, dt=torch.float32),
             "wifi_busy": e(E, R, dt=torch.float32)}
        c = _lib.InetWifiOutputs()
        for a, k in (("delivered", "delivered"), ("timed_out", "timed_out"), ("cap", "cap"), ("cls", "cls"),
                     ("delay", "delay"), ("newest", "newest"), ("queue_len", "queue_len"),
                     ("serving_cell", "serving_cell"), ("mcs", "wifi_mcs"), ("queue_bytes", "queue_bytes"),
                     ("sinr_db", "sinr_db"), ("rate_mbps", "wifi_rate_mbps"), ("access_ms", "wifi_access_ms"),
                     ("p_fail", "wifi_p_fail"), ("busy", "wifi_busy"), ("det_env", "det_env"), ("t", "t")):
            setattr(c, a, o[k].data_ptr())
        return o, c

    def step(self, t=None, x=None, cur_hid=None, *, rx_dbm=None, sense=None, counts=None):
        """Advance [t, t+1). x: poses [E,R,2|3] (through the APs' radio) or the SNR [E,R] in dB; rx_dbm= [E,R,A]
        gives the received power (dBm) instead (wifi/engine.py:207-225); sense= [E,R,R] bool (hidden nodes): robot i
        senses robot j, in place of the robot-robot path loss. counts= [E,R,NC] enqueues first, as
        submit_counts(counts, t) would, in the step's own launch; the dict then also holds "accepted" [E,R] int32.
        Returns the reference's dict, or (newest, det_env) in the legacy form with cur_hid."""
        if sense is not None and not self.wc.hidden_nodes:
            raise ValueError("sense= needs WifiConfig(hidden_nodes=True)")
        kind, xin = self._input(x, rx_dbm)
        tv = self._tvec(t)
        hid = None if cur_hid is None else torch.as_tensor(cur_hid).to(self.dev, torch.long).contiguous()
        sn = None
        if sense is not None:
            sn = sense.to(self.dev, torch.uint8).contiguous()
            if tuple(sn.shape) != (self.E, self.R, self.R):
                raise ValueError(f"sense must be [E,R,R] = {(self.E, self.R, self.R)}")
        self._cparams.sense = None if sn is None else sn.data_ptr()
        try:
            o = self._run(tv, kind, xin, hid, None if counts is None else self._counts(counts))
        finally:
            self._cparams.sense = None
        if cur_hid is not None:
            return o["newest"], o["det_env"]
        return o

    def _input(self, x, rx_dbm):
        """(input kind, contiguous float32 device tensor) of the step's input: 0 poses [E,R,2], 1 SNR [E,R], 2 received
        power [E,R,A]."""
        if x is None and rx_dbm is None:
            raise ValueError("pass poses, an SNR [E,R] or rx_dbm=[E,R,A]")
        E, R = self.E, self.R
        if rx_dbm is not None:
            xin = rx_dbm.to(self.dev, torch.float32).contiguous()
            if tuple(xin.shape) != (E, R, self.A):
                raise ValueError(f"rx_dbm must be [E,R,A] = {(E, R, self.A)}")
            kind = 2
        elif x.dim() == 3:
            xin, kind = x[..., :2].to(self.dev, torch.float32).contiguous(), 0
        else:
            if self.A != 1:
                raise ValueError(f"{self.A} APs: pass poses [E,R,2|3] or rx_dbm=[E,R,A], not an SNR")
            xin, kind = x.to(self.dev, torch.float32).contiguous(), 1
            if tuple(xin.shape) != (E, R):
                raise ValueError(f"SNR must be [E,R] = {(E, R)}")
        return kind, xin

    # static_outputs = True: every step writes the same output tensors (overwritten by the next step, as the
    # reference's graph backend returns them), which spares the host the step's output allocations
    static_outputs = False
    _static = None

    def _run(self, tv, kind, xin, hid, cnt=None):
        """Allocate the step's outputs (or reuse them, static_outputs) and launch the step kernel (timed by
        kernel_events when set); with cnt [E,R,NC] uint8 the launch enqueues them first."""
        if self.static_outputs:
            if self._static is None:
                o, c = self._alloc_out()
                o["accepted"] = torch.zeros(self.E, self.R, dtype=torch.int32, device=self.dev)
                self._static = (o, c)
            o, c = self._static
            o = dict(o)
            if cnt is None:
                del o["accepted"]
        else:
            o, c = self._alloc_out()
        p = self._cparams
        if cnt is not None:
            if "accepted" not in o:
                o["accepted"] = torch.empty(self.E, self.R, dtype=torch.int32, device=self.dev)
            p.step_counts, p.step_accepted, p.step_n_cls = cnt.data_ptr(), o["accepted"].data_ptr(), cnt.shape[-1]
        ev = self.kernel_events
        try:
            if ev is not None:
                ev.begin(torch.cuda.current_stream(self.dev))
            _lib.check(self._launch(tv, kind, xin, hid, c), "wifi step")
            if ev is not None:
                ev.end(torch.cuda.current_stream(self.dev))
        finally:
            p.step_counts, p.step_accepted, p.step_n_cls = None, None, 0
        return o

    def graph_step(self, n_cls=None):
        """The control step (the enqueue of per-class arrival counts, then the step: one launch) as HIP graph replays:
        returns a WifiGraphStep, called as g(x, counts) or g(counts=..., rx_dbm=...) in place of submit_counts + step.
        A graph is recorded for every input kind and replayed; it reads the control step from the engine's device
        clock."""
        return WifiGraphStep(self, len(self.config.msg_sizes) if n_cls is None else n_cls)

    def _launch(self, tv, kind, xin, hid, c):
        return self._lib.inet_wifi_step(
            C.byref(self._cstate), C.byref(self._cparams), None if tv is None else tv.data_ptr(), kind,
            xin.data_ptr(), None if hid is None else hid.data_ptr(), C.byref(c), self._stream())

    # set to an engine.KernelTimer to record HIP events around every step-kernel launch, on the launch stream
    kernel_events = None

    # ------------------------------------------------------------------ state in the reference's names
    def state_dict(self):
        """The state tensors of the reference's WifiNet.state_dict() (FIFO fields [E,R,F], clock, mean-field state,
        counter RNG, radio plane waves), on the engine's device."""
        st = self.st
        rs = lambda x: x.permute(0, 2, 1)  # noqa: E731
        L = lambda x: x.long()  # noqa: E731
        out = {"cap": rs(L(st["cap"])), "cls": rs(L(st["cls"])), "det": rs(st["det"] != 0), "hid": rs(L(st["hid"])),
               "rem": rs(st["rem"]), "dlv": torch.full_like(rs(st["rem"]), math.inf), "f_nact": rs(L(st["f_nact"])),
               "f_snr": rs(st["f_snr"]), "f_own": rs(L(st["f_own"])), "clock": st["clock"].clone(),
               "_last_snr": st["last_snr"], "_last_hid": st["last_hid"], "tau": st["tau"],
               "roam_left": L(st["roam_left"]), "att_n": st["att_n"], "att_logp": st["att_logp"],
               "credit": st["credit"], "serv": L(st["serv"]), "pending": st["pending"] != 0,
               "rng.episode": L(st["episode"]), "rng.ctr[1]": L(st["ctr_submit"]) + L(st["calls"]),
               "rng.ctr[2]": L(st["ctr_step"])}
        f = st["field"].permute(1, 0, 2, 3, 4)                     # [A, E, NF, K, 3]: the cells of RadioMC
        if self.config.channel == "tr38901":
            for j, n in enumerate(("sf_los", "sf_nlos", "los_field")):
                out[f"radio.ch.{n}.k"] = f[:, :, j, :, :2]
                out[f"radio.ch.{n}.phi"] = f[:, :, j, :, 2]
        else:
            out["radio.k"] = f[:, :, 0, :, :2]
            out["radio.phi"] = f[:, :, 0, :, 2]
        return out

    def load_state_dict(self, sd):
        """Load reference-named state (the keys of state_dict(); tensors on any device) into the device buffers."""
        st, d = self.st, self.dev
        g = lambda k: torch.as_tensor(sd[k]).to(d)  # noqa: E731
        rs = lambda x: x.permute(0, 2, 1).contiguous()  # noqa: E731
        I = lambda x: x.to(torch.int32)  # noqa: E731
        cap = g("cap")
        st["qlen"].copy_(I((cap >= 0).sum(-1)))
        for k in ("cap", "cls", "hid", "f_nact", "f_own"):
            st[k].copy_(rs(I(g(k))))
        st["det"].copy_(rs(g("det").to(torch.uint8)))
        st["rem"].copy_(rs(g("rem").float()))
        st["f_snr"].copy_(rs(g("f_snr").float()))
        st["clock"].copy_(g("clock").long())
        st["last_snr"].copy_(g("_last_snr").float())
        st["last_hid"].copy_(g("_last_hid").long())
        st["tau"].copy_(g("tau").float())
        for k in ("roam_left", "serv"):
            st[k].copy_(I(g(k)))
        for k in ("att_n", "att_logp", "credit"):
            st[k].copy_(g(k).float())
        st["pending"].copy_(g("pending").to(torch.uint8))
        st["episode"].copy_(I(g("rng.episode")))
        st["calls"].zero_()
        st["ctr_submit"].copy_(I(g("rng.ctr[1]")))
        st["ctr_step"].copy_(I(g("rng.ctr[2]")))
        names = (("sf_los", 0), ("sf_nlos", 1), ("los_field", 2)) if self.config.channel == "tr38901" else ()
        fv = st["field"].permute(1, 0, 2, 3, 4)                    # [A, E, NF, K, 3] view of the buffer
        if names:
            for n, j in names:
                if f"radio.ch.{n}.k" in sd:
                    fv[:, :, j, :, :2] = g(f"radio.ch.{n}.k")
                    fv[:, :, j, :, 2] = g(f"radio.ch.{n}.phi")
        elif "radio.k" in sd:
            fv[:, :, 0, :, :2] = g("radio.k")
            fv[:, :, 0, :, 2] = g("radio.phi")


class WifiGraphStep:
    """step(x, counts=) of a HipWifiEngine (level WIFI or WIFI_DCF) as HIP graphs (torch.cuda.CUDAGraph): one per
    input kind, recorded on first use and replayed at every control step. The inputs are copied into static buffers
    (a producer may also write g.counts and g.inputs[kind] itself and call g.replay(kind)); the returned dict is the
    graph's static output buffers, overwritten by its next replay. Each graph is one kernel node (the step launch with
    its enqueue)."""

    def __init__(self, eng, n_cls):
        self.eng = eng
        self.counts = torch.zeros(eng.E, eng.R, n_cls, dtype=torch.uint8, device=eng.dev)
        self.inputs = {}
        self.graphs = {}

    def __call__(self, x=None, counts=None, *, rx_dbm=None):
        eng = self.eng
        kind, xin = eng._input(x, rx_dbm)
        if counts is None or tuple(counts.shape) != tuple(self.counts.shape):
            raise ValueError(f"counts must be {tuple(self.counts.shape)}")
        if kind not in self.inputs:
            self.inputs[kind] = torch.empty_like(xin)
        self.inputs[kind].copy_(xin)
        self.counts.copy_(counts)
        return self.replay(kind)

    def replay(self, kind):
        """Replay the graph of input kind (0 poses, 1 SNR, 2 received power) on the current contents of g.counts and
        g.inputs[kind], recording it first if needed; returns the static outputs."""
        eng = self.eng
        hit = self.graphs.get(kind)
        if hit is None:
            torch.cuda.synchronize(eng.dev)
            g = torch.cuda.CUDAGraph()
            ev, eng.kernel_events = eng.kernel_events, None
            try:
                with torch.cuda.graph(g):
                    out = eng._run(None, kind, self.inputs[kind], None, self.counts)
            finally:
                eng.kernel_events = ev
            torch.cuda.synchronize(eng.dev)
            hit = self.graphs[kind] = (g, out)
        g, out = hit
        g.replay()
        return out


class HipWifiDcfEngine(HipWifiEngine):
    """Level WIFI_DCF on MI355X: the level WIFI API with per-slot CSMA/CA access (integer backoff counters, collisions,
    binary exponential backoff, retry limit) in place of the mean-field sub-steps. The semantics follow the
    reference's validation simulator (isaac_net/core/wifi/eventsim.py:56-186) on the engine's counter RNG; they are
    stated in full in include/inet_wifi.h and oracle/dcf_oracle.py's module docstring."""

    level = "WIFI_DCF"

    def __init__(self, E, R, device="cuda", cfg: NRConfig | None = None, seed=None, envs_per_wave=None):
        cfg = cfg if cfg is not None else NRConfig()
        wc = cfg.wifi if cfg.wifi is not None else WifiConfig()
        if wc.bg_stations > 0 or wc.class_ac is not None or len(wc.ap_xy(cfg)) != 1 or wc.hidden_nodes:
            raise HipUnsupported("level WIFI_DCF: one AP, one access category for every robot, no background "
                                 "stations and no hidden nodes")
        self._dcf_ready = False
        super().__init__(E, R, device, cfg, seed=seed, envs_per_wave=envs_per_wave)
        self._build_dcf()
        self._dcf_ready = True
        self.reset(None)

    def _build_dcf(self):
        from .wifi_config import AC_NAMES, ACK_BYTES, BLOCK_ACK_BYTES, CTS_BYTES, DATA_SUBCARRIERS, EDCA, \
            MODULATION, NON_HT_RATES, RTS_BYTES, mcs_numbers, preamble_us, symbol_us
        cfg, wc, E, R, d = self.config, self.wc, self.E, self.R, self.dev
        self.dst = {"b": torch.zeros(E, R, dtype=torch.int32, device=d),
                    "stage": torch.zeros(E, R, dtype=torch.int32, device=d),
                    "had": torch.zeros(E, R, dtype=torch.uint8, device=d),
                    "t_idle": torch.zeros(E, dtype=torch.int32, device=d)}
        s = _lib.InetDcfState()
        for n, _ in _lib.InetDcfState._fields_:
            setattr(s, n, self.dst[n].data_ptr())
        self._cdcf = s
        ns = lambda us: int(round(us * 1000.0))  # noqa: E731
        p = _lib.InetDcfParams()
        if wc.standard == "a":
            nd = [int(r * 4) for r in NON_HT_RATES]
        else:
            nsd = DATA_SUBCARRIERS[wc.standard][wc.bandwidth_mhz]
            nd = [int(round(nsd * MODULATION[m][0] * MODULATION[m][1] * wc.n_ss))
                  for m in mcs_numbers(wc.standard, wc.bandwidth_mhz, wc.n_ss)]
        for i, v in enumerate(nd):
            p.ndbps[i] = v
        T = cfg.control_step_ms * 1e6
        if abs(T - round(T)) > 1e-6 or round(T) > 1 << 30:
            raise HipUnsupported("level WIFI_DCF: the control step must be a whole number of ns up to 1.07 s")
        ctrl = lambda n: ns(20.0 + 4.0 * math.ceil((22 + 8 * n) / (wc.ctrl_rate_mbps * 4.0)))  # noqa: E731
        cw = EDCA[wc.access_category]
        p.T, p.tsym, p.pre = int(round(T)), ns(symbol_us(wc.standard, wc.gi_us)), ns(preamble_us(wc.standard, wc.n_ss))
        p.sifs, p.slot = ns(wc.sifs_us), ns(wc.slot_us)
        p.t_ack = ctrl(BLOCK_ACK_BYTES if wc.max_ampdu_bytes > 0 else ACK_BYTES)
        p.t_rts, p.t_cts = ctrl(RTS_BYTES), ctrl(CTS_BYTES)
        p.W0, p.Wmax, p.aifsn = cw[0] + 1, cw[1] + 1, int(cw[2])
        p.ovh, p.payload = int(wc.msdu_overhead_bytes), int(wc.msdu_payload_bytes)
        p.fer = float(np.float32(wc.frame_error_rate))
        self._cdparams = p
        self.dcf_ac = AC_NAMES.index(wc.access_category)

    env_offset = 0

    def set_env_offset(self, offset):
        """Key env row i by the global env id offset + i (isaac_net/core/sharded.py:61-78): the env ids move in
        place, the episode counters are rewound by one and every env is reset again under the global ids."""
        offset = int(offset)
        if offset == self.env_offset:
            return
        self.st["env_id"].add_(offset - self.env_offset)
        self.env_offset = offset
        self.st["episode"].sub_(1)
        self.reset(None)

    def _reset_launch(self, m8):
        if not getattr(self, "_dcf_ready", False):
            return                # the base constructor's reset: the full reset follows once the DCF state exists
        _lib.check(self._lib.inet_wifi_dcf_reset(C.byref(self._cstate), C.byref(self._cdcf), C.byref(self._cparams),
                                                 C.byref(self._cdparams), None if m8 is None else m8.data_ptr(),
                                                 self._stream()), "wifi dcf reset")

    def _launch(self, tv, kind, xin, hid, c):
        return self._lib.inet_wifi_dcf_step(
            C.byref(self._cstate), C.byref(self._cdcf), C.byref(self._cparams), C.byref(self._cdparams),
            None if tv is None else tv.data_ptr(), kind, xin.data_ptr(), None if hid is None else hid.data_ptr(),
            C.byref(c), self._stream())

    def state_dict(self):
        sd = super().state_dict()
        sd.update({"dcf.b": self.dst["b"].long(), "dcf.stage": self.dst["stage"].long(),
                   "dcf.had": self.dst["had"] != 0, "dcf.t_idle": self.dst["t_idle"].long()})
        return sd

    def load_state_dict(self, sd):
        super().load_state_dict(sd)
        g = lambda k: torch.as_tensor(sd[k]).to(self.dev)  # noqa: E731
        if "dcf.b" in sd:
            self.dst["b"].copy_(g("dcf.b").to(torch.int32))
            self.dst["stage"].copy_(g("dcf.stage").to(torch.int32))
            self.dst["had"].copy_(g("dcf.had").to(torch.uint8))
            self.dst["t_idle"].copy_(g("dcf.t_idle").to(torch.int32))

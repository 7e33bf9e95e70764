"""WifiConfig and the 802.11 PHY / EDCA constants of level "WIFI" (the mean-field 802.11 uplink of a robot fleet).

Same field names, meanings, defaults and checks as the reference dataclass (isaac_net/core/wifi/config.py:29-185),
and the same derived quantities as its PHY abstraction (isaac_net/core/wifi/phy.py:47-155):

  rates        data rate of every valid MCS: N_SD * bits per subcarrier * code rate * N_SS / T_sym (Mb/s)
  thresholds   receiver minimum input sensitivity at 20 MHz minus the -91 dBm noise it assumes (dB), + ra_margin_db
  PPDU time    preamble + T_sym * ceil((22 + 8 * air bytes) / (rate * T_sym))
  access time  Ts = AIFS [+ RTS + SIFS + CTS + SIFS] + PPDU + SIFS + (Block) ACK; Tc = AIFS + PPDU (basic, "difs"),
               = Ts ("ack"), or AIFS + RTS + SIFS + CTS (RTS/CTS)

Sources of the tables: IEEE Std 802.11-2016 Table 9-137 (EDCA defaults), Sec. 17 / 21 / 27 (OFDM, VHT, HE rates,
sensitivities, preambles), Sec. 21.5 (VHT MCS not valid at some bandwidths). The host computes every constant in
double precision and rounds it to float32 where the reference's torch code does, so the kernels see the same values.
"""
from __future__ import annotations

import copy
import math
from dataclasses import dataclass, replace

import numpy as np

# access categories: (CWmin, CWmax, AIFSN, TXOP limit in us); index = AC id (order of the reference's AC_NAMES)
AC_NAMES = ("BK", "BE", "VI", "VO", "DCF")
EDCA = {"BK": (15, 1023, 7, 0.0), "BE": (15, 1023, 3, 0.0), "VI": (7, 15, 2, 3008.0), "VO": (3, 7, 2, 1504.0),
        "DCF": (15, 1023, 2, 0.0)}
STANDARDS = ("ax", "ac", "a")
BANDWIDTHS = {"ax": (20, 40, 80, 160), "ac": (20, 40, 80, 160), "a": (20,)}

# (bits per subcarrier, code rate) of HT / VHT / HE MCS 0..11
MODULATION = ((1, 1 / 2), (2, 1 / 2), (2, 3 / 4), (4, 1 / 2), (4, 3 / 4), (6, 2 / 3), (6, 3 / 4), (6, 5 / 6),
              (8, 3 / 4), (8, 5 / 6), (10, 3 / 4), (10, 5 / 6))
SENSITIVITY_20MHZ = (-82, -79, -77, -74, -70, -66, -65, -64, -59, -57, -54, -52)      # dBm, MCS 0..11
NON_HT_RATES = (6, 9, 12, 18, 24, 36, 48, 54)                                          # Mb/s
NON_HT_SENSITIVITY = (-82, -81, -79, -77, -74, -70, -66, -65)                          # dBm
SENSITIVITY_NOISE_DBM = -174.0 + 10 * math.log10(20e6) + 10.0                          # -91 dBm
DATA_SUBCARRIERS = {"ax": {20: 234, 40: 468, 80: 980, 160: 1960}, "ac": {20: 52, 40: 108, 80: 234, 160: 468}}
LTF_COUNT = {1: 1, 2: 2, 3: 4, 4: 4}
ACK_BYTES, BLOCK_ACK_BYTES, RTS_BYTES, CTS_BYTES = 14, 32, 20, 14
PPDU_MAX_US = 5484.0
# (bandwidth MHz, VHT-MCS, N_SS) that IEEE 802.11-2016 Sec. 21.5 marks not valid
VHT_NOT_VALID = frozenset({(20, 9, n) for n in (1, 2, 4, 5, 7, 8)} | {(80, 6, 3), (80, 6, 7), (80, 9, 6),
                                                                       (160, 9, 3)})


@dataclass
class WifiConfig:
    """802.11 PHY, EDCA, access points and mean-field knobs of level WIFI (reference wifi/config.py:29-125)."""
    standard: str = "ax"
    bandwidth_mhz: int = 20
    n_ss: int = 1
    gi_us: float = 0.8
    carrier_ghz: float = 5.2
    ra_margin_db: float = 0.0
    ap_nf_db: float = 7.0
    sta_tx_dbm: float = 20.0
    access_category: str = "BE"
    class_ac: tuple | None = None
    rts_cts: bool = False
    max_tx: int = 7
    max_ampdu_bytes: int = 65535
    ba_window: int = 64
    msdu_payload_bytes: int = 1472
    msdu_overhead_bytes: int = 70
    slot_us: float = 9.0
    sifs_us: float = 16.0
    ctrl_rate_mbps: float = 24.0
    frame_error_rate: float = 0.0
    collision_time: str = "difs"
    ap_positions_m: tuple | None = None
    ap_height_m: float | None = None
    n_channels: int = 1
    ap_channels: tuple | None = None
    roam_hyst_db: float = 6.0
    roam_ms: float = 0.0
    bg_stations: int = 0
    bg_frame_bytes: int = 1500
    bg_mcs: int = 4
    bg_ac: str = "BE"
    hidden_nodes: bool = False
    cca_dbm: float = -82.0
    sta_pl_exp: float = 3.0
    sta_pl_1m_db: float | None = None
    substep_ms: float = 1.0
    fp_iters: int = 6
    fp_damping: float = 0.6
    access_noise: str = "poisson"

    def __post_init__(self):
        assert self.standard in STANDARDS, f"standard must be one of {STANDARDS}"
        assert self.bandwidth_mhz in BANDWIDTHS[self.standard], f"{self.standard}: bandwidth_mhz in " \
                                                                 f"{BANDWIDTHS[self.standard]}"
        assert 1 <= self.n_ss <= 4 and (self.standard != "a" or self.n_ss == 1)
        if self.standard == "ax":
            assert self.gi_us in (0.8, 1.6, 3.2), "ax: gi_us 0.8, 1.6 or 3.2"
        elif self.standard == "ac":
            assert self.gi_us in (0.4, 0.8), "ac: gi_us 0.4 or 0.8"
        assert self.access_category in EDCA and self.bg_ac in EDCA
        if self.class_ac is not None:
            self.class_ac = tuple(self.class_ac)
            assert all(a in EDCA for a in self.class_ac), f"class_ac entries in {tuple(EDCA)}"
        assert self.max_tx >= 1 and self.max_ampdu_bytes >= 0 and self.ba_window >= 1
        assert self.msdu_payload_bytes > 0 and self.msdu_overhead_bytes >= 0
        assert self.slot_us > 0 and self.sifs_us > 0 and self.ctrl_rate_mbps > 0
        assert 0.0 <= self.frame_error_rate < 1.0 and self.collision_time in ("ack", "difs")
        assert self.n_channels >= 1 and self.bg_stations >= 0 and self.bg_frame_bytes > 0 and self.bg_mcs >= 0
        assert self.roam_ms >= 0 and self.substep_ms > 0 and self.fp_iters >= 1 and 0 < self.fp_damping <= 1
        assert self.access_noise in ("poisson", "mean")
        if self.ap_positions_m is not None:
            self.ap_positions_m = tuple(tuple(float(v) for v in p) for p in self.ap_positions_m)
            assert len(self.ap_positions_m) >= 1
        if self.ap_channels is not None:
            self.ap_channels = tuple(int(c) for c in self.ap_channels)
            if self.ap_positions_m is not None:
                assert len(self.ap_channels) == len(self.ap_positions_m), "one channel per AP"

    def with_(self, **kw):
        return replace(self, **kw)

    def ap_xy(self, nr_cfg=None):
        if self.ap_positions_m is not None:
            return [tuple(p) for p in self.ap_positions_m]
        return nr_cfg.gnb_xy() if nr_cfg is not None else [(0.0, 0.0)]

    def channels(self, n_ap):
        if self.ap_channels is not None:
            assert len(self.ap_channels) == n_ap, "one channel per AP"
            return list(self.ap_channels)
        return [a % self.n_channels for a in range(n_ap)]

    def sta_pl_1m(self):
        """Robot-robot path loss at 1 m (dB): sta_pl_1m_db, else free space at the carrier (wifi/config.py:182-185)."""
        if self.sta_pl_1m_db is not None:
            return float(self.sta_pl_1m_db)
        return 20 * math.log10(4 * math.pi * self.carrier_ghz * 1e9 / 299_792_458.0)

    def substeps(self, control_step_ms):
        n = control_step_ms / self.substep_ms
        if abs(n - round(n)) > 1e-9 or round(n) < 1:
            raise ValueError(f"control_step_ms={control_step_ms} is not a whole number of substep_ms="
                             f"{self.substep_ms}")
        return int(round(n))

    def noise_dbm(self):
        """Thermal noise over the channel at the AP: -174 dBm/Hz + 10 log10(bandwidth) + NF."""
        return -174.0 + 10 * math.log10(self.bandwidth_mhz * 1e6) + self.ap_nf_db


# ---------------------------------------------------------------------------------------------- PHY
def symbol_us(std, gi_us):
    return {"ax": 12.8 + gi_us, "ac": 3.2 + gi_us, "a": 4.0}[std]


def preamble_us(std, n_ss=1):
    """Non-HT 20 us; VHT L-STF/LTF/SIG + VHT-SIG-A + VHT-STF + N_LTF x 4 us + VHT-SIG-B; HE SU 36 + N_LTF x 8 us."""
    if std == "a":
        return 20.0
    return 36.0 + (4.0 if std == "ac" else 8.0) * LTF_COUNT[n_ss]


def mcs_numbers(std, bandwidth_mhz=20, n_ss=1):
    if std == "a":
        return list(range(len(NON_HT_RATES)))
    top = 12 if std == "ax" else 10
    return [m for m in range(top) if not (std == "ac" and (bandwidth_mhz, m, n_ss) in VHT_NOT_VALID)]


def mcs_table(std, bandwidth_mhz=20, n_ss=1, gi_us=0.8):
    """(rates Mb/s, SNR thresholds dB) of the valid MCS, lowest first (double precision)."""
    if std == "a":
        return [float(r) for r in NON_HT_RATES], [s - SENSITIVITY_NOISE_DBM for s in NON_HT_SENSITIVITY]
    tsym, nsd = symbol_us(std, gi_us), DATA_SUBCARRIERS[std][bandwidth_mhz]
    rates, thr = [], []
    for m in mcs_numbers(std, bandwidth_mhz, n_ss):
        bits, code = MODULATION[m]
        rates.append(nsd * bits * code * n_ss / tsym)
        thr.append(SENSITIVITY_20MHZ[m] - SENSITIVITY_NOISE_DBM)
    return rates, thr


def ctrl_us(nbytes, rate_mbps):
    """Non-HT control frame: 20 us preamble + 4 us symbols of (22 + 8 bytes) bits."""
    return 20.0 + 4.0 * math.ceil((22 + 8 * nbytes) / (rate_mbps * 4.0))


def free_space_1m_db(carrier_ghz):
    return 20 * math.log10(4 * math.pi * carrier_ghz * 1e9 / 299_792_458.0)


def radio_config(cfg, wc: WifiConfig):
    """The NRConfig of the APs' radio (reference wifi/engine.py:82-97): AP positions as cells, the Wi-Fi carrier,
    the robot transmit power; log_distance with the default pl_const_db takes the free-space loss at 1 m."""
    c = copy.copy(cfg)
    xy = wc.ap_xy(cfg)
    c.n_cells, c.cell_layout, c.cell_positions_m = len(xy), "custom", tuple(tuple(p) for p in xy)
    c.carrier_ghz, c.ue_tx_dbm = wc.carrier_ghz, wc.sta_tx_dbm
    if cfg.channel == "log_distance" and cfg.pl_const_db == 40.0:
        c.pl_const_db = free_space_1m_db(wc.carrier_ghz)
    if wc.ap_height_m is not None:
        c.gnb_height_m = wc.ap_height_m
    return c


def poisson_cap(lam_max):
    """Support of the Poisson draw: ceil(lam_max + 6 sqrt(lam_max) + 1), lam_max floored at 1
    (reference wifi/engine.py:66-71)."""
    lam_max = max(float(lam_max), 1.0)
    return int(math.ceil(lam_max + 6.0 * math.sqrt(lam_max) + 1.0))


@dataclass
class WifiDerived:
    """Host-derived constants of one (NRConfig, WifiConfig): tables and float32 scalars the kernels read."""
    K: int                      # sub-steps per control step
    rates: np.ndarray           # [M] float32 Mb/s
    thr: np.ndarray             # [M] float32 dB (ra_margin_db included)
    mcs_ids: np.ndarray         # [M] int64 MCS number of each entry
    ac_W0: np.ndarray           # [5] float32 CWmin + 1
    ac_Wmax: np.ndarray         # [5] float32 CWmax + 1
    ac_aifsn: np.ndarray        # [5] float32
    ac_txop: np.ndarray         # [5] float32 us
    cls_ac: np.ndarray          # [n_cls + 1] int64 AC of each message class (entry 0: the default AC)
    per_class_ac: bool
    Z: int                      # AIFS zones (1 = one AIFSN among the robots' and background ACs)
    bg_ac: int
    bg_rate: float
    n_acc_max: int
    tau0: float
    noise_dbm: float
    tsym: float
    pre: float
    ovh1: float                 # 1 + msdu overhead / payload (float32 multiplier of the air bytes)
    t_ack: float
    t_rts: float
    t_cts: float
    ampdu_lim: float            # min(max_ampdu / (1 + ovh), ba_window * payload)
    dt_us: float
    lgamma: np.ndarray          # [n_acc_max] float32 lgamma(k + 1)


def derive(cfg, wc: WifiConfig) -> WifiDerived:
    """The constants of the reference's WifiNet._alloc (wifi/engine.py:114-177) for a single-AP config."""
    f32 = np.float32
    K = wc.substeps(cfg.control_step_ms)
    rates_d, thr_d = mcs_table(wc.standard, wc.bandwidth_mhz, wc.n_ss, wc.gi_us)
    rates = np.array(rates_d, dtype=f32)
    thr = (np.array(thr_d, dtype=f32) + f32(wc.ra_margin_db)).astype(f32)
    ids = mcs_numbers(wc.standard, wc.bandwidth_mhz, wc.n_ss)
    tab = np.array([EDCA[a] for a in AC_NAMES], dtype=f32)
    n_cls = len(cfg.msg_sizes)
    dflt = AC_NAMES.index(wc.access_category)
    per_cls = [dflt] + [AC_NAMES.index(wc.class_ac[c]) if wc.class_ac is not None and c < len(wc.class_ac)
                        else dflt for c in range(n_cls)]
    used = set(per_cls[1:]) | ({AC_NAMES.index(wc.bg_ac)} if wc.bg_stations > 0 else set())
    aif = [EDCA[AC_NAMES[a]][2] for a in used]
    bg_ac = AC_NAMES.index(wc.bg_ac)
    bg_rate = float(rates[max(i for i, m in enumerate(ids) if m <= wc.bg_mcs)])
    ovh = wc.msdu_overhead_bytes / wc.msdu_payload_bytes
    agg = wc.max_ampdu_bytes > 0
    t_ack = ctrl_us(BLOCK_ACK_BYTES if agg else ACK_BYTES, wc.ctrl_rate_mbps)
    # upper bound of the successful accesses per sub-step: Ts of a 1-byte access at the top rate after the shortest
    # AIFS (Python floats in the reference, so double precision here)
    aifsn_min = float(min(v[2] for v in EDCA.values()))
    ts_min = _ts_double(wc, 1.0, float(max(rates_d)), aifsn_min, t_ack)
    n_max = poisson_cap(wc.substep_ms * 1000.0 / float(ts_min))
    import torch
    lg = torch.lgamma(torch.arange(n_max, dtype=torch.float32) + 1.0).numpy()
    return WifiDerived(
        K=K, rates=rates, thr=thr, mcs_ids=np.array(ids, dtype=np.int64), ac_W0=tab[:, 0] + f32(1),
        ac_Wmax=tab[:, 1] + f32(1), ac_aifsn=tab[:, 2].copy(), ac_txop=tab[:, 3].copy(),
        cls_ac=np.array(per_cls, dtype=np.int64), per_class_ac=len(set(per_cls[1:])) > 1,
        Z=int(max(aif) - min(aif)) + 1, bg_ac=bg_ac, bg_rate=bg_rate, n_acc_max=n_max,
        tau0=float(f32(2.0) / (tab[dflt, 0] + f32(1) + f32(1.0))), noise_dbm=wc.noise_dbm(),
        tsym=symbol_us(wc.standard, wc.gi_us), pre=preamble_us(wc.standard, wc.n_ss), ovh1=1.0 + ovh, t_ack=t_ack,
        t_rts=ctrl_us(RTS_BYTES, wc.ctrl_rate_mbps), t_cts=ctrl_us(CTS_BYTES, wc.ctrl_rate_mbps),
        ampdu_lim=min(wc.max_ampdu_bytes / (1.0 + ovh), wc.ba_window * wc.msdu_payload_bytes),
        dt_us=wc.substep_ms * 1000.0, lgamma=lg.astype(f32))


def _ts_double(wc, B, rate, aifsn, t_ack):
    """Ts of one access of B bytes (reference wifi/phy.py:141-155 on Python floats)."""
    tsym = symbol_us(wc.standard, wc.gi_us)
    aifs = wc.sifs_us + aifsn * wc.slot_us
    air = B * (1.0 + wc.msdu_overhead_bytes / wc.msdu_payload_bytes)
    tdata = preamble_us(wc.standard, wc.n_ss) + tsym * math.ceil((22.0 + 8.0 * air) / (rate * tsym))
    if wc.rts_cts:
        hs = ctrl_us(RTS_BYTES, wc.ctrl_rate_mbps) + wc.sifs_us + ctrl_us(CTS_BYTES, wc.ctrl_rate_mbps) + wc.sifs_us
        return aifs + hs + tdata + wc.sifs_us + t_ack
    return aifs + tdata + wc.sifs_us + t_ack

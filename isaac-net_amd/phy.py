"""PHY abstraction tables of the NR uplink engine, built once on the host (numpy) and uploaded to the device.

Restates isaac_net/core/phy.py for the single-layer, Sionna-table ("pdsch") path:
  * MCS tables 38.214 5.1.3.1-1 / -2 (phy.py:21-29) and the 38.214 5.1.3.2 TBS (phy.py:77-106);
  * LDPC code-block segmentation 38.212 5.2.2 (phy.py:109-119);
  * the BLER table post-processing of the shipped Sionna SYS 2.2.0 export (phy.py:405-482): missing curves filled
    from the other table or by a Shannon-gap shift, the waterfall continued above the last simulated SNR, the grid
    padded down to -15 dB with BLER 1, and BLER made non-increasing in SNR;
  * the target-BLER thresholds thr / thr_ref (phy.py:234-243, 287-295) and the HARQ-IR equivalent MCS (phy.py:224-230);
  * the per-(PRBs, MCS) link-adaptation tables the kernel reads: TBS, code-block-size index and interpolation weight,
    number of code blocks (the same numbers phy.select_mcs computes per call, phy.py:339-350).
float64 where phy.py computes in float64, float32 where it rounds to float32, so every table value equals what the
reference's torch code produces (pinned by the golden PHY fixture).
The data file data/sionna_phy_tables.npz is the reference's shipped Sionna export (Apache-2.0, LICENSE next to it).
"""
from __future__ import annotations

import json
import math
import os

import numpy as np

MCS_T1 = [(2, 120), (2, 157), (2, 193), (2, 251), (2, 308), (2, 379), (2, 449), (2, 526), (2, 602),
          (2, 679), (4, 340), (4, 378), (4, 434), (4, 490), (4, 553), (4, 616), (4, 658), (6, 438),
          (6, 466), (6, 517), (6, 567), (6, 616), (6, 666), (6, 719), (6, 772), (6, 822), (6, 873),
          (6, 910), (6, 948)]
MCS_T2 = [(2, 120), (2, 193), (2, 308), (2, 449), (2, 602), (4, 378), (4, 434), (4, 490), (4, 553),
          (4, 616), (4, 658), (6, 466), (6, 517), (6, 567), (6, 616), (6, 666), (6, 719), (6, 772),
          (6, 822), (6, 873), (8, 682.5), (8, 711), (8, 754), (8, 797), (8, 841), (8, 885),
          (8, 916.5), (8, 948)]
MCS_TABLES = {1: MCS_T1, 2: MCS_T2}
# TS 38.214 Table 5.2.2.1-2 (4-bit CQI table 1) and Table 5.2.2.1-3 (table 2, up to 256QAM): (Qm, code rate x 1024)
# of CQI 1..15
CQI_T1 = [(2, 78), (2, 120), (2, 193), (2, 308), (2, 449), (2, 602), (4, 378), (4, 490), (4, 616), (6, 466), (6, 567),
          (6, 666), (6, 772), (6, 873), (6, 948)]
CQI_T2 = [(2, 78), (2, 193), (2, 449), (4, 378), (4, 490), (4, 616), (6, 466), (6, 567), (6, 666), (6, 772), (6, 873),
          (8, 711), (8, 797), (8, 885), (8, 948)]
CQI_TABLES = {1: CQI_T1, 2: CQI_T2}
# TS 38.214 Table 5.1.3.2-1: TBS for N_info <= 3824
TBS_TABLE = np.array([24, 32, 40, 48, 56, 64, 72, 80, 88, 96, 104, 112, 120, 128, 136, 144, 152, 160, 168, 176,
                      184, 192, 208, 224, 240, 256, 272, 288, 304, 320, 336, 352, 368, 384, 408, 432, 456, 480,
                      504, 528, 552, 576, 608, 640, 672, 704, 736, 768, 808, 848, 888, 928, 984, 1032, 1064,
                      1128, 1160, 1192, 1224, 1256, 1288, 1320, 1352, 1416, 1480, 1544, 1608, 1672, 1736, 1800,
                      1864, 1928, 2024, 2088, 2152, 2216, 2280, 2408, 2472, 2536, 2600, 2664, 2728, 2792, 2856,
                      2976, 3104, 3240, 3368, 3496, 3624, 3752, 3824], dtype=np.float64)
SNR_MIN = -15.0
DATA = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data", "sionna_phy_tables.npz")
_f32 = np.float32


def tbs_38214(qm, r, n_prb, nsym, dmrs=12, oh=0, layers=1):
    """Exact TBS (bits) of 38.214 5.1.3.2 steps 1-4, elementwise over broadcast float64 arrays; 0 PRBs -> 0."""
    qm, r, n_prb, nsym = (np.asarray(v, dtype=np.float64) for v in (qm, r, n_prb, nsym))
    n_re = np.minimum(12 * nsym - float(dmrs) - float(oh), 156.0) * n_prb
    n_info = n_re * r * qm * float(layers)
    with np.errstate(divide="ignore", invalid="ignore"):
        n = np.maximum(np.floor(np.log2(np.maximum(n_info, 1.0))) - 6, 3.0)
        ninfo_q = np.maximum(2 ** n * np.floor(n_info / 2 ** n), 24.0)
        idx = np.minimum(np.searchsorted(TBS_TABLE, ninfo_q, side="left"), len(TBS_TABLE) - 1)
        tbs_small = TBS_TABLE[idx]
        n4 = np.floor(np.log2(np.maximum(n_info - 24, 1.0))) - 5
        x = (n_info - 24) / 2 ** n4
        ninfo_q4 = np.maximum(2 ** n4 * np.floor(x + 0.5), 3840.0)
        c_low = np.ceil((ninfo_q4 + 24) / 3816)
        tbs_low = 8 * c_low * np.ceil((ninfo_q4 + 24) / (8 * c_low)) - 24
        c_hi = np.ceil((ninfo_q4 + 24) / 8424)
        tbs_hi = 8 * c_hi * np.ceil((ninfo_q4 + 24) / (8 * c_hi)) - 24
        tbs_mid = 8 * np.ceil((ninfo_q4 + 24) / 8) - 24
    tbs_large = np.where(r <= 0.25, tbs_low, np.where(ninfo_q4 > 8424, tbs_hi, tbs_mid))
    tbs = np.where(n_info <= 3824, tbs_small, tbs_large)
    return np.where(n_re > 0, tbs, 0.0).astype(np.int64)


def segment(tbs, r):
    """(code-block size incl. CRC, number of code blocks), float64, 38.212 5.2.2 as phy.segment."""
    t = np.asarray(tbs, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    bg2 = (t <= 292) | ((t <= 3824) & (r <= 0.67)) | (r <= 0.25)
    kcb = np.where(bg2, 3840.0, 8448.0)
    b = t + np.where(t > 3824, 24.0, 16.0)
    c = np.where(b <= kcb, 1.0, np.ceil(b / (kcb - 24)))
    bp = np.where(c > 1, b + 24 * c, b)
    return bp / c, c


def build_bler_table(d, mcs_table):
    """[M, C, G] float32 BLER table and the padded SNR grid [G] float32 from the Sionna export d (npz mapping).

    Both directions use the PDSCH curves (bler_source "pdsch", the reference default). Steps (reference phy.py:405-482):
    pad the grid to SNR_MIN with BLER 1; drop curves that never reach 0.1 on the reference code-block size inside
    the simulated range; continue every curve log-linearly above the last simulated SNR (slope of its last segment,
    at least one decade per dB); fill missing curves from the other table (same Qm and R) or by the Shannon-gap shift
    of the nearest valid MCS; finally clip to [0, 1] and take the running minimum along SNR."""
    cat = "dl"
    fname = "PDSCH_table{}.json"
    snr0 = d["snr_grid"].astype(np.float64)
    ds = snr0[1] - snr0[0]
    pad = int(round((snr0[0] - SNR_MIN) / ds))
    snr = np.concatenate([snr0[0] + ds * np.arange(-pad, 0), snr0])
    ci_ref = int(np.argmin(np.abs(d["cbs_grid"] - 1924)))
    raw_all = json.loads(bytes(d["raw_json"]).decode())

    def gap(q, c):
        return 10 * math.log10(2 ** (q * c / 1024) - 1)

    def load(tab):
        a = d[f"bler_{cat}_t{tab}"].astype(np.float64)
        a = np.concatenate([np.ones(a.shape[:-1] + (pad,)), a], -1)
        av = d[f"avail_{cat}_t{tab}"].copy()
        raw = raw_all[fname.format(tab)]["category"]
        raw = raw[list(raw.keys())[0]]["index"][str(tab)]["MCS"]
        s_last = max(max(v["SNR_db"]) for v in raw.values())
        s_step = min(np.diff(v["SNR_db"]).min() for v in raw.values())
        inr = snr <= s_last + 1e-6
        for m in range(a.shape[0]):
            if av[m] and not (a[m, ci_ref, inr] <= 0.1).any():
                av[m] = False
        last = int(np.searchsorted(snr, s_last - 1e-6))
        j1 = int(np.searchsorted(snr, s_last - s_step - 1e-6))
        b1 = np.clip(a[..., j1], 1e-9, 1)
        b2 = np.clip(a[..., last], 1e-9, 1)
        slope = np.maximum((np.log10(b1) - np.log10(b2)) / (snr[last] - snr[j1]), 1.0)
        ext = np.log10(b2)[..., None] - slope[..., None] * (snr[None, None, last:] - snr[last])
        a[..., last:] = np.where(a[..., last:last + 1] > 0, 10 ** ext, 0.0)
        return a, av

    tabs = {t: load(t) for t in (1, 2)}
    for t in (1, 2):
        a, av = tabs[t]
        mcs = MCS_TABLES[t]
        for m in range(len(mcs)):
            if av[m]:
                continue
            o = 3 - t
            oa, oav = tabs[o]
            same = [k for k in range(len(MCS_TABLES[o])) if MCS_TABLES[o][k] == mcs[m] and oav[k]]
            if same:
                a[m] = oa[same[0]]
                continue
            cand = [k for k in range(len(mcs)) if av[k]]
            k = min(cand, key=lambda k: abs(k - m))
            steps = (gap(*mcs[m]) - gap(*mcs[k])) / (snr[1] - snr[0])
            xs = np.arange(len(snr)) - steps
            a[m] = np.stack([np.interp(xs, np.arange(len(snr)), row, left=1.0,
                                       right=0.0 if row[-1] < 1e-9 else row[-1]) for row in a[k]])
        if t == 1:
            tabs[1] = (a, np.ones_like(av))
    a = tabs[mcs_table][0][: len(MCS_TABLES[mcs_table])]
    a = np.minimum.accumulate(np.clip(a, 0, 1), axis=-1)
    return a.astype(np.float32), snr.astype(np.float32)


class PhyTables:
    """Host copy of every table the uplink step reads, for MCS table `mcs_table` (float32 unless stated).

    bler [M, C, G], snr_grid [G], cbs_axis [C], beta [M] (EESM), qm / r / se [M], thr [M, C] (smallest SINR with
    code-block BLER <= target per code-block-size point), thr_ref [M] (threshold of one 10-PRB RBG, 12 symbols),
    mcs_eq [M, max_tx + 1] int64, mcs_max, and scalars s0, ds (SNR grid origin and step), c0, dc (code-block axis)."""

    def __init__(self, mcs_table=1, bler_target=0.1, max_tx=4, mcs_cap=None, data=DATA):
        mcs = MCS_TABLES[mcs_table]
        self.M = M = len(mcs)
        self.qm = np.array([q for q, _ in mcs], dtype=_f32)
        self.r = np.array([c / 1024 for _, c in mcs], dtype=_f32)
        self.se = (self.qm * self.r).astype(_f32)
        with np.load(data, allow_pickle=False) as d:
            tab, grid = build_bler_table(d, mcs_table)
            self.cbs_axis = d["cbs_grid"].astype(_f32)
            self.beta = d[f"eesm_beta_t{mcs_table}"][:M].astype(_f32)
        self.bler = np.ascontiguousarray(tab[:M])
        self.snr_grid = grid
        self.C = self.bler.shape[1]
        self.G = self.bler.shape[2]
        self.s0 = float(self.snr_grid[0])
        self.ds = float(self.snr_grid[1] - self.snr_grid[0])
        self.c0 = float(self.cbs_axis[0])
        self.dc = float(self.cbs_axis[1] - self.cbs_axis[0])
        mt = max(max_tx, 2)
        eq = np.tile(np.arange(M)[:, None], (1, mt + 1))
        for m in range(1, M):
            for n in range(2, mt + 1):
                reff = mcs[m][1] / 1024 / n
                eq[m, n] = m - sum(1 for k in range(m) if mcs[k][0] == mcs[m][0] and mcs[k][1] / 1024 > reff)
        self.mcs_eq = eq.astype(np.int64)
        self.mcs_max = M - 1 if mcs_cap is None else min(int(mcs_cap), M - 1)
        self.target = float(bler_target)
        ok = self.bler <= _f32(bler_target)
        first = np.where(ok.any(-1), ok.argmax(-1), self.G - 1)
        self.thr = self.snr_grid[first]                                       # [M, C]
        tb = self.tbs_all(np.array(10.0), 12, 12)                             # one 10-PRB RBG
        cbs, _ = segment(tb, self.r.astype(np.float64))
        i0, wi = self.cidx(cbs.astype(_f32))
        m_ = np.arange(M)
        self.thr_ref = (self.thr[m_, i0] * (_f32(1) - wi) + self.thr[m_, i0 + 1] * wi).astype(_f32)

    def tbs_all(self, n_prb, nsym, dmrs=12, oh=0):
        """TBS (bits) of every MCS for PRB counts n_prb [...] -> [..., M] int64."""
        n = np.asarray(n_prb, dtype=np.float64)[..., None]
        return tbs_38214(self.qm.astype(np.float64), self.r.astype(np.float64), n, float(nsym), dmrs, oh)

    def cidx(self, cbs):
        """Code-block-size index i0 (int) and interpolation weight (float32) of cbs (float32), phy._cidx."""
        cbs = np.asarray(cbs, dtype=_f32)
        x = np.clip((cbs - _f32(self.c0)) / _f32(self.dc), _f32(0), _f32(self.C - 1)).astype(_f32)
        i0 = np.minimum(np.floor(x), _f32(self.C - 2)).astype(np.int64)
        return i0, (x - i0.astype(_f32)).astype(_f32)

    def la_tables(self, nprb_max, nsym, dmrs=12, oh=0):
        """Per-(PRBs, MCS) link-adaptation tables at nsym data symbols: tbs [N+1, M] int32, code-block index
        [N+1, M] int32, its weight [N+1, M] float32 and the number of code blocks [N+1, M] float32."""
        n = np.arange(nprb_max + 1, dtype=np.float64)
        tbs = self.tbs_all(n, nsym, dmrs, oh)
        cbs, c = segment(tbs, self.r.astype(np.float64)[None, :])
        i0, wi = self.cidx(cbs.astype(_f32))
        return (tbs.astype(np.int32), i0.astype(np.int32), wi.astype(_f32), c.astype(_f32))


def cqi_tables(tabs, mcs_table):
    """The 38.214 CQI report of the DL (cqi_table="38214", reference core/phy.py:366-391) for PhyTables tabs:
    (thr [15] float32, cqi_mcs [16] int64). thr[k - 1] is the SINR from which CQI k is reported: thr_ref of the MCS
    with the CQI's spectral efficiency, or of the nearest one shifted by the Shannon-gap difference
    10 log10((2^se - 1) / (2^se_mcs - 1)) (ties to the lower MCS), made non-decreasing. cqi_mcs[k] is the highest
    MCS <= mcs_max whose spectral efficiency does not exceed CQI k's (0 for CQI 0 and below every MCS)."""
    se_c = [q * r / 1024 for q, r in CQI_TABLES[mcs_table]]
    se_m = [float(x) for x in tabs.se]
    thr_m = [float(x) for x in tabs.thr_ref]

    def gap(e):
        return 10 * math.log10(2 ** e - 1)
    thr = []
    for e in se_c:
        m = min(range(tabs.M), key=lambda k: (abs(se_m[k] - e), k))
        thr.append(thr_m[m] + (0.0 if abs(se_m[m] - e) < 1e-6 else gap(e) - gap(se_m[m])))
    for k in range(1, len(thr)):
        thr[k] = max(thr[k], thr[k - 1])
    cqi_mcs = [0]
    for e in se_c:
        ok = [m for m in range(tabs.mcs_max + 1) if se_m[m] <= e + 1e-6]
        cqi_mcs.append(max(ok) if ok else 0)
    return np.array(thr, dtype=_f32), np.array(cqi_mcs, dtype=np.int64)

"""TR 38.901 (V17.0.0) large-scale parameters the engine's radio prologue needs (host side, Python floats).

Restates the scenario table and formulas of isaac_net/core/channels/tr38901.py:54-255 for the deterministic-LOS
case (tr38901_los "los" / "nlos") and the log-distance model of core/radio.py:265-273. The per-robot evaluation runs in
the HIP step kernel; this module supplies the scenario constants and the plane-wave shadowing fields' parameters.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

C_LIGHT = 3.0e8


@dataclass(frozen=True)
class Scenario:
    name: str
    h_bs: float
    los_corr_m: float
    sf_corr_los_m: float
    sf_corr_nlos_m: float


SCENARIOS = {
    "RMa": Scenario("RMa", 35.0, 60.0, 37.0, 120.0),
    "UMa": Scenario("UMa", 25.0, 50.0, 37.0, 50.0),
    "UMi": Scenario("UMi", 10.0, 50.0, 10.0, 13.0),
    "InH": Scenario("InH", 3.0, 10.0, 10.0, 6.0),
    "InF-SL": Scenario("InF-SL", 1.5, 5.0, 10.0, 10.0),
    "InF-DL": Scenario("InF-DL", 1.5, 1.0, 10.0, 10.0),
    "InF-SH": Scenario("InF-SH", 8.0, 5.0, 10.0, 10.0),
    "InF-DH": Scenario("InF-DH", 8.0, 1.0, 10.0, 10.0),
}
ALIASES = {"rma": "RMa", "uma": "UMa", "umi": "UMi", "inh": "InH", "inh_office": "InH", "inf_sl": "InF-SL",
           "inf_dl": "InF-DL", "inf_sh": "InF-SH", "inf_dh": "InF-DH"}
UT_HEIGHT_RANGE = {"UMa": (1.5, 22.5), "UMi": (1.5, 22.5), "RMa": (1.0, 10.0)}
# (sigma_SF LOS, sigma_SF NLOS) dB, Table 7.4.1-1 (RMa LOS depends on the breakpoint, handled by the caller)
SIGMA_SF = {"UMa": (4.0, 6.0), "UMi": (4.0, 7.82), "InH": (3.0, 8.03), "InF-SL": (4.3, 5.7),
            "InF-DL": (4.3, 7.2), "InF-SH": (4.3, 5.9), "InF-DH": (4.3, 4.0)}


def scenario_name(s):
    if s in SCENARIOS:
        return s
    key = s.lower().replace("-", "_")
    if key in ALIASES:
        return ALIASES[key]
    raise ValueError(f"unknown TR 38.901 scenario {s!r}; one of {tuple(SCENARIOS)}")


def check_heights(scn, h_bs, h_ut):
    """Table 7.4.1-1 applicability of UMa / UMi / RMa heights (reference tr38901.py:120-141)."""
    if scn in UT_HEIGHT_RANGE:
        lo, hi = UT_HEIGHT_RANGE[scn]
        if not lo - 1e-9 <= h_ut <= hi + 1e-9:
            raise ValueError(f"TR 38.901 {scn} path loss is defined for {lo:g} m <= ue_height_m <= {hi:g} m")
        if h_bs <= (1.0 if scn in ("UMa", "UMi") else 0.0):
            raise ValueError(f"TR 38.901 {scn}: BS height too low for a positive breakpoint distance")


def breakpoint_m(scn, fc_ghz, h_bs, h_ut):
    """d'_BP with h_E = 1 m for UMa / UMi (Note 1), d_BP for RMa (Note 5), inf indoors."""
    check_heights(scn, h_bs, h_ut)
    fc = fc_ghz * 1e9
    if scn == "RMa":
        return 2 * math.pi * h_bs * h_ut * fc / C_LIGHT
    if scn in ("UMa", "UMi"):
        return 4 * (h_bs - 1.0) * (h_ut - 1.0) * fc / C_LIGHT
    return math.inf


# ------------------------------------------------------------------ frequency-correlated fading
def _corr_sqrt(cfg, tau_ns):
    """L [..., S, S] (float32, torch) for rms delay spreads tau_ns [...] (ns, float64): the subband centres are the
    cumulated RBG widths (PRBs x 12 x SCS) less half a width (nr_engine.py:125-129); the correlation of subbands i, j
    is |1 / (1 + j 2 pi df tau)| = 1 / sqrt(1 + (2 pi df tau)^2) of an exponential power-delay profile
    (nr_engine.py:132-156); L is its Cholesky factor with rows scaled to unit norm, one diagonal jitter for the whole
    batch while any factorization fails (nr_engine.py:159-168), in float64, rounded once to float32."""
    import torch
    w = torch.tensor([float(x) for x in cfg.subband_prbs], dtype=torch.float64) * (12 * cfg.scs_khz * 1e3)
    f = torch.cumsum(w, 0) - w / 2
    x = 2 * math.pi * (f[:, None] - f[None, :]) * (torch.as_tensor(tau_ns, dtype=torch.float64) * 1e-9)[..., None, None]
    c = 1.0 / torch.sqrt(1.0 + x * x)
    eye = torch.eye(c.shape[-1], dtype=c.dtype)
    for eps in (0.0, 1e-12, 1e-10, 1e-8, 1e-6):
        L, info = torch.linalg.cholesky_ex(c + eps * eye)
        if not bool((info != 0).any()):
            return (L / L.norm(dim=-1, keepdim=True)).float().contiguous()
    raise ValueError("subband correlation matrix is not positive definite")


def subband_fading_sqrt(cfg):
    """The lower-triangular square root L [S,S] (float32, torch) of the subband correlation of the fading innovations
    for the fixed rms delay spread cfg.fading_delay_spread_ns, or None (freq_corr_mode is not "fixed")."""
    if cfg.freq_corr_mode != "fixed":
        return None
    return _corr_sqrt(cfg, cfg.fading_delay_spread_ns)


def delay_spread_grid(cfg):
    """Per-link delay spreads (freq_corr_mode "los", nr_engine.py:320-340): the log grid of fading_ds_grid
    (lo ns, hi ns, G points; torch.logspace in float64) and its square roots L [G,S,S] float32."""
    import torch
    lo, hi, G = cfg.fading_ds_grid
    grid = torch.logspace(math.log10(lo), math.log10(hi), int(G), dtype=torch.float64)
    return grid, _corr_sqrt(cfg, grid)


# mean and spread of lgDS = log10(DS / 1 s), TR 38.901 V17.0.0 Table 7.5-6 (fc in GHz; the tables' frequency floors,
# 2 GHz for UMi, 6 GHz for UMa and InH), as (LOS, NLOS) pairs of (mu, sigma)
def lg_ds_params(scn, fc_ghz, los):
    """(mu_lgDS, sigma_lgDS) of scenario scn in the LOS or NLOS state (nr_engine.py:92-113), Python floats."""
    lg = math.log10
    if scn == "UMi":
        f = lg(1 + max(fc_ghz, 2.0))
        return (-0.24 * f - 7.14, 0.38) if los else (-0.24 * f - 6.83, 0.16 * f + 0.28)
    if scn == "UMa":
        f = lg(max(fc_ghz, 6.0))
        return (-6.955 - 0.0963 * f, 0.66) if los else (-6.28 - 0.204 * f, 0.39)
    if scn == "InH":
        f = lg(1 + max(fc_ghz, 6.0))
        return (-0.01 * f - 7.692, 0.18) if los else (-0.28 * f - 7.173, 0.10 * f + 0.055)
    raise ValueError(f"per-link delay spreads: no lgDS table for scenario {scn}")


# Rician K-factor of LOS links, (mu_K, sigma_K) in dB per scenario: TR 38.901 V17.0.0 Table 7.5-6 (UMi-Street Canyon
# 9 / 5, UMa 9 / 3.5, RMa 7 / 4, Indoor-Office 7 / 4, InF 7 / 8; K is defined for LOS links only)
RICIAN_K_DB = {"UMi": (9.0, 5.0), "UMa": (9.0, 3.5), "RMa": (7.0, 4.0), "InH": (7.0, 4.0),
               "InF-SL": (7.0, 8.0), "InF-DL": (7.0, 8.0), "InF-SH": (7.0, 8.0), "InF-DH": (7.0, 8.0)}


def sum_of_cosines_cdf_table(K, n=1 << 16, seed=0):
    """Sorted samples [n] (float32, torch) of sqrt(2/K) sum_k cos(U_k), U_k ~ U(0, 2 pi) drawn from a CPU generator
    seeded with seed, in float64 (fields.py:94-100): the empirical marginal of a unit plane-wave field, through which
    the LOS-state field becomes a U(0, 1) value (the kernels search it as torch.searchsorted does)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    z = math.sqrt(2 / K) * torch.cos(torch.rand(n, K, generator=g, dtype=torch.float64) * 2 * math.pi).sum(-1)
    return z.sort().values.float()

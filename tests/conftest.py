"""pytest setup: the `gpu` marker, and the product package loaded from its directory (isaac-net_amd/)."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def load_package():
    if "isaac_net_amd" in sys.modules:
        return sys.modules["isaac_net_amd"]
    d = os.path.join(ROOT, "isaac-net_amd")
    spec = importlib.util.spec_from_file_location("isaac_net_amd", os.path.join(d, "__init__.py"),
                                                  submodule_search_locations=[d])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["isaac_net_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libinet_nr.so")
    config.addinivalue_line("markers", "slow: longer CPU runs")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


# one cell; s14 / s18_ir / s10_w2: 14, 18 and 10 RBGs (106, 273 and 78 PRB at the 38.214 RBG sizes); w4: envs of
# 200 robots (four wavefronts); lena_pf: the PF
# average moved per RBG grant and frozen outside the active list; wb_pc / pc1: whole-band UL power and UL power control
# at one cell; tdma / amc_prev / lena_v2 / wb_amc: TDMA UL retransmissions and the UL MCS on the previous PUSCH's PRBs,
# alone, with every other switch, and with whole-band power; fcorr / fcorr_w2: frequency-correlated fading (fixed delay
# spread), 13 RBGs and 8 RBGs on two-wavefront envs; rice_los / rice_snr: Rician K from the LOS state (poses: the
# link's LOS draw; SNR input: no LOS state, K = 0); los_sto (and _dl, _mc): the TR 38.901 stochastic LOS state;
# rice_sto (and _dl, _slow): Rician K from the stochastic LOS state, ramps of 4, 0 and 50 slots; fcorr_los (and _dl,
# _rice): per-link delay spreads from the LOS state (13, 14 and 18 RBGs); sto64 / sto100: the stochastic LOS state,
# Rician K from it and per-link delay spreads on 64-robot envs (one wavefront) and 100-robot envs (two wavefronts)
CASES = ["c1", "c2", "c2heavy", "snr_drop", "snr3_ir", "logd_meandb", "c5", "s14", "s18_ir", "s10_w2", "lena_pf",
         "wb_pc", "pc1", "w4", "s14_w4", "s18_w4", "tdma", "amc_prev", "lena_v2", "wb_amc", "fcorr", "fcorr_w2",
         "rice_los", "rice_snr", "los_sto", "rice_sto", "rice_sto_slow",
         "fcorr_los", "fcorr_los_rice", "sto64", "sto100", "dop", "wb_pf", "wb_maxci_md"]
# the downlink on (NRConfig(dl=True)); s17_dl: 17 RBGs; lena_dl: the frozen PF average on both links
DL_CASES = ["dl_c2", "dl_snr", "dl_ir_rr", "s17_dl", "lena_dl", "fcorr_dl", "rice_los_dl", "los_sto_dl",
            "rice_sto_dl", "fcorr_los_dl", "dop_vel_dl", "pfwb_dl", "dl_w2", "dl_w2_snr"]
MC_CASES = ["mc3", "mc3_ho", "mc2", "mc2_ho", "mc2_lena", "fcorr_mc2", "los_sto_mc", "mc2_rice",
            "mc3_rice_sto", "mc3_flush", "mc3_a3floor", "mc2_fcorr_los", "mc3_rice64", "mc3_rice48",
            "mc3_ho48", "mc3_rice48c", "mc3_rice32", "mc2_dop", "mc2_wb", "mc3_pg", "mc3_rlf", "mc2_rlf_flush",
            "mc4", "mc5", "mc6", "mc7"]
# several cells (NRConfig(n_cells=2..7)), uplink; mc4..mc7: four to seven hex cells; mc3_flush: ho_rlc="flush"; mc3_a3floor: the A3 admission floor;
# mc2_fcorr_los: per-link delay spreads; mc3_rice64 / mc3_rice48: Rician links on 64- and 48-robot envs

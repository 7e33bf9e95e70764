"""ctypes binding of libinet_nr.so (include/inet_nr.h, include/inet_wifi.h). No torch types cross the ABI: only
pointers and sizes."""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# INET_NR_LIB names another build of the same sources (bench.py --phase-clocks loads libinet_nr_phase.so)
LIB_PATH = os.environ.get("INET_NR_LIB") or os.path.join(HERE, "libinet_nr.so")

P = C.c_void_p
i32, i64, f32, u32 = C.c_int32, C.c_int64, C.c_float, C.c_uint32


class InetNrState(C.Structure):
    _fields_ = [(n, P) for n in (
        "sent", "floor_", "bsr", "sr_t", "last_tx", "olla", "avg", "enq", "qlen", "csi", "h_re", "h_im",
        "h_meta", "h_lo", "h_hi", "h_ready", "h_tbs", "h_comb", "h_lexp", "h_nrb",
        "q_cap", "q_start", "q_end", "q_fin", "q_meta", "q_hid", "spec_re", "spec_im", "k_lin",
        "env_id", "episode", "ctr_step", "ctr_submit", "epoch", "field", "ctr", "hist", "clock", "base", "last_nprb", "k_los", "k_from", "k_g0", "k_fresh", "fc_idx", "fc_idl", "fc_idn",
        "prev_pos", "has_prev", "rho_ms")]


class InetNrTables(C.Structure):
    _fields_ = [(n, P) for n in ("bler", "thr_ref", "se", "beta", "rate", "mcs_eq", "la_tbs", "la_ci0", "la_cwi",
                                 "la_ncb", "w", "logw", "wdb")] + \
               [(n, f32) for n in ("s0", "ds", "c0", "dc")] + \
               [(n, i32) for n in ("M", "C", "G", "NPRB", "EQW", "mcs_max", "thr_monotone", "pad")]


class InetNrParams(C.Structure):
    _fields_ = [(n, i32) for n in (
        "E", "R", "S", "P", "F", "N", "sched", "comb", "eesm", "harq_drop", "olla", "phr_cap", "retx_prio", "rician",
        "fading", "purge", "input_kind", "radio_model", "out_ref", "max_tx", "sr_delay", "ul_rtt", "rlc_retx",
        "timeout", "tb_oh", "n_fields", "n_modes", "seed_key", "n_data", "n_cells", "rebase_at", "pf_rbg", "pf_freeze",
        "whole_band", "pc1_on", "retx_tdma", "amc_prev", "fc_on", "k_from_los", "los_sto", "plos_scn", "k_ramp", "fc_G",
        "doppler", "pf_wb")] + \
               [(n, f32) for n in (
        "olla_up", "olla_dn", "pf_a", "pf_b", "target", "phr_min", "snr_ref_prbs", "w0", "ref_off", "noise_prb",
        "ue_tx", "subband_noise", "gnb_x", "gnb_y", "hh2", "dbp", "pl_a", "pl_n1", "pl_c20", "pl_c2", "nl_b1",
        "nl_b0", "nl_c", "nl_d", "sig", "amp", "pl_const", "pl_exp10", "proc_off_hi", "proc_off_lo", "wb_db", "pc_p0",
        "pc_alpha", "k_mu", "k_sigma", "sig_nlos", "k_rinv", "ds_mu_n", "ds_sig_n", "ds_mu_l", "ds_sig_l", "ds_c1",
        "ds_c2", "dop_floor", "dop_kf", "dop_kx", "dop_dt")] + [("fc_L", P), ("los_cdf", P), ("fc_tab", P), ("vel", P)]


class InetNrOutputs(C.Structure):
    _fields_ = [(n, P) for n in ("delivered", "timed_out", "dropped", "cap", "cls", "cap32", "cls8", "delay",
                                 "newest", "queue_len", "serving_cell", "queue_bytes", "sinr_db", "det_env", "t")]


class InetNrDlState(C.Structure):
    _fields_ = [(n, P) for n in (
        "sent", "floor_", "last_tx", "olla", "avg", "enq", "qlen", "csi", "h_meta", "h_lo", "h_hi", "h_ready", "h_tbs",
        "h_comb", "h_lexp", "h_nrb", "q_cap", "q_start", "q_end", "q_fin", "q_meta", "newest", "ctr", "hist",
        "out_newest", "out_queue_len", "out_delay", "cqi_thr", "cqi_mcs", "base")] + \
               [("gnb_proc", i32), ("snr_offset", i32), ("ref_off", f32), ("noise_prb", f32), ("snr_off", f32),
                ("pad", i32)]


MAX_C = 7


class InetNrCells(C.Structure):
    _fields_ = [(n, P) for n in ("serv", "a3_cand", "a3_cnt", "ho_end", "n_ho", "pending", "ni_ul", "ion")] + \
               [("gnb_xy", f32 * (2 * MAX_C))] + \
               [(n, i32) for n in ("C", "ttt", "ho_int", "ho_flush", "use_int", "pc_on", "has_floor")] + \
               [(n, f32) for n in ("a3_off", "a3_hyst", "floor_rx", "noise_mw", "ref_db", "li_a", "li_b", "pc_p0",
                                   "pc_alpha")] + \
               [(n, P) for n in ("rlf_active", "oos_cnt", "is_cnt", "t310_end", "t311_end", "reest_end", "reest_cell",
                                 "n_rlf", "rlf_ctr", "out_rlf")] + \
               [(n, i32) for n in ("rlf", "rlf_flush", "n310", "n311", "t310", "t311", "reest")] + \
               [("qout", f32), ("qin", f32), ("pad_r", i32)]


class InetNrArrivals(C.Structure):
    _fields_ = [("counts", P), ("sizes", P), ("accepted", P), ("n_cls", i32), ("discard_pdcp", i32),
                ("pkt_payload", i32), ("pkt_overhead", i32)]


class InetWifiState(C.Structure):
    _fields_ = [(n, P) for n in (
        "cap", "cls", "det", "hid", "rem", "f_nact", "f_snr", "f_own", "qlen", "last_snr", "roam_left", "serv",
        "att_n", "att_logp", "credit", "tau", "clock", "last_hid", "pending", "env_id", "episode", "ctr_step",
        "ctr_submit", "field", "calls")]


WIFI_MAX_M, WIFI_MAX_CLS, WIFI_MAX_NACC, WIFI_MAX_A = 16, 16, 128, 8


class InetWifiParams(C.Structure):
    _fields_ = [(n, i32) for n in (
        "E", "R", "F", "K", "M", "L", "n_cls", "n_acc_max", "fp_iters", "timeout", "access_noise", "rts_cts",
        "coll_ack", "per_class_ac", "no_aggr", "radio_model", "n_fields", "n_modes", "seed_key", "roam_sub", "bg_ac",
        "envs_per_wave", "spectrum", "pad0")] + \
               [(n, f32) for n in (
        "noise_dbm", "roam_hyst", "damp", "fer1", "dt_us", "tau0", "slot_us", "sifs_us", "pre", "tsym", "ovh1",
        "t_ack", "t_rts", "t_cts", "hs", "ampdu_lim", "msdu_payload", "ppdu_max", "bg_w", "bg_rate", "bg_B")] + \
               [("dcorr", f32 * 3), ("rates", f32 * WIFI_MAX_M), ("thr", f32 * WIFI_MAX_M),
                ("mcs_ids", i32 * WIFI_MAX_M), ("ac_W0", f32 * 5), ("ac_Wmax", f32 * 5), ("ac_aifsn", f32 * 5),
                ("ac_txop", f32 * 5), ("cls_ac", i32 * (WIFI_MAX_CLS + 1)), ("sizes", f32 * WIFI_MAX_CLS),
                ("lgamma", f32 * WIFI_MAX_NACC)] + \
               [(n, f32) for n in (
        "gnb_x", "gnb_y", "hh2", "dbp", "pl_a", "pl_n1", "pl_c20", "pl_c2", "nl_b1", "nl_b0", "nl_c", "nl_d", "sig",
        "amp", "pl_const", "pl_exp10", "ue_tx")] + \
               [("los_sto", i32), ("plos_scn", i32), ("sig_nlos", f32), ("A", i32), ("los_cdf", P),
                ("ap_xy", f32 * (2 * WIFI_MAX_A)), ("step_counts", P), ("step_accepted", P),
                ("step_n_cls", i32), ("n_dom", i32), ("ap_dom", i32 * WIFI_MAX_A), ("Z", i32),
                ("hidden", i32), ("cca_dbm", f32), ("sta_c0", f32), ("sta_c1", f32), ("sense", P)]


class InetWifiOutputs(C.Structure):
    _fields_ = [(n, P) for n in ("delivered", "timed_out", "cap", "cls", "delay", "newest", "queue_len",
                                 "serving_cell", "mcs", "queue_bytes", "sinr_db", "rate_mbps", "access_ms", "p_fail",
                                 "busy", "det_env", "t")]


class InetDcfState(C.Structure):
    _fields_ = [(n, P) for n in ("b", "stage", "had", "t_idle")]


class InetDcfParams(C.Structure):
    _fields_ = [("ndbps", i32 * WIFI_MAX_M)] + [(n, i32) for n in (
        "T", "tsym", "pre", "sifs", "slot", "t_ack", "t_rts", "t_cts", "W0", "Wmax", "aifsn", "ovh", "payload")] + \
               [("fer", f32)]


ROW_DTYPE_FIELDS = ("rel", "nsym_idx", "flags", "re_prb", "rho", "c1", "salt_fade", "salt_bler")   # 8 x 4 bytes
ERRORS = {-1: "invalid argument (size or pointer)", -2: "unsupported configuration for this build",
          -3: "HIP launch failed"}

ABI_VERSION = 15
WIFI_ABI_VERSION = 7
_LIB = None


def load(path=LIB_PATH):
    """Load the library (built in-tree by build.py); raises if it is missing: there is no CPU fallback."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `python isaac-net_amd/build.py` (hipcc, gfx950)")
    # torch ships its own HIP runtime: it must be the one this library binds to (loaded first, the library would bind
    # the system's, and its launches on torch's streams would fail)
    import torch  # noqa: F401
    lib = C.CDLL(path)
    lib.inet_nr_abi_version.restype = i32
    lib.inet_nr_build_info.restype = C.c_char_p
    lib.inet_nr_step.argtypes = [C.POINTER(InetNrState), C.POINTER(InetNrTables), C.POINTER(InetNrParams), P, i32,
                                 i64, P, P, C.POINTER(InetNrOutputs), P]
    lib.inet_nr_step.restype = i32
    lib.inet_nr_submit.argtypes = [C.POINTER(InetNrState), C.POINTER(InetNrParams), i64, P, P, P, P, i32, P, i32, i32,
                                   i32, P, P]
    lib.inet_nr_submit.restype = i32
    lib.inet_nr_reset.argtypes = [C.POINTER(InetNrState), C.POINTER(InetNrParams), P, i64, f32, C.POINTER(f32), i32,
                                  P]
    lib.inet_nr_reset.restype = i32
    lib.inet_nr_submit_step.argtypes = [C.POINTER(InetNrState), C.POINTER(InetNrTables), C.POINTER(InetNrParams), P,
                                        i32, i64, P, P, C.POINTER(InetNrOutputs), C.POINTER(InetNrArrivals), P]
    lib.inet_nr_submit_step.restype = i32
    lib.inet_nr_dl_step.argtypes = [C.POINTER(InetNrState), C.POINTER(InetNrDlState), C.POINTER(InetNrTables),
                                    C.POINTER(InetNrParams), P, i32, i64, P, P]
    lib.inet_nr_dl_step.restype = i32
    lib.inet_nr_dl_submit.argtypes = [C.POINTER(InetNrState), C.POINTER(InetNrDlState), C.POINTER(InetNrParams), i64,
                                      P, P, i32, i32, i32, P, P]
    lib.inet_nr_dl_submit.restype = i32
    lib.inet_nr_dl_reset.argtypes = [C.POINTER(InetNrDlState), C.POINTER(InetNrParams), P, P]
    lib.inet_nr_dl_reset.restype = i32
    lib.inet_nr_step_cells.argtypes = [C.POINTER(InetNrState), C.POINTER(InetNrCells), C.POINTER(InetNrTables),
                                       C.POINTER(InetNrParams), P, i32, i64, P, P, C.POINTER(InetNrOutputs),
                                       C.POINTER(InetNrArrivals), P]
    lib.inet_nr_step_cells.restype = i32
    lib.inet_nr_cells_reset.argtypes = [C.POINTER(InetNrCells), C.POINTER(InetNrParams), P, P]
    lib.inet_nr_cells_reset.restype = i32
    lib.inet_wifi_abi_version.restype = i32
    lib.inet_wifi_step.argtypes = [C.POINTER(InetWifiState), C.POINTER(InetWifiParams), P, i32, P, P,
                                   C.POINTER(InetWifiOutputs), P]
    lib.inet_wifi_step.restype = i32
    lib.inet_wifi_submit.argtypes = [C.POINTER(InetWifiState), C.POINTER(InetWifiParams), P, P, P, P, P, P, i32, P, P]
    lib.inet_wifi_submit.restype = i32
    lib.inet_wifi_reset.argtypes = [C.POINTER(InetWifiState), C.POINTER(InetWifiParams), P, P]
    lib.inet_wifi_reset.restype = i32
    lib.inet_wifi_dcf_step.argtypes = [C.POINTER(InetWifiState), C.POINTER(InetDcfState), C.POINTER(InetWifiParams),
                                       C.POINTER(InetDcfParams), P, i32, P, P, C.POINTER(InetWifiOutputs), P]
    lib.inet_wifi_dcf_step.restype = i32
    lib.inet_wifi_dcf_reset.argtypes = [C.POINTER(InetWifiState), C.POINTER(InetDcfState), C.POINTER(InetWifiParams),
                                        C.POINTER(InetDcfParams), P, P]
    lib.inet_wifi_dcf_reset.restype = i32
    if lib.inet_nr_abi_version() != ABI_VERSION or lib.inet_wifi_abi_version() != WIFI_ABI_VERSION:
        raise RuntimeError("libinet_nr.so ABI version mismatch; rebuild it")
    from .build import source_hash
    built = lib.inet_nr_build_info().decode().rsplit("src=", 1)[-1]
    if built != source_hash():
        raise RuntimeError(f"{path} was built from other sources (src={built}, the tree's is {source_hash()}): "
                           "rebuild it with `python isaac-net_amd/build.py`")
    _LIB = lib
    return lib


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: {ERRORS.get(rc, rc)}")

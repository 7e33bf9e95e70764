"""Write the golden vectors that pin the oracle (run in the build container only; needs the reference checkout).

The reference package (isaac-net, pure Python + PyTorch) is imported from /root/reference and its CPU
`backend="reference"` NR engine is run on small scenarios. What is written is data only: per-step inputs,
the step output dicts, the engine state after every step, and the processed PHY tables. Nothing from the
reference is copied. The vectors pin what no closed form or known answer pins:

  * multi-slot trajectories of NRNet.step / step_rx (scheduler, link adaptation, HARQ, RLC interplay, CPU argsort
    tie order), isaac_net/core/nr_engine.py:613-668, core/mac.py:228-508;
  * the processed BLER table and thr_ref (core/phy.py:234-243, 405-482);
  * the plane-wave shadowing draws of the radio (core/radio.py:185-189, core/channels/fields.py:38-64);
  * the eager _finish / compaction output layout (core/nr_engine.py:843-888, core/queues.py:105-110);
  * the statistics of NRNet with log_stats on (core/nr_engine.py:440-446, 885-914): collect(), queued(), refused_env;
  * level WIFI trajectories (core/wifi/engine.py:100-403 WifiNet on the levels/base.py:43-360 FIFO): the mean-field
    solve per sub-step (core/wifi/meanfield.py:187-209), the Poisson / renewal access counts, the FIFO service and the
    retry-limit loss, with SNR inputs and with poses through the APs' radio.

Usage:  python tests/golden/make_fixtures.py            (writes tests/golden/*.npz)
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import sys

import numpy as np
import torch

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def _ref():
    sys.path.insert(0, REF)
    from isaac_net.core.config import NRConfig
    from isaac_net.core.engine import make_engine
    from isaac_net.core.nr_fast import state_dict
    from isaac_net.core.traffic import Requests
    return NRConfig, make_engine, state_dict, Requests


# ---------------------------------------------------------------------------------------------- scenarios
# Each case: config overrides, E, R, steps, input kind, pose / traffic generator parameters, resets.
CASES = {
    # the CPU-runnable NR plumbing scenario, shrunk: RR, K=4 UL slots, 1500 B, Poisson 0.5
    "c1": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="rr", n_harq=4,
                        max_harq_tx=4, frame_buffer=16, msg_sizes=(1500.0,), fading_rho_per_ms=0.0,
                        channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                        cell_positions_m=((50.0, 50.0),), gnb_height_m=10.0),
               E=4, R=8, steps=40, kind="pose", arena=100.0, walk=0.0, rates=(0.5,), resets={25: [2]}),
    # the RL-scale scenario, shrunk: PF alpha 0.01, Rician K 3 dB, two classes, random walk
    "c2": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=25.0, scheduler="pf", pf_window=100.0,
                        n_harq=8, max_harq_tx=5, frame_buffer=32, msg_sizes=(200.0, 4000.0), fading_rho_per_ms=0.0,
                        fading_rician=True, rician_k_db=3.0, channel="tr38901", tr38901_scenario="UMi",
                        tr38901_los="los", cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
               E=4, R=8, steps=40, kind="pose", arena=200.0, walk=0.025, rates=(0.8, 0.1), resets={20: [1]}),
    # heavy load on the config-2 MAC: contention, retransmissions, exhaustion, purge timeouts
    "c2heavy": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=25.0, scheduler="pf",
                             n_harq=8, max_harq_tx=3, frame_buffer=12, msg_sizes=(2000.0, 9000.0),
                             fading_rho_per_ms=0.0, fading_rician=True, rician_k_db=3.0, timeout_steps=3,
                             channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                             cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
                    E=4, R=16, steps=30, kind="pose", arena=400.0, walk=0.5, rates=(2.0, 0.7), resets={12: [0, 3]}),
    # SNR input, correlated AR(1) Rayleigh fading, RLC UM drop, small FIFO (overflow), max C/I
    "snr_drop": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="maxci", n_harq=4, max_harq_tx=2,
                              harq_fail="drop", frame_buffer=6, msg_sizes=(3000.0, 500.0), timeout_steps=6),
                     E=3, R=8, steps=30, kind="snr", snr=(-4.0, 14.0), rates=(1.2, 0.6), resets={17: [1]}),
    # per-subband SNR input, IR combining, no retransmission priority, no PHR cap, stack processing offset
    "snr3_ir": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="pf", n_harq=4, max_harq_tx=3,
                             harq_combining="ir_lena", retx_priority=False, phr_cap=False, frame_buffer=8,
                             msg_sizes=(2500.0,), proc_offset_ms=4.0, discard="none"),
                    E=3, R=8, steps=30, kind="snr3", snr=(-2.0, 16.0), rates=(1.0,), resets={}),
    # log-distance radio, mean-dB effective SINR without combining, round robin, PDCP discard on arrival
    "logd_meandb": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=5.0, scheduler="rr", n_harq=2, max_harq_tx=4,
                                 harq_combining="none", eff_sinr="mean_db", frame_buffer=10, msg_sizes=(1200.0,),
                                 discard="pdcp_arrival", timeout_steps=4, cell_positions_m=((20.0, 30.0),)),
                        E=3, R=8, steps=30, kind="pose", arena=120.0, walk=1.0, rates=(1.3,), resets={9: [0, 2]}),
    # downlink on (NRNet with DlMac): the RL-scale MAC with PF, Rician fading, CQI every 10 slots, two DL classes
    "dl_c2": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=25.0, scheduler="pf", pf_window=100.0,
                           n_harq=8, max_harq_tx=5, frame_buffer=16, msg_sizes=(200.0, 4000.0), fading_rho_per_ms=0.0,
                           fading_rician=True, rician_k_db=3.0, channel="tr38901", tr38901_scenario="UMi",
                           tr38901_los="los", cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0, dl=True),
                  E=4, R=8, steps=40, kind="pose", arena=200.0, walk=0.025, rates=(0.8, 0.1),
                  dl_sizes=(6000.0, 30000.0), dl_rates=(0.6, 0.2), resets={20: [1]}),
    # downlink with SNR input: correlated AR(1) fading, 38.214 CQI every 5 slots, K1 = 3, DL MCS cap, max C/I, RLC UM
    # drop, small FIFOs (DL overflow), DL SNR offset
    "dl_snr": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="maxci", n_harq=4, max_harq_tx=3,
                            harq_fail="drop", frame_buffer=6, msg_sizes=(3000.0,), timeout_steps=6,
                            fading_rho_per_ms=0.9, dl=True, cqi_table="38214", cqi_period_slots=5, k1=3,
                            dl_mcs_max=20, dl_snr_offset_db=6.0),
                   E=3, R=8, steps=30, kind="snr", snr=(-4.0, 14.0), rates=(0.8,), dl_sizes=(9000.0, 1500.0),
                   dl_rates=(0.9, 0.8), resets={17: [1]}),
    # the downlink with envs of 72 and 100 robots (two wavefronts per env): dl_c2's link on poses, dl_snr's on SNR
    "dl_w2": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=25.0, scheduler="pf", pf_window=100.0,
                           n_harq=8, max_harq_tx=5, frame_buffer=16, msg_sizes=(200.0, 4000.0), fading_rho_per_ms=0.0,
                           fading_rician=True, rician_k_db=3.0, channel="tr38901", tr38901_scenario="UMi",
                           tr38901_los="los", cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0, dl=True),
                  E=2, R=72, steps=20, kind="pose", arena=200.0, walk=0.025, rates=(0.5, 0.1),
                  dl_sizes=(6000.0, 30000.0), dl_rates=(0.4, 0.1), resets={11: [1]}),
    "dl_w2_snr": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="maxci", n_harq=4, max_harq_tx=3,
                               harq_fail="drop", frame_buffer=6, msg_sizes=(3000.0,), timeout_steps=6,
                               fading_rho_per_ms=0.9, dl=True, cqi_table="38214", cqi_period_slots=5, k1=3,
                               dl_mcs_max=20, dl_snr_offset_db=6.0),
                      E=2, R=100, steps=20, kind="snr", snr=(-4.0, 14.0), rates=(0.5,), dl_sizes=(9000.0, 1500.0),
                      dl_rates=(0.5, 0.4), resets={9: [0]}),
    # downlink with per-subband SNR: IR combining, no retransmission priority, round robin, PDCP discard, gNB
    # processing 2 slots
    "dl_ir_rr": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="rr", n_harq=4, max_harq_tx=3,
                              harq_combining="ir_lena", retx_priority=False, frame_buffer=8, msg_sizes=(2500.0,),
                              discard="pdcp_arrival", timeout_steps=5, gnb_proc_slots=2, dl=True),
                     E=3, R=8, steps=30, kind="snr3", snr=(-2.0, 16.0), rates=(0.7,), dl_sizes=(5000.0,),
                     dl_rates=(1.1,), resets={11: [0, 2]}),
    # config 5 shrunk: 128 robots per env (two wavefronts per env on the GPU), 273 PRB in 8 RBGs of 35, i.i.d.
    # Rayleigh fading per subband and slot, PF, K = 20 UL slots per step, 16 HARQ processes, 800 B, FIFO 16
    "c5": dict(cfg=dict(mu=1, n_prb=273, rbg_size=35, tdd_pattern="DDDSU", control_step_ms=50.0, scheduler="pf",
                        n_harq=16, max_harq_tx=4, frame_buffer=16, msg_sizes=(800.0,), fading_rho_per_ms=0.0,
                        channel="tr38901", tr38901_scenario="UMi", tr38901_los="los", cell_positions_m=((100.0, 100.0),),
                        gnb_height_m=10.0),
               E=2, R=128, steps=8, kind="pose", arena=200.0, walk=1.0, rates=(0.6,), resets={5: [1]}),
    # several cells (NRNet.step_cells): config 3 shrunk (3 hex cells 150 m apart, 106 PRB, PF, thermal noise with
    # same-slot UL interference, fractional UL power control, correlated fading on every link, no handover)
    "mc3": dict(cfg=dict(mu=1, n_prb=106, tdd_pattern="DDDSU", control_step_ms=25.0, scheduler="pf", n_harq=8,
                         max_harq_tx=5, frame_buffer=12, msg_sizes=(1200.0,), n_cells=3, cell_layout="hex",
                         cell_isd_m=150.0, noise_model="thermal", a3_offset_db=float("inf"), channel="tr38901",
                         tr38901_scenario="UMi", tr38901_los="los", gnb_height_m=10.0),
                E=2, R=16, steps=30, kind="pose", arena=260.0, walk=0.5, rates=(0.6,), resets={17: [1]}),
    # several cells with A3 handovers (fast motion, short time-to-trigger and interruption), maxCI, RLC UM drop,
    # i.i.d. fading, log-distance radio, an EWMA N+I estimate
    "mc3_ho": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="maxci", n_harq=4,
                            max_harq_tx=3, harq_fail="drop", frame_buffer=8, msg_sizes=(2500.0, 400.0), n_cells=3,
                            cell_layout="hex", cell_isd_m=120.0, noise_model="thermal", a3_ttt_ms=20.0,
                            ho_interruption_ms=5.0, li_alpha=0.5, fading_rho_per_ms=0.0,
                            cell_center_m=(60.0, 60.0)),
                   E=3, R=8, steps=40, kind="pose", arena=200.0, walk=6.0, rates=(0.5, 1.0), resets={25: [0]}),
    # one cell at other RBG counts: 106 PRB (14 RBGs of 8), PF, Rician fading, poses, two classes, 16 robots
    "s14": dict(cfg=dict(mu=1, n_prb=106, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                         max_harq_tx=4, frame_buffer=16, msg_sizes=(300.0, 3000.0), fading_rho_per_ms=0.0,
                         fading_rician=True, rician_k_db=3.0, channel="tr38901", tr38901_scenario="UMi",
                         tr38901_los="los", cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
                E=3, R=16, steps=30, kind="pose", arena=200.0, walk=1.0, rates=(1.0, 0.3), resets={14: [1]}),
    # 273 PRB at the default RBG size (18 RBGs of 16, the last one of 1 PRB), per-subband SNR, HARQ-IR, max C/I
    "s18_ir": dict(cfg=dict(mu=1, n_prb=273, control_step_ms=10.0, scheduler="maxci", n_harq=4, max_harq_tx=3,
                            harq_combining="ir_lena", frame_buffer=8, msg_sizes=(6000.0,), fading_rho_per_ms=0.3),
                   E=3, R=8, steps=25, kind="snr3", subbands=18, snr=(-4.0, 14.0), rates=(0.9,), resets={12: [2]}),
    # 133 PRB (17 RBGs of 8, the last of 5 PRB) with the downlink, SNR input, round robin
    "s17_dl": dict(cfg=dict(mu=1, n_prb=133, control_step_ms=10.0, scheduler="rr", n_harq=4, max_harq_tx=3,
                            frame_buffer=8, msg_sizes=(2000.0,), fading_rho_per_ms=0.0, dl=True),
                   E=3, R=8, steps=25, kind="snr", snr=(-2.0, 16.0), rates=(0.8,), dl_sizes=(7000.0,),
                   dl_rates=(0.7,), resets={9: [0]}),
    # 78 PRB (10 RBGs of 8, the last of 6 PRB) on envs of 96 robots (two wavefronts), PF, poses
    "s10_w2": dict(cfg=dict(mu=1, n_prb=78, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                            max_harq_tx=4, frame_buffer=8, msg_sizes=(700.0,), fading_rho_per_ms=0.0,
                            channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                            cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
                   E=2, R=96, steps=10, kind="pose", arena=200.0, walk=1.0, rates=(0.4,), resets={6: [1]}),
    # 106 PRB (14 RBGs of 8) and 273 PRB (18 RBGs of 16) on envs of 160 and 144 robots (four wavefronts)
    "s14_w4": dict(cfg=dict(mu=1, n_prb=106, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                            max_harq_tx=4, frame_buffer=8, msg_sizes=(600.0,), fading_rho_per_ms=0.5,
                            channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                            cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
                   E=2, R=160, steps=8, kind="pose", arena=200.0, walk=1.0, rates=(0.3,), resets={5: [1]}),
    "s18_w4": dict(cfg=dict(mu=1, n_prb=273, control_step_ms=10.0, scheduler="maxci", n_harq=4, max_harq_tx=3,
                            harq_combining="ir_lena", frame_buffer=8, msg_sizes=(4000.0,), fading_rho_per_ms=0.3),
                   E=2, R=144, steps=8, kind="snr", snr=(-4.0, 14.0), rates=(0.4,), resets={4: [0]}),
    # two cells per env: 14 RBGs, PF, thermal noise with UL interference, power control, correlated fading
    "mc2": dict(cfg=dict(mu=1, n_prb=106, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                         max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=2, cell_layout="hex",
                         cell_isd_m=120.0, noise_model="thermal", a3_offset_db=float("inf"), channel="tr38901",
                         tr38901_scenario="UMi", tr38901_los="los", gnb_height_m=10.0, fading_rho_per_ms=0.5),
                E=3, R=16, steps=25, kind="pose", arena=220.0, walk=0.5, rates=(0.7,), resets={12: [1]}),
    # two cells with A3 handovers, 13 RBGs, max C/I, RLC UM drop, log-distance radio
    "mc2_ho": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="maxci", n_harq=4,
                            max_harq_tx=3, harq_fail="drop", frame_buffer=8, msg_sizes=(2500.0, 400.0), n_cells=2,
                            cell_layout="hex", cell_isd_m=100.0, noise_model="thermal", a3_ttt_ms=10.0,
                            ho_interruption_ms=5.0, li_alpha=0.5, fading_rho_per_ms=0.0,
                            cell_center_m=(60.0, 60.0)),
                   E=3, R=8, steps=30, kind="pose", arena=160.0, walk=6.0, rates=(0.5, 1.0), resets={20: [0]}),
    # envs of 200 robots (four wavefronts per env on the GPU): 52 PRB (13 RBGs), PF, poses, 8 HARQ
    "w4": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                        max_harq_tx=4, frame_buffer=8, msg_sizes=(500.0,), fading_rho_per_ms=0.0, channel="tr38901",
                        tr38901_scenario="UMi", tr38901_los="los", cell_positions_m=((100.0, 100.0),),
                        gnb_height_m=10.0),
               E=2, R=200, steps=8, kind="pose", arena=200.0, walk=1.0, rates=(0.3,), resets={5: [0]}),
    # 5G-LENA MAC switches (mac.py:26-31): PF average moved by every RBG grant, only for robots with new data
    "lena_pf": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                             pf_window=20.0, pf_update="rbg", pf_avg_idle="freeze", n_harq=8, max_harq_tx=4,
                             frame_buffer=16, msg_sizes=(600.0, 5000.0), fading_rho_per_ms=0.0, fading_rician=True,
                             rician_k_db=3.0, channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                             cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
                    E=3, R=16, steps=30, kind="pose", arena=240.0, walk=1.0, rates=(1.0, 0.3), resets={15: [2]}),
    # the same freeze on both links with the downlink on, max C/I (the frozen average is state only), SNR input
    "lena_dl": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="pf", pf_avg_idle="freeze", n_harq=4,
                             max_harq_tx=3, frame_buffer=8, msg_sizes=(2500.0,), fading_rho_per_ms=0.5, dl=True),
                    E=3, R=8, steps=25, kind="snr", snr=(-2.0, 16.0), rates=(0.9,), dl_sizes=(6000.0,),
                    dl_rates=(0.8,), resets={11: [1]}),
    # whole-band UL power (fixed PSD over the carrier, no PHR cap) with UL power control at one cell, per-subband SNR,
    # round robin, HARQ-IR
    "wb_pc": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="rr", n_harq=4, max_harq_tx=3,
                           harq_combining="ir_lena", frame_buffer=8, msg_sizes=(2000.0,), ul_power="whole_band",
                           ul_pc=True, ul_pc_p0_dbm=-95.0, ul_pc_alpha=0.8, fading_rho_per_ms=0.0),
                  E=3, R=8, steps=25, kind="snr3", snr=(0.0, 20.0), rates=(1.0,), resets={13: [0]}),
    # UL power control at one cell with poses (path loss from the UL reference SINR), PF
    "pc1": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                         max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), ul_pc=True, ul_pc_p0_dbm=-90.0,
                         ul_pc_alpha=0.7, fading_rho_per_ms=0.0, channel="tr38901", tr38901_scenario="UMi",
                         tr38901_los="los", cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
                E=3, R=12, steps=25, kind="pose", arena=200.0, walk=1.0, rates=(0.8,), resets={10: [1]}),
    # 5G-LENA UL HARQ in TDMA (mac.py:279-299): one retransmission per slot, the oldest NACK, alone in its slot; PF,
    # poses at the cell edge (many NACKs), i.i.d. fading
    "tdma": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                          max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0, 300.0), ul_retx_sched="tdma",
                          fading_rho_per_ms=0.0, channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                          cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
                 E=3, R=16, steps=30, kind="pose", arena=400.0, walk=1.0, rates=(0.8, 0.5), resets={14: [1]}),
    # 5G-LENA UL AMC on the previous PUSCH's PRBs (mac.py:393-401, 484), SNR input, round robin, chase combining
    "amc_prev": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="rr", n_harq=4, max_harq_tx=3,
                              frame_buffer=8, msg_sizes=(3000.0, 700.0), ul_amc_alloc="previous",
                              fading_rho_per_ms=0.5),
                     E=3, R=8, steps=25, kind="snr", snr=(0.0, 18.0), rates=(0.9, 0.6), resets={12: [2]}),
    # every 5G-LENA MAC switch this engine runs together (LENA_MAC_V2 without the BSR grant pipeline): per-RBG PF
    # updates frozen while idle, TDMA retransmissions, AMC on the previous PUSCH, 8 B of MAC overhead, HARQ-IR
    "lena_v2": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                             pf_window=20.0, pf_update="rbg", pf_avg_idle="freeze", ul_retx_sched="tdma",
                             ul_amc_alloc="previous", tb_overhead_bytes=8, n_harq=8, max_harq_tx=4,
                             harq_combining="ir_lena", frame_buffer=16, msg_sizes=(600.0, 5000.0),
                             fading_rho_per_ms=0.0, channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                             cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
                    E=3, R=16, steps=30, kind="pose", arena=320.0, walk=1.0, rates=(1.0, 0.3), resets={15: [0]}),
    # whole-band UL power with AMC on the previous PUSCH (the MCS over every RBG), per-subband SNR, HARQ-IR
    "wb_amc": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="rr", n_harq=4, max_harq_tx=3,
                            harq_combining="ir_lena", frame_buffer=8, msg_sizes=(2000.0,), ul_power="whole_band",
                            ul_amc_alloc="previous", ul_retx_sched="tdma", fading_rho_per_ms=0.0),
                   E=3, R=8, steps=25, kind="snr3", snr=(0.0, 20.0), rates=(1.0,), resets={13: [0]}),
    # two cells with TDMA retransmissions and AMC on the previous PUSCH, per cell (mac.py:286-297), 14 RBGs
    "mc2_lena": dict(cfg=dict(mu=1, n_prb=106, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                              n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=2,
                              cell_layout="hex", cell_isd_m=120.0, noise_model="thermal", a3_offset_db=float("inf"),
                              channel="tr38901", tr38901_scenario="UMi", tr38901_los="los", gnb_height_m=10.0,
                              fading_rho_per_ms=0.0, ul_retx_sched="tdma", ul_amc_alloc="previous"),
                     E=3, R=16, steps=25, kind="pose", arena=260.0, walk=0.5, rates=(0.8,), resets={12: [1]}),
    # frequency-correlated fading (nr_engine.py:43-48, 320-368): the innovations and the initial state correlated
    # across the 13 RBGs by a fixed 300 ns delay spread; PF, poses, correlated fading in time
    "fcorr": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                           max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0, 300.0), fading_freq_corr=True,
                           fading_delay_spread_ns=300.0, fading_rho_per_ms=0.5, channel="tr38901",
                           tr38901_scenario="UMi", tr38901_los="los", cell_positions_m=((100.0, 100.0),),
                           gnb_height_m=10.0),
                  E=3, R=16, steps=30, kind="pose", arena=240.0, walk=1.0, rates=(0.8, 0.5), resets={14: [1]}),
    # the same on both links (SNR input, i.i.d. in time, 60 ns: strongly correlated subbands), HARQ-IR
    "fcorr_dl": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="maxci", n_harq=4, max_harq_tx=3,
                              harq_combining="ir_lena", frame_buffer=8, msg_sizes=(2500.0,), fading_freq_corr=True,
                              fading_delay_spread_ns=60.0, fading_rho_per_ms=0.0, dl=True),
                     E=3, R=8, steps=25, kind="snr", snr=(-2.0, 16.0), rates=(0.9,), dl_sizes=(6000.0,),
                     dl_rates=(0.8,), resets={11: [1]}),
    # two cells, every robot-cell link correlated across 14 RBGs (1 us delay spread)
    "fcorr_mc2": dict(cfg=dict(mu=1, n_prb=106, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                               max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=2, cell_layout="hex",
                               cell_isd_m=120.0, noise_model="thermal", a3_offset_db=float("inf"), channel="tr38901",
                               tr38901_scenario="UMi", tr38901_los="los", gnb_height_m=10.0, fading_rho_per_ms=0.5,
                               fading_freq_corr=True, fading_delay_spread_ns=1000.0),
                      E=3, R=16, steps=25, kind="pose", arena=220.0, walk=0.5, rates=(0.7,), resets={12: [1]}),
    # envs of 100 robots on two wavefronts, 273 PRB in 8 RBGs of 35, 100 ns
    "fcorr_w2": dict(cfg=dict(mu=1, n_prb=273, rbg_size=35, tdd_pattern="DDDSU", control_step_ms=10.0,
                              scheduler="pf", n_harq=8, max_harq_tx=4, frame_buffer=8, msg_sizes=(800.0,),
                              fading_freq_corr=True, fading_delay_spread_ns=100.0, fading_rho_per_ms=0.0,
                              channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                              cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
                     E=2, R=100, steps=12, kind="pose", arena=200.0, walk=1.0, rates=(0.3,), resets={7: [0]}),
    # Rician fading with K from the LOS state (rician_k_db None: a log-normal K per link, TR 38.901 Table 7.5-6, that
    # applies once the radio reports the link LOS, nr_engine.py:282-419): UMi LOS, PF, correlated fading, a reset
    "rice_los": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                              max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0, 300.0), fading_rician=True,
                              fading_rho_per_ms=0.5, channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                              cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0),
                     E=3, R=16, steps=30, kind="pose", arena=240.0, walk=1.0, rates=(0.8, 0.5), resets={14: [1]}),
    # the same with the downlink, UMa
    "rice_los_dl": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                 n_harq=8, max_harq_tx=4, frame_buffer=8, msg_sizes=(2000.0,), fading_rician=True,
                                 fading_rho_per_ms=0.0, channel="tr38901", tr38901_scenario="UMa", tr38901_los="los",
                                 cell_positions_m=((100.0, 100.0),), gnb_height_m=25.0, dl=True),
                        E=3, R=8, steps=25, kind="pose", arena=260.0, walk=1.0, rates=(0.8,), dl_sizes=(4000.0,),
                        dl_rates=(0.6,), resets={11: [2]}),
    # SNR input: the radio reports no LOS state, so K stays 0 (Rayleigh) however long the run
    "rice_snr": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="maxci", n_harq=4, max_harq_tx=3,
                              frame_buffer=8, msg_sizes=(2500.0,), fading_rician=True, fading_rho_per_ms=0.5),
                     E=3, R=8, steps=20, kind="snr", snr=(-2.0, 16.0), rates=(0.9,), resets={9: [0]}),
    # the TR 38.901 stochastic LOS state (the reference's default): LOS where the LOS-state field's uniform is below
    # Pr_LOS(d_2D) (models.py:121-167): UMi at distances where both states occur, fast motion, a reset
    "los_sto": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                             max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0, 300.0), fading_rho_per_ms=0.5,
                             channel="tr38901", tr38901_scenario="UMi", tr38901_los="stochastic",
                             cell_positions_m=((150.0, 150.0),), gnb_height_m=10.0),
                    E=3, R=16, steps=30, kind="pose", arena=300.0, walk=4.0, rates=(0.8, 0.5), resets={14: [1]}),
    # three cells on UMa with the stochastic LOS state of every robot-cell link, interference
    "los_sto_mc": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                                max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=3, cell_layout="hex",
                                cell_isd_m=200.0, noise_model="thermal", a3_offset_db=float("inf"), channel="tr38901",
                                tr38901_scenario="UMa", tr38901_los="stochastic", gnb_height_m=25.0,
                                fading_rho_per_ms=0.5),
                       E=2, R=16, steps=25, kind="pose", arena=300.0, walk=3.0, rates=(0.7,), resets={12: [1]}),
    # indoor hotspot with the downlink
    "los_sto_dl": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                n_harq=4, max_harq_tx=3, frame_buffer=8, msg_sizes=(2000.0,), fading_rho_per_ms=0.0,
                                channel="tr38901", tr38901_scenario="InH", tr38901_los="stochastic",
                                cell_positions_m=((30.0, 30.0),), gnb_height_m=3.0, dl=True),
                       E=3, R=8, steps=25, kind="pose", arena=60.0, walk=1.0, rates=(0.8,), dl_sizes=(4000.0,),
                       dl_rates=(0.6,), resets={11: [2]}),
    # Rician K from the stochastic LOS state (the reference's defaults: fading_rician, K from LOS, a 4-slot ramp):
    # links flip between LOS and NLOS as the robots move, and K ramps to each new target (nr_engine.py:370-419)
    "rice_sto": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                              max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0, 300.0), fading_rician=True,
                              fading_rho_per_ms=0.5, channel="tr38901", tr38901_scenario="UMi",
                              tr38901_los="stochastic", cell_positions_m=((150.0, 150.0),), gnb_height_m=10.0),
                     E=3, R=16, steps=30, kind="pose", arena=300.0, walk=4.0, rates=(0.8, 0.5), resets={14: [1]}),
    # the same on InH with the downlink and no ramp (a new target applies at once)
    "rice_sto_dl": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                 n_harq=4, max_harq_tx=3, frame_buffer=8, msg_sizes=(2000.0,), fading_rician=True,
                                 fading_rho_per_ms=0.5, rician_k_ramp_slots=0, channel="tr38901",
                                 tr38901_scenario="InH", tr38901_los="stochastic", cell_positions_m=((30.0, 30.0),),
                                 gnb_height_m=3.0, dl=True),
                        E=3, R=8, steps=25, kind="pose", arena=60.0, walk=2.0, rates=(0.8,), dl_sizes=(4000.0,),
                        dl_rates=(0.6,), resets={11: [2]}),
    # UMa with a ramp longer than two control steps (50 slots against 20 per step): ramps carry over steps, restart
    # from a K on the way, and a checkpoint is taken mid-ramp
    "rice_sto_slow": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                   n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), fading_rician=True,
                                   fading_rho_per_ms=0.0, rician_k_ramp_slots=50, channel="tr38901",
                                   tr38901_scenario="UMa", tr38901_los="stochastic",
                                   cell_positions_m=((150.0, 150.0),), gnb_height_m=25.0),
                          E=3, R=16, steps=30, kind="pose", arena=300.0, walk=5.0, rates=(0.8,), resets={17: [0]}),
    # Rician fading on every robot-cell link (nr_engine.py:282-319, 602-611, 740-752): two cells with a fixed K of
    # 6 dB, UMi LOS; three cells with K from the stochastic LOS state of each link (4-slot ramp), UMa
    "mc2_rice": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                              max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=2, cell_layout="hex",
                              cell_isd_m=150.0, noise_model="thermal", channel="tr38901", tr38901_scenario="UMi",
                              tr38901_los="los", gnb_height_m=10.0, fading_rho_per_ms=0.5, fading_rician=True,
                              rician_k_db=6.0),
                     E=2, R=16, steps=25, kind="pose", arena=250.0, walk=3.0, rates=(0.7,), resets={12: [1]}),
    "mc3_rice_sto": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                  n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=3,
                                  cell_layout="hex", cell_isd_m=200.0, noise_model="thermal", channel="tr38901",
                                  tr38901_scenario="UMa", tr38901_los="stochastic", gnb_height_m=25.0,
                                  fading_rho_per_ms=0.5, fading_rician=True, rician_k_ramp_slots=30),
                         E=2, R=16, steps=25, kind="pose", arena=300.0, walk=5.0, rates=(0.7,), resets={12: [1]}),
    # frequency-correlated fading with per-link delay spreads (fading_delay_spread_ns None, the reference's default
    # with fading_freq_corr): a TR 38.901 lgDS draw per link and LOS state on the log grid of fading_ds_grid, the LOS
    # or NLOS one by the radio's state (nr_engine.py:320-381): UMi with the stochastic LOS state and fast motion
    "fcorr_los": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                               max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0, 300.0), fading_rho_per_ms=0.5,
                               fading_freq_corr=True, channel="tr38901", tr38901_scenario="UMi",
                               tr38901_los="stochastic", cell_positions_m=((150.0, 150.0),), gnb_height_m=10.0),
                      E=3, R=16, steps=30, kind="pose", arena=300.0, walk=4.0, rates=(0.8, 0.5), resets={14: [1]}),
    # InH in a fixed LOS state with the downlink, 106 PRB (14 RBGs), a grid of 8 points
    "fcorr_los_dl": dict(cfg=dict(mu=1, n_prb=106, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                  n_harq=4, max_harq_tx=3, frame_buffer=8, msg_sizes=(2000.0,), fading_rho_per_ms=0.5,
                                  fading_freq_corr=True, fading_ds_grid=(5.0, 500.0, 8), channel="tr38901",
                                  tr38901_scenario="InH", tr38901_los="los", cell_positions_m=((30.0, 30.0),),
                                  gnb_height_m=3.0, dl=True),
                         E=3, R=8, steps=25, kind="pose", arena=60.0, walk=2.0, rates=(0.8,), dl_sizes=(4000.0,),
                         dl_rates=(0.6,), resets={11: [2]}),
    # UMa with Rician K and the delay spread both from the stochastic LOS state, 273 PRB (18 RBGs)
    "fcorr_los_rice": dict(cfg=dict(mu=1, n_prb=273, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                    n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(3000.0,),
                                    fading_rho_per_ms=0.3, fading_freq_corr=True, fading_rician=True,
                                    channel="tr38901", tr38901_scenario="UMa", tr38901_los="stochastic",
                                    cell_positions_m=((150.0, 150.0),), gnb_height_m=25.0),
                           E=3, R=16, steps=25, kind="pose", arena=300.0, walk=5.0, rates=(0.8,), resets={12: [0]}),
    # several cells with A3 handovers under ho_rlc="flush" (every queued frame of a robot dropped at its switch,
    # mac.py:557-581): fast motion, round robin, an N+I EWMA, a reset
    "mc3_flush": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="rr", n_harq=4,
                               max_harq_tx=3, frame_buffer=8, msg_sizes=(2500.0, 400.0),
                               n_cells=3, cell_layout="hex", cell_isd_m=120.0, cell_center_m=(60.0, 60.0),
                               noise_model="thermal", a3_ttt_ms=10.0, ho_interruption_ms=2.5, ho_rlc="flush",
                               li_alpha=0.3, fading_rho_per_ms=0.5),
                      E=3, R=16, steps=30, kind="pose", arena=200.0, walk=8.0, rates=(0.5, 1.0), resets={12: [1]}),
    # the A3 target admission floor (a3_min_target_rsrp_dbm, radio.py:311-361: a neighbour whose RSRP is below it
    # never satisfies A3): three cells far apart, fast motion, so that some targets at the cell edge are refused
    "mc3_a3floor": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="maxci",
                                 n_harq=4, max_harq_tx=3, harq_fail="drop", frame_buffer=8,
                                 msg_sizes=(2500.0, 400.0), n_cells=3, cell_layout="hex", cell_isd_m=200.0,
                                 noise_model="thermal", a3_ttt_ms=20.0, ho_interruption_ms=5.0, li_alpha=0.5,
                                 fading_rho_per_ms=0.0, cell_center_m=(100.0, 100.0), channel="tr38901",
                                 tr38901_scenario="UMi", tr38901_los="los", gnb_height_m=10.0,
                                 a3_min_target_rsrp_dbm=-68.0),
                        E=3, R=16, steps=40, kind="pose", arena=300.0, walk=6.0, rates=(0.5, 1.0), resets={25: [0]}),
    # two cells with per-link delay spreads (fading_delay_spread_ns None): each robot-cell link's own lgDS draws, the
    # LOS or NLOS grid index by that link's stochastic LOS state (nr_engine.py:320-381), UMi, 13 RBGs
    # the wideband rate in the PF metric (mac.py:259-264): pf_metric="wideband" on per-subband SNR (RBGs of different
    # SINR, so the wideband MCS differs from the per-RBG ones), the per-RBG PF update, 16 robots
    "wb_pf": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="pf", pf_metric="wideband",
                           pf_update="rbg", n_harq=4, max_harq_tx=3, frame_buffer=8, msg_sizes=(2500.0, 400.0),
                           fading_rho_per_ms=0.7),
                  E=3, R=16, steps=30, kind="snr3", snr=(-4.0, 18.0), rates=(0.8, 0.6), resets={15: [2]}),
    # scheduler="pf_wideband" with the downlink, poses on UMi LOS, Rician K
    "pfwb_dl": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf_wideband",
                             n_harq=4, max_harq_tx=3, frame_buffer=8, msg_sizes=(2000.0,), fading_rician=True,
                             rician_k_db=3.0, channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                             cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0, dl=True),
                    E=3, R=8, steps=25, kind="pose", arena=200.0, walk=1.0, rates=(0.8,), dl_sizes=(4000.0,),
                    dl_rates=(0.6,), resets={11: [2]}),
    # the wideband rate under max C/I with the mean-dB effective SINR, log-distance radio
    "wb_maxci_md": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="maxci", pf_metric="wideband",
                                 eff_sinr="mean_db", n_harq=4, max_harq_tx=4, frame_buffer=10, msg_sizes=(1500.0,),
                                 cell_positions_m=((60.0, 60.0),), fading_rho_per_ms=0.5),
                        E=3, R=8, steps=25, kind="pose", arena=150.0, walk=1.0, rates=(1.0,), resets={12: [0]}),
    # two cells, pf_wideband: one wideband PF scheduler per cell
    "mc2_wb": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf_wideband",
                            n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=2,
                            cell_layout="hex", cell_isd_m=150.0, noise_model="thermal", fading_rho_per_ms=0.5),
                   E=2, R=16, steps=25, kind="pose", arena=300.0, walk=1.0, rates=(0.7,), resets={12: [1]}),
    # several cells with the path gain given (step(pathgain_db=[E,R,C]), engine.py:909-915): three cells, A3
    # handovers as the per-link gains drift, Rician K fixed, interference and power control
    "mc3_pg": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                            max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=3, cell_layout="hex",
                            cell_isd_m=200.0, noise_model="thermal", a3_offset_db=1.0, a3_ttt_ms=2.0,
                            fading_rician=True, rician_k_db=6.0, rician_k_from_los=False, fading_rho_per_ms=0.5),
                   E=3, R=16, steps=25, kind="pg", pg=(-125.0, -75.0), pg_walk=2.5, rates=(0.7,), resets={12: [1]}),
    # radio link failure (nr_engine.py:691-707, 733-736, 778-787; radio.py:456-531) on the path gain input: the
    # serving SINR crosses Qout / Qin as the per-link gains drift, T310 of 30 ms, re-establishment after 20 ms at the
    # strongest suitable cell, T311 of 60 ms to idle; A3 handovers that stop T310
    "mc3_rlf": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                             max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=3, cell_layout="hex",
                             cell_isd_m=200.0, noise_model="thermal", a3_offset_db=2.0, a3_ttt_ms=5.0,
                             fading_rho_per_ms=0.5, rlf=True, n310=1, n311=2, t310_ms=30.0, t311_ms=60.0,
                             reest_delay_ms=20.0),
                    E=3, R=16, steps=30, kind="pg", pg=(-150.0, -100.0), pg_walk=5.0, rates=(0.7,),
                    resets={15: [1]}),
    # radio link failure with poses, the RLC flushed at RLF, the A3 floor (also the cell search's), no handovers
    "mc2_rlf_flush": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                   n_harq=4, max_harq_tx=3, frame_buffer=10, msg_sizes=(1500.0,), n_cells=2,
                                   cell_layout="hex", cell_isd_m=500.0, noise_model="thermal",
                                   a3_offset_db=float("inf"), a3_min_target_rsrp_dbm=-112.0, channel="tr38901",
                                   tr38901_scenario="UMa", tr38901_los="nlos", gnb_height_m=25.0, rlf=True,
                                   rlf_rlc="flush", n310=2, n311=1, t310_ms=20.0, t311_ms=50.0, reest_delay_ms=10.0,
                                   fading_rho_per_ms=0.5),
                          E=3, R=16, steps=30, kind="pose", arena=900.0, walk=25.0, rates=(0.8,), resets={14: [2]}),
    # four to seven cells (radio.py gnb_xy: the hex centre site and the first ring, up to the full 7-site cluster):
    # mc4: 4 cells, 106 PRB (14 RBGs), PF, Rician TR 38.901 UMi LOS links, same-slot UL interference;
    # mc5: 5 cells, 273 PRB in 8 RBGs of 35, maxCI, A3 handovers, RLC UM drop; mc6: 6 cells, 52 PRB, round robin,
    # radio link failure on path gains; mc7: the full cluster, 52 PRB, PF, A3 handovers with fast motion
    "mc4": dict(cfg=dict(mu=1, n_prb=106, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                         max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=4,
                         cell_layout="hex", cell_isd_m=150.0, cell_center_m=(120.0, 120.0), noise_model="thermal",
                         channel="tr38901", tr38901_scenario="UMi", tr38901_los="los", gnb_height_m=10.0,
                         fading_rho_per_ms=0.5, fading_rician=True, rician_k_db=3.0),
                E=2, R=16, steps=18, kind="pose", arena=240.0, walk=3.0, rates=(0.7,), resets={11: [1]}),
    "mc5": dict(cfg=dict(mu=1, n_prb=273, rbg_size=35, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="maxci",
                         n_harq=4, max_harq_tx=3, harq_fail="drop", frame_buffer=8, msg_sizes=(2500.0, 400.0),
                         n_cells=5, cell_layout="hex", cell_isd_m=120.0, cell_center_m=(120.0, 120.0),
                         noise_model="thermal", a3_ttt_ms=20.0, ho_interruption_ms=5.0, li_alpha=0.5,
                         fading_rho_per_ms=0.0),
                E=3, R=8, steps=30, kind="pose", arena=240.0, walk=6.0, rates=(0.5, 1.0), resets={20: [0]}),
    "mc6": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="rr", n_harq=8,
                         max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=6, cell_layout="hex",
                         cell_isd_m=200.0, noise_model="thermal", a3_offset_db=2.0, a3_ttt_ms=5.0,
                         fading_rho_per_ms=0.5, rlf=True, n310=1, n311=2, t310_ms=30.0, t311_ms=60.0,
                         reest_delay_ms=20.0),
                E=2, R=16, steps=24, kind="pg", pg=(-172.0, -118.0), pg_walk=6.0, rates=(0.7,), resets={12: [1]}),
    "mc7": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                         max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=7, cell_layout="hex",
                         cell_isd_m=120.0, cell_center_m=(150.0, 150.0), noise_model="thermal", a3_ttt_ms=10.0,
                         ho_interruption_ms=5.0, fading_rho_per_ms=0.5, channel="tr38901", tr38901_scenario="UMi",
                         tr38901_los="los", gnb_height_m=10.0),
                E=2, R=16, steps=30, kind="pose", arena=300.0, walk=8.0, rates=(0.6,), resets={18: [0]}),
    # per-robot Doppler (fading_doppler="per_robot": engine.py:862-864, radio.py:285-300, channels/doppler.py:23-29,
    # nr_engine.py:583-589): speeds from consecutive poses, 0 .. 25 m/s (J0 reaches its first zero near 13 m/s at
    # 3.5 GHz, rho 0 from there), a 0.5 m/s floor
    "dop": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                         max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0, 300.0), fading_doppler="per_robot",
                         doppler_min_speed_mps=0.5, cell_positions_m=((100.0, 100.0),)),
                E=3, R=16, steps=30, kind="pose", arena=200.0, walk_max=0.25, rates=(0.8, 0.5), resets={14: [1]}),
    # the velocity input (vel=, |v| of normal components with sigma 8 m/s) with the downlink and Rician K on UMi LOS
    "dop_vel_dl": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=4,
                                max_harq_tx=3, frame_buffer=8, msg_sizes=(2000.0,), fading_doppler="per_robot",
                                fading_rician=True, rician_k_db=3.0, channel="tr38901", tr38901_scenario="UMi",
                                tr38901_los="los", cell_positions_m=((100.0, 100.0),), gnb_height_m=10.0, dl=True),
                       E=3, R=8, steps=25, kind="pose", arena=200.0, walk=1.0, vel=8.0, rates=(0.8,),
                       dl_sizes=(4000.0,), dl_rates=(0.6,), resets={11: [2]}),
    # two cells, every robot-cell link with the robot's correlation, a 1 m/s floor
    "mc2_dop": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                             max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=2, cell_layout="hex",
                             cell_isd_m=150.0, noise_model="thermal", fading_doppler="per_robot",
                             doppler_min_speed_mps=1.0),
                    E=2, R=16, steps=25, kind="pose", arena=300.0, walk_max=0.3, rates=(0.7,), resets={12: [1]}),
    "mc2_fcorr_los": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                   n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=2,
                                   cell_layout="hex", cell_isd_m=150.0, noise_model="thermal",
                                   a3_offset_db=float("inf"), channel="tr38901", tr38901_scenario="UMi",
                                   tr38901_los="stochastic", gnb_height_m=10.0, fading_rho_per_ms=0.5,
                                   fading_freq_corr=True),
                          E=2, R=16, steps=25, kind="pose", arena=250.0, walk=4.0, rates=(0.7,), resets={12: [1]}),
    # three cells at 64 robots per env (one env per wavefront on the GPU: the cooperative interference list) with
    # Rician fading on every link, K from each link's stochastic LOS state with a 6-slot ramp, UMa, 14 RBGs
    "mc3_rice64": dict(cfg=dict(mu=1, n_prb=106, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(1200.0,), n_cells=3,
                                cell_layout="hex", cell_isd_m=200.0, noise_model="thermal",
                                a3_offset_db=float("inf"), channel="tr38901", tr38901_scenario="UMa",
                                tr38901_los="stochastic", gnb_height_m=25.0, fading_rho_per_ms=0.5,
                                fading_rician=True, rician_k_ramp_slots=6),
                       E=2, R=64, steps=14, kind="pose", arena=300.0, walk=5.0, rates=(0.4,), resets={8: [1]}),
    # the same three cells at 48 robots per env with a fixed K of 6 dB and the A3 handover on (UMi LOS)
    "mc3_rice48": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=3,
                                cell_layout="hex", cell_isd_m=150.0, noise_model="thermal", a3_ttt_ms=10.0,
                                ho_interruption_ms=2.5, channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                                gnb_height_m=10.0, fading_rho_per_ms=0.0, fading_rician=True, rician_k_db=6.0),
                       E=2, R=48, steps=16, kind="pose", arena=260.0, walk=6.0, rates=(0.5,), resets={9: [0]}),
    # the same without Rician fading (A3 handovers and i.i.d. fading on 48-robot envs), with correlated fading in time,
    # and on 32-robot envs (two envs per wavefront)
    "mc3_ho48": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                              n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=3,
                              cell_layout="hex", cell_isd_m=150.0, noise_model="thermal", a3_ttt_ms=10.0,
                              ho_interruption_ms=2.5, channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                              gnb_height_m=10.0, fading_rho_per_ms=0.0),
                     E=2, R=48, steps=16, kind="pose", arena=260.0, walk=6.0, rates=(0.5,), resets={9: [0]}),
    "mc3_rice48c": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                 n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=3,
                                 cell_layout="hex", cell_isd_m=150.0, noise_model="thermal", a3_ttt_ms=10.0,
                                 ho_interruption_ms=2.5, channel="tr38901", tr38901_scenario="UMi",
                                 tr38901_los="los", gnb_height_m=10.0, fading_rho_per_ms=0.5, fading_rician=True,
                                 rician_k_db=6.0),
                        E=2, R=48, steps=16, kind="pose", arena=260.0, walk=6.0, rates=(0.5,), resets={9: [0]}),
    "mc3_rice32": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                                n_harq=8, max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0,), n_cells=3,
                                cell_layout="hex", cell_isd_m=150.0, noise_model="thermal", a3_ttt_ms=10.0,
                                ho_interruption_ms=2.5, channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                                gnb_height_m=10.0, fading_rho_per_ms=0.0, fading_rician=True, rician_k_db=6.0),
                       E=2, R=32, steps=16, kind="pose", arena=260.0, walk=6.0, rates=(0.5,), resets={9: [0]}),
    # one cell at 64 robots per env (one env per wavefront) with the per-link features of TR 38.901: the stochastic
    # LOS state, Rician K from it with the default ramp, per-link delay spreads, UMi, 13 RBGs
    "sto64": dict(cfg=dict(mu=1, n_prb=52, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf", n_harq=8,
                           max_harq_tx=4, frame_buffer=12, msg_sizes=(1500.0, 300.0), fading_rho_per_ms=0.5,
                           fading_rician=True, fading_freq_corr=True, channel="tr38901", tr38901_scenario="UMi",
                           tr38901_los="stochastic", cell_positions_m=((150.0, 150.0),), gnb_height_m=10.0),
                  E=2, R=64, steps=16, kind="pose", arena=300.0, walk=4.0, rates=(0.5, 0.3), resets={9: [1]}),
    # the same on envs of 100 robots (two wavefronts per env), UMa, 8 RBGs of 35 PRB, a 10-slot ramp
    "sto100": dict(cfg=dict(mu=1, n_prb=273, rbg_size=35, tdd_pattern="DDDSU", control_step_ms=10.0, scheduler="pf",
                            n_harq=8, max_harq_tx=4, frame_buffer=8, msg_sizes=(900.0,), fading_rho_per_ms=0.3,
                            fading_rician=True, rician_k_ramp_slots=10, fading_freq_corr=True, channel="tr38901",
                            tr38901_scenario="UMa", tr38901_los="stochastic", cell_positions_m=((150.0, 150.0),),
                            gnb_height_m=25.0),
                   E=2, R=100, steps=10, kind="pose", arena=300.0, walk=5.0, rates=(0.3,), resets={6: [0]}),
}


# Statistics cases (NREngine.log_stats / collect / queued, isaac_net/core/nr_engine.py:440-446, 885-914): the
# engine runs with log_stats on from construction; every step's queued() and refused_env and the final collect()
# are recorded. "log_cap_max": set on the reference's NRNet (frames captured later are not logged).
STATS_CASES = {
    # UL: HARQ drop (dropped frames), purge timeouts (timed out, late), a small FIFO (overflow), two classes, poses
    # (frame SNR = the previous step's SNR), partial resets
    "stats_ul": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="pf", n_harq=4, max_harq_tx=2,
                              harq_fail="drop", frame_buffer=6, msg_sizes=(3000.0, 600.0), timeout_steps=4,
                              fading_rho_per_ms=0.0, channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                              cell_positions_m=((60.0, 60.0),), gnb_height_m=10.0),
                     E=4, R=12, steps=30, kind="pose", arena=260.0, walk=2.0, rates=(1.2, 0.8),
                     resets={14: [1, 3]}),
    # UL + DL: PDCP discard on arrival (discarded), small FIFOs (UL and DL overflow), SNR input, RLC UM drop, DL delays,
    # a log cap
    "stats_dl": dict(cfg=dict(mu=1, n_prb=52, control_step_ms=10.0, scheduler="rr", n_harq=4, max_harq_tx=2,
                              harq_fail="drop", frame_buffer=5, msg_sizes=(2500.0,), timeout_steps=5,
                              discard="pdcp_arrival", dl=True),
                     E=3, R=8, steps=30, kind="snr", snr=(-6.0, 12.0), rates=(1.4,), dl_sizes=(4000.0,),
                     dl_rates=(1.1,), resets={10: [0]}, log_cap_max=20),
}


# Level WIFI cases (make_engine("WIFI", ...)): NRConfig fields, WifiConfig fields, sizes, inputs and resets.
WIFI_CASES = {
    # defaults (802.11ax 20 MHz, BE, A-MPDU, Poisson accesses), SNR input over the whole MCS range and below MCS 0
    "w_snr": dict(cfg=dict(control_step_ms=10.0, frame_buffer=8, msg_sizes=(1500.0,), timeout_steps=5),
                  wifi=dict(), E=3, R=8, steps=30, kind="snr", snr=(-2.0, 42.0), rates=(2.5,), resets={12: [1]}),
    # renewal ("mean") accesses, RTS/CTS, ACK collision time, no aggregation, VI (TXOP limit), residual FER, few
    # attempts, VHT 40 MHz, two classes, short FIFO and timeout
    "w_mean": dict(cfg=dict(control_step_ms=5.0, frame_buffer=6, msg_sizes=(200.0, 3000.0), timeout_steps=3),
                   wifi=dict(access_noise="mean", rts_cts=True, collision_time="ack", max_ampdu_bytes=0,
                             access_category="VI", frame_error_rate=0.1, max_tx=3, standard="ac", bandwidth_mhz=40),
                   E=3, R=8, steps=30, kind="snr", snr=(4.0, 40.0), rates=(2.0, 0.8), resets={9: [0, 2]}),
    # poses through the log-distance radio of one AP, non-HT 802.11a, rate margin, background stations, undamped
    # solve with 3 iterations, 16 robots
    "w_logd": dict(cfg=dict(control_step_ms=10.0, frame_buffer=12, msg_sizes=(1500.0,), timeout_steps=6,
                            cell_positions_m=((40.0, 40.0),)),
                   wifi=dict(standard="a", ra_margin_db=2.0, bg_stations=2, fp_iters=3, fp_damping=1.0, max_tx=4),
                   E=2, R=16, steps=25, kind="pose", arena=80.0, walk=1.0, rates=(1.0,), resets={10: [1]}),
    # poses through TR 38.901 UMi LOS, one AC per message class (VO / VI: same AIFSN), HE 80 MHz 2 streams, 2 ms
    # sub-steps
    "w_tr": dict(cfg=dict(control_step_ms=8.0, frame_buffer=10, msg_sizes=(400.0, 2500.0), timeout_steps=4,
                          channel="tr38901", tr38901_scenario="UMi", tr38901_los="los",
                          cell_positions_m=((75.0, 75.0),)),
                 wifi=dict(class_ac=("VO", "VI"), bandwidth_mhz=80, n_ss=2, gi_us=1.6, substep_ms=2.0,
                           ap_height_m=6.0),
                 E=3, R=8, steps=25, kind="pose", arena=150.0, walk=2.0, rates=(1.5, 0.5), resets={15: [2]}),
    # poses through TR 38.901 UMi with the stochastic LOS state (the reference's default), the AP in the middle of a
    # 300 m arena so that links cross the LOS / NLOS boundary as the robots move
    "w_sto": dict(cfg=dict(control_step_ms=10.0, frame_buffer=10, msg_sizes=(600.0, 1500.0), timeout_steps=5,
                           channel="tr38901", tr38901_scenario="UMi", tr38901_los="stochastic",
                           cell_positions_m=((150.0, 150.0),)),
                  wifi=dict(ap_height_m=6.0),
                  E=3, R=16, steps=30, kind="pose", arena=300.0, walk=4.0, rates=(1.5, 0.5), resets={14: [0]}),
    # three APs on one channel (one collision domain, the reference's default n_channels=1): max-RSSI association,
    # roaming with a 3 dB hysteresis and a 2-sub-step interruption, one background station per AP, robots crossing a
    # 240 m arena
    "w_multi": dict(cfg=dict(control_step_ms=10.0, frame_buffer=10, msg_sizes=(800.0, 2000.0), timeout_steps=5),
                    wifi=dict(ap_positions_m=((40.0, 40.0), (200.0, 60.0), (120.0, 200.0)), roam_hyst_db=3.0,
                              roam_ms=2.0, bg_stations=1),
                    E=3, R=16, steps=30, kind="pose", arena=240.0, walk=6.0, rates=(1.0, 0.4), resets={14: [1]}),
    # APs on two channels (two collision domains): APs 0 and 2 share channel 1, AP 1 is on channel 6; robots roam
    # between the domains
    "w_chan": dict(cfg=dict(control_step_ms=10.0, frame_buffer=10, msg_sizes=(800.0, 2000.0), timeout_steps=5),
                   wifi=dict(ap_positions_m=((40.0, 40.0), (200.0, 60.0), (120.0, 200.0)), ap_channels=(1, 6, 1),
                             roam_hyst_db=3.0, roam_ms=2.0, bg_stations=2),
                   E=3, R=16, steps=30, kind="pose", arena=240.0, walk=6.0, rates=(1.2, 0.4), resets={17: [2]}),
    # four APs spread round robin over three channels (n_channels), the log-distance radio
    "w_chan3": dict(cfg=dict(control_step_ms=10.0, frame_buffer=8, msg_sizes=(1200.0,), timeout_steps=4,
                             channel="log_distance"),
                    wifi=dict(ap_positions_m=((0.0, 0.0), (120.0, 0.0), (0.0, 120.0), (120.0, 120.0)), n_channels=3,
                              roam_hyst_db=2.0, bg_stations=1),
                    E=2, R=12, steps=25, kind="pose", arena=130.0, walk=8.0, rates=(1.5,), resets={}),
    # AIFS zones: the robots in AC_VI (AIFSN 2) beside background stations in AC_BE (AIFSN 3): two zones
    "w_aifs": dict(cfg=dict(control_step_ms=10.0, frame_buffer=8, msg_sizes=(1000.0,), timeout_steps=4),
                   wifi=dict(access_category="VI", bg_stations=3, bg_ac="BE"),
                   E=3, R=12, steps=25, kind="disc", radius=40.0, walk=1.0, rates=(1.6,), resets={11: [0]}),
    # six AIFS zones (per-class ACs VO and BK, background stations in BE) on two APs on two channels
    "w_aifs_cls": dict(cfg=dict(control_step_ms=10.0, frame_buffer=10, msg_sizes=(600.0, 3000.0), timeout_steps=5),
                       wifi=dict(class_ac=("VO", "BK"), bg_stations=2, bg_ac="BE",
                                 ap_positions_m=((30.0, 30.0), (150.0, 60.0)), ap_channels=(1, 6), roam_hyst_db=2.0),
                       E=2, R=14, steps=25, kind="pose", arena=180.0, walk=7.0, rates=(0.9, 0.5), resets={13: [1]}),
    # hidden nodes: robots in a 110 m disc around one AP, out of each other's carrier sense beyond ~120 m
    "w_hidden": dict(cfg=dict(control_step_ms=10.0, frame_buffer=8, msg_sizes=(1500.0,), timeout_steps=4,
                              cell_positions_m=((0.0, 0.0),)),
                     wifi=dict(hidden_nodes=True),
                     E=3, R=12, steps=25, kind="disc", radius=110.0, walk=3.0, rates=(1.5,), resets={12: [2]}),
    # hidden nodes with RTS/CTS on two APs on two channels, background stations
    "w_hidden_rts": dict(cfg=dict(control_step_ms=10.0, frame_buffer=8, msg_sizes=(800.0, 2400.0), timeout_steps=5),
                         wifi=dict(hidden_nodes=True, rts_cts=True, ap_positions_m=((0.0, 0.0), (90.0, 0.0)),
                                   ap_channels=(1, 6), bg_stations=1, roam_hyst_db=2.0),
                         E=2, R=12, steps=25, kind="pose", arena=160.0, walk=6.0, rates=(0.8, 0.5), resets={}),
    # the DCF workload: legacy DCF parameters (CWmin 15, CWmax 1023), 16 stations uniform in a 50 m disc around the
    # AP, 1500 B messages, 20 sub-steps per control step
    "w_dcf": dict(cfg=dict(control_step_ms=20.0, frame_buffer=16, msg_sizes=(1500.0,),
                           cell_positions_m=((0.0, 0.0),)),
                  wifi=dict(access_category="DCF"),
                  E=4, R=16, steps=20, kind="disc", radius=50.0, walk=0.5, rates=(2.0,), resets={8: [3]}),
}


def _inputs(name, c):
    """Per-step inputs of a case: poses or SNR, and per-class arrival counts (numpy, seeded by the case name)."""
    rs = np.random.default_rng(int.from_bytes(hashlib.sha256(name.encode()).digest()[:4], "little"))
    E, R, T = c["E"], c["R"], c["steps"]
    n_cls = len(c["rates"])
    counts = np.stack([rs.poisson(lam, size=(T, E, R)) for lam in c["rates"]], -1).astype(np.int64)
    if c["kind"] == "disc":
        rad, ang0 = c["radius"] * np.sqrt(rs.uniform(size=(E, R))), rs.uniform(0.0, 2 * math.pi, size=(E, R))
        p = np.stack([rad * np.cos(ang0), rad * np.sin(ang0)], -1)
        xs = []
        for _ in range(T):
            xs.append(p.copy())
            ang = rs.uniform(0.0, 2 * math.pi, size=(E, R))
            p = p + c["walk"] * np.stack([np.cos(ang), np.sin(ang)], -1)
        x = np.stack(xs).astype(np.float32)
    elif c["kind"] == "pose":
        a = c["arena"]
        p = rs.uniform(0.0, a, size=(E, R, 2))
        xs = []
        for _ in range(T):
            xs.append(p.copy())
            ang = rs.uniform(0.0, 2 * math.pi, size=(E, R))
            # walk_max: a step length per robot and step, uniform in [0, walk_max] (robots of different speeds)
            w = c["walk"] if "walk_max" not in c else rs.uniform(0.0, c["walk_max"], size=(E, R))[..., None]
            p = np.clip(p + w * np.stack([np.cos(ang), np.sin(ang)], -1), 0.0, a)
        x = np.stack(xs).astype(np.float32)
    elif c["kind"] == "snr":
        lo, hi = c["snr"]
        x = rs.uniform(lo, hi, size=(T, E, R)).astype(np.float32)
    elif c["kind"] == "pg":
        # the path gain of every robot-cell link [T,E,R,C] (dB): a per-link level plus a slow random walk
        lo, hi = c["pg"]
        p = rs.uniform(lo, hi, size=(E, R, c["cfg"]["n_cells"]))
        xs = []
        for _ in range(T):
            xs.append(p.copy())
            p = np.clip(p + rs.normal(0.0, c["pg_walk"], size=p.shape), lo, hi)
        x = np.stack(xs).astype(np.float32)
    else:
        lo, hi = c["snr"]
        x = rs.uniform(lo, hi, size=(T, E, R, 1)) + rs.normal(0.0, 2.0, size=(T, E, R, c.get("subbands", 13)))
        x = x.astype(np.float32)
    assert counts.shape == (T, E, R, n_cls)
    if "dl_rates" in c:
        dl = np.stack([rs.poisson(lam, size=(T, E, R)) for lam in c["dl_rates"]], -1).astype(np.int64)
        return x, counts, dl
    return x, counts


def _vel(name, c):
    """The velocity input [T,E,R,2] float32 (m/s, normal with sigma c["vel"] per axis) of a case with one, else None."""
    if "vel" not in c:
        return None
    rs = np.random.default_rng(int.from_bytes(hashlib.sha256((name + ":vel").encode()).digest()[:4], "little"))
    return rs.normal(0.0, c["vel"], size=(c["steps"], c["E"], c["R"], 2)).astype(np.float32)


def _np(v):
    """A copy (the reference updates some state tensors in place: rng counters, episode, epoch)."""
    return np.array(v.detach().cpu().numpy(), copy=True)


def run_case(name, c):
    NRConfig, make_engine, state_dict, Requests = _ref()
    cfg = NRConfig(**c["cfg"], seed=0)
    E, R, T = c["E"], c["R"], c["steps"]
    eng = make_engine("L2", E, R, "cpu", cfg, backend="reference", seed=0, strict=None)
    x, counts, *dl = _inputs(name, c)
    dl_counts = dl[0] if dl else None
    vel = _vel(name, c)
    out = {"x": x, "counts": counts, "E": np.int64(E), "R": np.int64(R), "steps": np.int64(T),
           "cfg_json": np.frombuffer(json.dumps(c["cfg"]).encode(), dtype=np.uint8),
           "kind": np.frombuffer(c["kind"].encode(), dtype=np.uint8)}
    if dl_counts is not None:
        out["dl_counts"] = dl_counts
        out["dl_sizes"] = np.asarray(c["dl_sizes"], dtype=np.float32)
    if vel is not None:
        out["vel"] = vel
    reset_mask = np.zeros((T, E), dtype=np.bool_)
    for s, ids in c["resets"].items():
        reset_mask[s, ids] = True
    out["reset_mask"] = reset_mask
    keys_seen = set()

    def snap(prefix):
        sd = state_dict(eng)
        for k, v in sd.items():
            if torch.is_tensor(v):
                out[f"{prefix}/{k}"] = _np(v)
                keys_seen.add(k)
        rad = eng.radio
        if rad is not None:
            if rad.k is not None:
                out[f"{prefix}/radio.k"] = _np(rad.k)
                out[f"{prefix}/radio.phi"] = _np(rad.phi)
            if rad.ch is not None:
                for fname in ("sf_los", "sf_nlos", "los_field"):
                    f = getattr(rad.ch, fname)
                    out[f"{prefix}/radio.{fname}.k"] = _np(f.k)
                    out[f"{prefix}/radio.{fname}.phi"] = _np(f.phi)

    snap("init")
    for s in range(T):
        ids = np.nonzero(reset_mask[s])[0]
        if len(ids):
            eng.reset(torch.tensor(ids, dtype=torch.long))
            snap(f"reset{s:03d}")
        # arrivals: for each class in order, one submit per message index (harness order, class 1 first)
        acc_all = []
        for ci in range(counts.shape[-1]):
            n = torch.from_numpy(counts[s, :, :, ci])
            for i in range(int(n.max())):
                send = torch.where(n > i, torch.full_like(n, ci + 1), torch.zeros_like(n))
                acc_all.append(_np(eng.submit(None, Requests(send=send))))
        out[f"s{s:03d}/n_submit"] = np.int64(len(acc_all))
        if acc_all:
            out[f"s{s:03d}/accepted"] = np.stack(acc_all)
        if dl_counts is not None:
            # downlink arrivals: for each DL class in order, one add_dl_frames per message index (bytes, class)
            for ci in range(dl_counts.shape[-1]):
                n = torch.from_numpy(dl_counts[s, :, :, ci])
                for i in range(int(n.max())):
                    nb = torch.where(n > i, torch.full(n.shape, c["dl_sizes"][ci]), torch.zeros(n.shape))
                    eng.add_dl_frames(None, nb, torch.where(n > i, torch.full_like(n, ci + 1), torch.zeros_like(n)))
        xs = torch.from_numpy(x[s])
        if c["kind"] == "pose":
            o = eng.step(None, xs, vel=None if vel is None else torch.from_numpy(vel[s]))
        elif c["kind"] == "snr":
            o = eng.step(None, xs)
        elif c["kind"] == "pg":
            o = eng.step(None, pathgain_db=xs)
        else:
            o = eng.step(None, snr_db=xs)
        for k, v in o.items():
            out[f"s{s:03d}/out.{k}"] = _np(v)
        snap(f"s{s:03d}")
    out["counters_json"] = np.frombuffer(json.dumps(eng.counters()).encode(), dtype=np.uint8)
    np.savez_compressed(os.path.join(HERE, f"traj_{name}.npz"), **out)
    print(name, "state keys:", len(keys_seen), "arrays:", len(out))


def run_stats_case(name, c):
    """The statistics of NRNet with log_stats on: per step queued() and refused_env, at the end collect() (each list
    entry as one array, each count as an int64)."""
    NRConfig, make_engine, state_dict, Requests = _ref()
    cfg = NRConfig(**c["cfg"], seed=0)
    E, R, T = c["E"], c["R"], c["steps"]
    eng = make_engine("L2", E, R, "cpu", cfg, backend="reference", seed=0, strict=None)
    eng.log_stats = True
    if "log_cap_max" in c:
        eng.net.log_cap_max = c["log_cap_max"]
    x, counts, *dl = _inputs(name, c)
    dl_counts = dl[0] if dl else None
    out = {"x": x, "counts": counts, "E": np.int64(E), "R": np.int64(R), "steps": np.int64(T),
           "cfg_json": np.frombuffer(json.dumps(c["cfg"]).encode(), dtype=np.uint8),
           "kind": np.frombuffer(c["kind"].encode(), dtype=np.uint8),
           "log_cap_max": np.int64(c.get("log_cap_max", 10 ** 9))}
    if dl_counts is not None:
        out["dl_counts"] = dl_counts
        out["dl_sizes"] = np.asarray(c["dl_sizes"], dtype=np.float32)
    reset_mask = np.zeros((T, E), dtype=np.bool_)
    for s, ids in c["resets"].items():
        reset_mask[s, ids] = True
    out["reset_mask"] = reset_mask
    for s in range(T):
        ids = np.nonzero(reset_mask[s])[0]
        if len(ids):
            eng.reset(torch.tensor(ids, dtype=torch.long))
        for ci in range(counts.shape[-1]):
            n = torch.from_numpy(counts[s, :, :, ci])
            for i in range(int(n.max())):
                eng.submit(None, Requests(send=torch.where(n > i, torch.full_like(n, ci + 1), torch.zeros_like(n))))
        if dl_counts is not None:
            for ci in range(dl_counts.shape[-1]):
                n = torch.from_numpy(dl_counts[s, :, :, ci])
                for i in range(int(n.max())):
                    nb = torch.where(n > i, torch.full(n.shape, c["dl_sizes"][ci]), torch.zeros(n.shape))
                    eng.add_dl_frames(None, nb, torch.where(n > i, torch.full_like(n, ci + 1), torch.zeros_like(n)))
        xs = torch.from_numpy(x[s])
        eng.step(None, xs) if c["kind"] != "snr3" else eng.step(None, snr_db=xs)
        out[f"s{s:03d}/queued"] = _np(eng.queued())
        out[f"s{s:03d}/refused_env"] = _np(eng.net.refused_env)
    col = eng.collect()
    out["collect_keys"] = np.frombuffer(json.dumps(list(col.keys())).encode(), dtype=np.uint8)
    for k, v in col.items():
        out[f"collect/{k}"] = _np(v) if torch.is_tensor(v) else np.int64(v)
    np.savez_compressed(os.path.join(HERE, f"stats_{name[len('stats_'):]}.npz"), **out)
    print(name, {k: (tuple(v.shape) if torch.is_tensor(v) else v) for k, v in col.items()})


def run_wifi_case(name, c):
    """A level WIFI trajectory: per step the submits (one call per class and message index), the step dict and the
    engine's state_dict() after the step (FIFO, clock, mean-field state, counter RNG, radio)."""
    sys.path.insert(0, REF)
    from isaac_net.core.config import NRConfig
    from isaac_net.core.engine import make_engine
    from isaac_net.core.wifi import WifiConfig
    cfg = NRConfig(**c["cfg"], wifi=WifiConfig(**c["wifi"]), seed=0)
    E, R, T = c["E"], c["R"], c["steps"]
    eng = make_engine("WIFI", E, R, "cpu", cfg, backend="reference", seed=0, strict=None)
    x, counts = _inputs(name, c)
    out = {"x": x, "counts": counts, "E": np.int64(E), "R": np.int64(R), "steps": np.int64(T),
           "cfg_json": np.frombuffer(json.dumps(c["cfg"]).encode(), dtype=np.uint8),
           "wifi_json": np.frombuffer(json.dumps(c["wifi"]).encode(), dtype=np.uint8),
           "kind": np.frombuffer(("snr" if c["kind"] == "snr" else "pose").encode(), dtype=np.uint8),
           "K": np.int64(eng.Ksub), "n_acc_max": np.int64(eng.n_acc_max)}
    reset_mask = np.zeros((T, E), dtype=np.bool_)
    for s, ids in c["resets"].items():
        reset_mask[s, ids] = True
    out["reset_mask"] = reset_mask

    dynamic = ("cap", "cls", "det", "hid", "rem", "dlv", "f_nact", "f_snr", "f_own", "clock", "_last_snr",
               "_last_hid", "tau", "roam_left", "att_n", "att_logp", "credit", "serv", "pending", "rng.episode",
               "rng.ctr[1]", "rng.ctr[2]")

    def snap(prefix, full=False):
        """full: every tensor of state_dict() but generator states; else the state that a step or reset changes
        (and the radio's plane waves)."""
        for k, v in eng.state_dict().items():
            if not torch.is_tensor(v) or k.endswith("gen"):
                continue
            if full or k in dynamic or (k.startswith("radio.") and k.endswith((".k", ".phi"))):
                out[f"{prefix}/{k}"] = _np(v)

    snap("init", full=True)
    for s in range(T):
        ids = np.nonzero(reset_mask[s])[0]
        if len(ids):
            eng.reset(torch.tensor(ids, dtype=torch.long))
            snap(f"reset{s:03d}")
        acc_all = []
        for ci in range(counts.shape[-1]):
            n = torch.from_numpy(counts[s, :, :, ci])
            for i in range(int(n.max())):
                send = torch.where(n > i, torch.full_like(n, ci + 1), torch.zeros_like(n))
                acc_all.append(_np(eng.submit(None, send)))
        out[f"s{s:03d}/n_submit"] = np.int64(len(acc_all))
        if acc_all:
            out[f"s{s:03d}/accepted"] = np.stack(acc_all)
        o = eng.step(None, torch.from_numpy(x[s]))
        for k, v in o.items():
            out[f"s{s:03d}/out.{k}"] = _np(v)
        snap(f"s{s:03d}")
    np.savez_compressed(os.path.join(HERE, f"traj_{name}.npz"), **out)
    print(name, "arrays:", len(out))


def checkpoint_vectors(name, k_steps=10):
    """The reference engine's checkpoint (core/checkpoint.py:103-143 collect: NREngine.state_dict()) of a golden
    case after k_steps steps, with the case's own inputs: tensors under "ck/<key>", host values as JSON."""
    NRConfig, make_engine, state_dict, Requests = _ref()
    c = CASES[name]
    cfg = NRConfig(**c["cfg"], seed=0)
    E, R = c["E"], c["R"]
    eng = make_engine("L2", E, R, "cpu", cfg, backend="reference", seed=0, strict=None)
    x, counts, *dl = _inputs(name, c)
    dl_counts = dl[0] if dl else None
    for s in range(k_steps):
        assert not any(s == r for r in c["resets"])
        for ci in range(counts.shape[-1]):
            n = torch.from_numpy(counts[s, :, :, ci])
            for i in range(int(n.max())):
                eng.submit(None, Requests(send=torch.where(n > i, torch.full_like(n, ci + 1), torch.zeros_like(n))))
        if dl_counts is not None:
            for ci in range(dl_counts.shape[-1]):
                n = torch.from_numpy(dl_counts[s, :, :, ci])
                for i in range(int(n.max())):
                    nb = torch.where(n > i, torch.full(n.shape, c["dl_sizes"][ci]), torch.zeros(n.shape))
                    eng.add_dl_frames(None, nb, torch.where(n > i, torch.full_like(n, ci + 1), torch.zeros_like(n)))
        eng.step(None, torch.from_numpy(x[s]))
    sd = eng.state_dict()
    out, host = {}, {}
    for k, v in sd.items():
        if torch.is_tensor(v):
            out["ck/" + k] = _np(v)
        else:
            host[k] = v if not isinstance(v, tuple) else list(v)
    out["host_json"] = np.frombuffer(json.dumps(host).encode(), dtype=np.uint8)
    out["k_steps"] = np.int64(k_steps)
    np.savez_compressed(os.path.join(HERE, f"ckpt_{name}.npz"), **out)
    print(name, "checkpoint:", len(sd), "entries,", len(host), "host values")


def eventsim_vectors():
    """Saturation statistics of the reference's CSMA/CA event simulator (core/wifi/eventsim.py:56-186) for the
    exchange times of the DCF level (802.11ax 20 MHz MCS 11, 1472-byte MSDUs without aggregation, legacy DCF
    parameters): per n stations, attempts, successes and the busy share over 4 s. The DCF level's oracle is compared
    with them statistically (its draws come from the engine's counter RNG, the simulator's from numpy PCG64)."""
    sys.path.insert(0, REF)
    sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
    from isaac_net.core.wifi import eventsim as ev
    import importlib.util
    d = os.path.join(os.path.dirname(os.path.dirname(HERE)), "isaac-net_amd")
    spec = importlib.util.spec_from_file_location("isaac_net_amd", os.path.join(d, "__init__.py"),
                                                  submodule_search_locations=[d])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["isaac_net_amd"] = mod
    spec.loader.exec_module(mod)
    from oracle.dcf_oracle import DcfOracle
    from isaac_net_amd.wifi_config import WifiConfig
    cfg = mod.NRConfig(control_step_ms=20.0, msg_sizes=(60000.0,), wifi=WifiConfig(access_category="DCF",
                                                                                     max_ampdu_bytes=0))
    o = DcfOracle(1, 2, cfg)
    succ_ns, coll_ns = o.busy(1472, o.k["ndbps"][-1])
    out = {"busy_succ_us": np.float64(succ_ns / 1000.0), "busy_coll_us": np.float64(coll_ns / 1000.0),
           "n": np.array([5, 10, 20], np.int64), "sim_us": np.float64(4e6)}
    att, succ, busy = [], [], []
    for n in (5, 10, 20):
        st = [ev.Station(16, 1024, 2, 1472.0, ev.Const(succ_ns / 1000.0), ev.Const(coll_ns / 1000.0), 7, 0.0)
              for _ in range(n)]
        r = ev.run(st, 4e6, 9.0, 16.0, arrivals=None, seed=0)
        att.append(int(r["n_att"].sum()))
        succ.append(int(r["n_succ"].sum()))
        busy.append(float(r["busy_frac"]))
    out.update(n_att=np.array(att, np.int64), n_succ=np.array(succ, np.int64), busy_frac=np.array(busy))
    np.savez_compressed(os.path.join(HERE, "eventsim_sat.npz"), **out)
    print("eventsim vectors written", att, succ, busy)


def phy_tables():
    """Processed PHY tables of both MCS tables (core/phy.py PHY): BLER table, grids, betas, thresholds, TBS."""
    NRConfig, make_engine, state_dict, Requests = _ref()
    from isaac_net.core.phy import PHY, tbs_38214, segment
    out = {}
    for mt in (1, 2):
        ph = PHY("ul", mt, "cpu")
        b = ph.bler.numpy()
        out[f"t{mt}/bler_sha256"] = np.frombuffer(hashlib.sha256(np.ascontiguousarray(b).tobytes()).digest(),
                                                  dtype=np.uint8)
        out[f"t{mt}/bler_shape"] = np.array(b.shape, dtype=np.int64)
        rs = np.random.default_rng(mt)
        idx = np.stack([rs.integers(0, s, size=4000) for s in b.shape[1:]], -1)
        out[f"t{mt}/sample_idx"] = idx
        out[f"t{mt}/sample_val"] = b[0, idx[:, 0], idx[:, 1], idx[:, 2]]
        out[f"t{mt}/snr_grid"] = ph.snr_grid.numpy()
        out[f"t{mt}/cbs_axis"] = ph.cbs_axis.numpy()
        out[f"t{mt}/beta"] = ph.beta.numpy()
        out[f"t{mt}/thr_ref"] = ph.thr_ref.numpy()
        out[f"t{mt}/thr"] = ph.thr.numpy()
        out[f"t{mt}/mcs_eq"] = ph.mcs_eq.numpy()
        out[f"t{mt}/se"] = ph.se.numpy()
        for ns in (2, 4, 12, 13):
            n = torch.arange(0, 274, dtype=torch.float32)
            tbs = ph.tbs_all(n, ns, 12, 0)
            out[f"t{mt}/tbs_ns{ns}"] = tbs.numpy()
            cbs, c, bg = ph.cb(tbs, ph.r)
            out[f"t{mt}/cbs_ns{ns}"] = cbs.numpy()
            out[f"t{mt}/ncb_ns{ns}"] = c.numpy()
    # a few TBS values at other dmrs / overhead and two layers
    n = torch.arange(0, 274, dtype=torch.float32)[:, None]
    out["tbs_oh6_l2"] = tbs_38214(torch.tensor([2.0, 4.0, 6.0, 8.0]), torch.tensor([0.2, 0.5, 0.7, 0.93]), n, 12,
                                  12, 6, 2).numpy()
    np.savez_compressed(os.path.join(HERE, "phy_tables.npz"), **out)
    print("phy tables written")


def rng_vectors():
    """Counter-RNG draws (core/proto/rng.py) for a few keys: uniforms and normals, step and reset channels."""
    sys.path.insert(0, REF)
    from isaac_net.core.proto import rng as R_
    out = {}
    r = R_.CounterRNG(0xC0FFEE1234, 6, "cpu")
    r.reset(None)
    r.reset(torch.tensor([1, 4]))
    r.tick(R_.STEP)
    r.tick(R_.STEP)
    out["seed"] = np.int64(0xC0FFEE1234)
    out["episode"] = r.episode.numpy()
    out["ctr_step"] = r.ctr[R_.STEP].numpy()
    out["u_step_s5"] = r.uniform(R_.STEP, (2 << 16) | 5, 37).numpy()
    out["n_step_s3"] = r.normal(R_.STEP, (1 << 16) | 3, 52).numpy()
    out["u_reset_s0"] = r.reset_uniform(None, 6 << 16, 9).numpy()
    out["n_reset_s0"] = r.reset_normal(None, 4 << 16, 20).numpy()
    out["s0"] = np.int64(r.s0)
    np.savez_compressed(os.path.join(HERE, "rng_vectors.npz"), **out)
    print("rng vectors written")


if __name__ == "__main__":
    torch.set_num_threads(1)
    names = sys.argv[1:] or list(CASES) + list(WIFI_CASES) + list(STATS_CASES) + ["eventsim"]
    if not sys.argv[1:]:
        rng_vectors()
        phy_tables()
    for n in names:
        if n == "eventsim":
            eventsim_vectors()
        elif n.startswith("ckpt_"):
            checkpoint_vectors(n[len("ckpt_"):])
        elif n in WIFI_CASES:
            run_wifi_case(n, WIFI_CASES[n])
        elif n in STATS_CASES:
            run_stats_case(n, STATS_CASES[n])
        else:
            run_case(n, CASES[n])

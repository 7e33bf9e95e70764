/*
 * inet_nr.h -- C ABI of the MI355X-native NR engine (libinet_nr.so, HIP kernels for gfx950).
 *
 * Drop-in boundary for isaac-net's per-control-step NR engine hot path (level "L2": one cell with uplink and
 * downlink, or several cells with the uplink). The reference launches its fused Triton kernel through
 *     nr_triton.launch_step(eng, uref, dref, pc, itab, ftab, K, gate, dgate)      isaac_net/core/nr_triton.py:1104-1167
 * from NRTritonEngine._triton_step (isaac_net/core/nr_fast.py:702-752), and runs the enqueue (NRNet.add_frames,
 * isaac_net/core/nr_engine.py:466-487) and partial reset (NREngine.reset, isaac_net/core/engine.py:763-794) as eager
 * torch code. This library replaces all three with plain-pointer entry points:
 *
 *   inet_nr_step    one control step: radio prologue, every scheduled slot (fading, SR, UL MAC), the RLC
 *                   epilogue (delivered / timed-out / dropped, compaction) and the step outputs.
 *                   Replaces launch_step + the torch prologue/epilogue of _triton_step (nr_fast.py:702-752,
 *                   nr_engine.py:843-888) and the radio of NREngine._pathgain (engine.py:853-865).
 *   inet_nr_submit  enqueue one message per robot (FrameQueue.add / NRNet.add_frames, queues.py:87-103,
 *                   nr_engine.py:466-487), or several per robot in class order (counts form).
 *   inet_nr_reset   partial or full reset of an env mask (NRNet.reset, MacLink.reset, FrameQueue.reset,
 *                   NRRng.reset_mask, RadioMC.reset: nr_engine.py:250-320, mac.py:176-189, queues.py:70-78,
 *                   nr_rng.py:45-52, radio.py:200-219).
 *   inet_nr_dl_step, inet_nr_dl_submit, inet_nr_dl_reset   the downlink of NRConfig(dl=True) (DlMac, mac_dl.py:19-49;
 *                   NRNet.add_dl_frames, nr_engine.py:489-497), declared at the end of this header.
 *   inet_nr_step_cells, inet_nr_cells_reset   several cells per env (NRNet.step_cells, nr_engine.py:718-788, with
 *                   CellAssociation, radio.py:303-453): the step with association, A3 handover, one scheduler per
 *                   cell and same-slot inter-cell interference, and the reset of the association state.
 *
 * Conventions
 *   Ownership  The caller allocates and owns every buffer (device memory); the library never allocates or frees
 *              and updates state in place, so a call can be captured in a HIP graph.
 *   Layout     Robot-minor SoA: per-robot scalars [E][R]; per-subband [E][S][R]; per-HARQ-process [E][P][R];
 *              per-frame state [E][F][R]. Step outputs use the reference's [E][R][F] layout and dtypes.
 *   Errors     Every entry point returns 0 on success or a negative INET_NR_E* code, checked before any launch.
 *   Threading  Call from one host thread; work is enqueued on `stream` (a hipStream_t), with no host sync and no
 *              host read of device data.
 */
#ifndef INET_NR_H
#define INET_NR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define INET_NR_ABI_VERSION 15
#define INET_NR_MAX_S 32          /* subbands (RBGs) */
#define INET_NR_MAX_P 16          /* HARQ processes */
#define INET_NR_MAX_R 256         /* robots per env: a segment of one 64-wide wavefront (up to 64), or two / four
                                     wavefronts (65..128 / 129..256: the UL with pose or SNR [E][R] input, one cell;
                                     four wavefronts with 8 or 13 subbands) */
#define INET_NR_MAX_KF 16         /* plane waves per shadowing field */
#define INET_NR_NCTR 13           /* per-env counters, see InetNrState.ctr */
#define INET_NR_MAX_ROWS 64       /* scheduled slots (InetNrRow) per control step */
#define INET_NR_MAX_C 7           /* cells per env */

#define INET_NR_OK 0
#define INET_NR_EINVAL (-1)       /* a size or pointer argument is out of range or missing */
#define INET_NR_EUNSUPPORTED (-2) /* a feature flag this build does not implement */
#define INET_NR_ELAUNCH (-3)      /* the HIP runtime refused a launch */

/* Per-env engine state (all device pointers). */
typedef struct InetNrState {
    /* MAC per robot [E][R] (mac.py:67-81, mac_ul.py) */
    int32_t *sent, *floor_, *bsr, *sr_t, *last_tx;
    float *olla, *avg;
    /* queue per robot [E][R]: stream length and number of queued frames (frames are a prefix) */
    int32_t *enq, *qlen;
    /* per subband [E][S][R]: CSI (last PUSCH gain, dB); the AR(1) fading state h = re + j im of every robot-cell
       link [E][C][S][R] (C = n_cells) */
    float *csi, *h_re, *h_im;
    /* HARQ [E][P][R]: meta = state | ntx << 8 | mcs << 16 | nsb << 24; byte ranges, ready slot, TBS (bits),
       chase-combined linear SINR, IR log-sum and PRB count */
    uint32_t *h_meta;
    int32_t *h_lo, *h_hi, *h_ready, *h_tbs;
    float *h_comb, *h_lexp, *h_nrb;
    /* frames [E][F][R]: capture step, byte range, completion slot (INT32_MAX = not completed),
       meta = lost | det << 1 | cls << 8, hazard id */
    int32_t *q_cap, *q_start, *q_end, *q_fin;
    uint32_t *q_meta;
    int32_t *q_hid;
    /* Rician specular phasor and K (linear) per robot-cell link [E][C][R] (C = n_cells, 1 with one cell; several
       cells since ABI 14) */
    float *spec_re, *spec_im, *k_lin;
    /* counter RNG per env [E]: env id (global), episode, step and submit call counters */
    int32_t *env_id, *episode, *ctr_step, *ctr_submit;
    /* engine clock epoch per env [E] */
    int32_t *epoch;
    /* shadowing plane waves per env and cell [E][C][NF][KF][3] = (kx, ky, phi), NF = 3 (tr38901) or 1
       (log_distance) */
    float *field;
    /* per-env counters [E][INET_NR_NCTR] int64: tb_new, tb_retx, tb_ok, tb_fail, exhaust, bytes_ok, bytes_new,
       lost_frames, new_while_pending, prb_used, and the 5G-LENA grant accounting tb_bytes, tb_empty, retx_block
       (mac.py:119-122, 299, 492-493; accumulated always, reported by the engine when a LENA switch is on); and
       per-env HARQ histograms
       [E][3][max_tx + 1] int64: decoded TBs by transmissions, TBs sent as transmission k, failed as transmission k */
    int64_t *ctr, *hist;
    /* the engine's control-step counter T on the device [1] int64: read by inet_nr_step / inet_nr_submit when
       they are called with T < 0 (a launch recorded once in a HIP graph and replayed at every step) */
    int64_t *clock;
    /* per robot [E][R] int64: the byte-stream base of the link. The reference's stream offsets (sent, floor, enq,
       h_lo, h_hi, q_start, q_end: int64 in queues.py:52-60, mac.py:67-81) are base + the int32 values above. When a
       robot's floor reaches params.rebase_at at the end of a step, the step moves its offsets down by the floor and
       adds it to base, so the int32 values stay below 2^31 for any run length. */
    int64_t *base;
    /* per robot [E][R] float: PRBs of the robot's last PUSCH (UlMac.last_nprb, mac_ul.py:51, mac.py:484), read and
       written only with params.amc_prev (ABI version 8) */
    float *last_nprb;
    /* per link [E][C][R] float: the LOS K draw of Rician fading with K from the LOS state (NRNet.k_los,
       nr_engine.py:300-303), written by inet_nr_reset with params.k_from_los (ABI version 10) */
    float *k_los;
    /* Rician K from the LOS state, the ramp (nr_engine.py:402-419; ABI 12): per link [E][C][R] the ramp start k_from and
       its slot k_g0 (k_lin is the target), per env [E] k_fresh (no LOS state seen since the reset). The step kernels
       apply NRNet.set_los with the radio's LOS state of a pose step (K target = k_los where LOS, else 0; a fresh env
       takes it at once), start a ramp of k_ramp slots where the target changed, and evaluate K in every slot. */
    float *k_from;
    int32_t *k_g0, *k_fresh;
    /* Per-link delay spreads (fc_on = 2, nr_engine.py:341-381; ABI 13): per robot [E][R] the grid index of fc_tab in
       use (fc_idx) and those of the link's LOS and NLOS draws (fc_idl, fc_idn), drawn at reset; a pose step on TR 38.901
       selects the LOS or NLOS one by the radio's LOS state (NLOS until one is reported). */
    int32_t *fc_idx, *fc_idl, *fc_idn;
    /* Per-robot Doppler (fading_doppler = "per_robot": engine.py:862-864, radio.py:285-300, channels/doppler.py:23-29;
       ABI 15): per robot [E][R] the last pose (x, y) ([E][R][2]), whether it is set (0 after a reset), and the AR(1)
       correlation per ms (NRNet.fading_rho_ms; the caller sets it to fading_rho_per_ms at creation). A pose step sets
       the speed from params.vel or |pose - last pose| / control step, floored at dop_floor, and from it the
       correlation J0(dop_kx v dop_kf)^(1 / 2.5) (0 from the first zero of J0 on); every fading row then evolves with
       rho = rho_ms^(row.rho) (row.rho holds the exponent dt slot_ms) and sqrt(1 - rho^2). The DL step reads them,
       the UL step writes them. */
    float *prev_pos;
    int32_t *has_prev;
    float *rho_ms;
} InetNrState;

/* Device tables (PHY) and the host constants that go with them. */
typedef struct InetNrTables {
    const float *bler;        /* [M][C][G] code-block BLER */
    const float *thr_ref;     /* [M] target-BLER SINR of one 10-PRB RBG */
    const float *se;          /* [M] spectral efficiency Qm R */
    const float *beta;        /* [M] EESM beta */
    const float *rate;        /* [M] code rate R */
    const int32_t *mcs_eq;    /* [M][EQW] HARQ-IR equivalent MCS */
    const int32_t *la_tbs;    /* [NSYM][NPRB + 1][M] TBS bits */
    const int32_t *la_ci0;    /* [NSYM][NPRB + 1][M] code-block-size index */
    const float *la_cwi;      /* [NSYM][NPRB + 1][M] its interpolation weight */
    const float *la_ncb;      /* [NSYM][NPRB + 1][M] number of code blocks */
    const float *w;           /* [S] PRBs per subband */
    const float *logw;        /* [S] log(w) */
    const float *wdb;         /* [S] 10 log10(w / snr_ref_prbs) */
    float s0, ds, c0, dc;     /* SNR grid origin / step, code-block axis origin / step */
    int32_t M, C, G, NPRB, EQW, mcs_max;
    int32_t thr_monotone;     /* informational: thr_ref[0..mcs_max] non-decreasing (the kernels search its suffix
                                 minima, which give the highest passing MCS for any table) */
    int32_t pad;
} InetNrTables;

/* Config constants of the step (derived on the host from NRConfig). */
typedef struct InetNrParams {
    int32_t E, R, S, P, F, N;         /* envs, robots, subbands, HARQ processes, frame buffer, slots per step */
    int32_t sched;                    /* 0 pf, 1 maxci, 2 rr */
    int32_t comb;                     /* 0 none, 1 cc, 2 ir_lena */
    int32_t eesm;                     /* 1 eesm, 0 mean_db */
    int32_t harq_drop, olla, phr_cap, retx_prio, rician, fading, purge, input_kind, radio_model, out_ref;
    int32_t max_tx, sr_delay, ul_rtt, rlc_retx, timeout, tb_oh, n_fields, n_modes, seed_key;
    int32_t n_data;                   /* data rows (flag 2) among the step's rows: sizes the kernel's per-slot LDS
                                         history (0: n_rows); must not be smaller than the actual count */
    int32_t n_cells;                  /* cells per env C (1: the single-cell engine; > 1: inet_nr_step_cells) */
    int32_t rebase_at;                /* floor (bytes) from which a step rebases a robot's byte offsets (InetNrState.base;
                                         2^30; 0: never) */
    /* 5G-LENA MAC switches (isaac_net/core/mac.py:26-31, 525-554; mac_ul.py:154-180) and UL power control at one cell
       (nr_engine.py:649-650, 671-675); ABI version 7 */
    int32_t pf_rbg;                   /* pf_update="rbg": the winner's PF average moves after every RBG grant */
    int32_t pf_freeze;                /* pf_avg_idle="freeze": only robots with new data to schedule update it */
    int32_t whole_band;               /* ul_power="whole_band": fixed PSD over the carrier (wb_db), no PHR cap */
    int32_t pc1_on;                   /* one cell, UL power control from the mean UL reference SINR */
    int32_t retx_tdma;                /* ul_retx_sched="tdma" (mac.py:279-299): one UL retransmission per slot and cell,
                                         the oldest NACK, and no new data in that slot (ABI version 8) */
    int32_t amc_prev;                 /* ul_amc_alloc="previous" (mac.py:393-401): the UL MCS for the PRBs of the last
                                         PUSCH (InetNrState.last_nprb), the TB for this allocation (ABI version 8) */
    int32_t fc_on;                    /* frequency-correlated fading (nr_engine.py:43-48, 320-368): every fading
                                         innovation and reset draw z becomes L z; 1: L = fc_L, one fixed delay spread
                                         (ABI 9); 2: L = fc_tab[fc_idx] per link, per-link delay spreads (ABI 13) */
    int32_t k_from_los;               /* Rician K from the LOS state: inet_nr_reset draws k_los = 10^((k_mu + k_sigma z)
                                         / 10), z the link's KFAC normal, and sets k_lin = 0 (ABI 10) */
    int32_t los_sto;                  /* TR 38.901 stochastic LOS state (models.py:121-167): LOS where u(x) < Pr_LOS(d_2D),
                                         u the LOS-state field (field 2) through los_cdf; NLOS path loss and sig_nlos
                                         elsewhere (ABI 11) */
    int32_t plos_scn;                 /* los_sto: the Pr_LOS formula, 0 UMi, 1 UMa (h_UT <= 13 m), 2 InH */
    int32_t k_ramp;                   /* k_from_los: rician_k_ramp_slots (0: a new target applies at once) */
    int32_t fc_G;                     /* fc_on 2: grid points of fc_tab (fading_ds_grid) */
    int32_t doppler;                  /* per-robot Doppler (InetNrState.rho_ms; ABI 15) */
    int32_t pf_wb;                    /* the wideband rate in the scheduler's metric (pf_metric "wideband", scheduler
                                         "pf_wideband"; mac.py:259-264; ABI 15): every RBG gets the rate of the highest
                                         MCS whose effective SINR over all RBGs reaches its threshold */
    float olla_up, olla_dn, pf_a, pf_b, target, phr_min, snr_ref_prbs, w0;
    float ref_off, noise_prb, ue_tx, subband_noise;   /* ul_ref = (pg + ref_off) - noise_prb; snr = (pg + ue_tx) - subband_noise */
    /* radio constants (float32 values of the reference's Python doubles) */
    float gnb_x, gnb_y, hh2, dbp, pl_a, pl_n1, pl_c20, pl_c2, nl_b1, nl_b0, nl_c, nl_d, sig, amp, pl_const, pl_exp10;
    float proc_off_hi, proc_off_lo;   /* proc_offset_ms / control_step_ms as a double split in two floats */
    float wb_db;                      /* whole_band: 10 log10(nprb / snr_ref_prbs) */
    float pc_p0, pc_alpha;            /* pc1_on: P0 (dBm) and alpha of the fractional power control */
    float k_mu, k_sigma;              /* k_from_los: (mu_K, sigma_K) dB of the scenario, TR 38.901 Table 7.5-6 */
    float sig_nlos;                   /* los_sto: NLOS shadow-fading sigma (dB); sig is the LOS one */
    float k_rinv;                     /* k_from_los: 1 / k_ramp as float32 (the ramp's step per slot) */
    /* fc_on 2: lgDS = mu + sigma z (float32) of the NLOS and the LOS state (TR 38.901 Table 7.5-6), its grid index
       round((lgDS + 9 - ds_c1) ds_c2) clamped to [0, fc_G - 1], ds_c1 = log10(min ns), ds_c2 = (G - 1) / log10(max/min) */
    float ds_mu_n, ds_sig_n, ds_mu_l, ds_sig_l, ds_c1, ds_c2;
    /* doppler: speed floor (m/s), f_c / c (float32 of carrier_ghz 1e9 / c), 2 pi 2.5 ms (float32), control step (s) */
    float dop_floor, dop_kf, dop_kx, dop_dt;
    const float *fc_L;                /* fc_on: [S][S] lower-triangular square root of the subband correlation */
    const float *los_cdf;             /* los_sto: [65536] sorted samples of a unit sum of cosines (fields.py:94-106) */
    const float *fc_tab;              /* fc_on 2: [fc_G][S][S] square roots of the subband correlation on the grid */
    const float *vel;                 /* doppler, this call only: the velocity input [E][R][2] (m/s) of a pose step, or
                                         NULL (the speed from consecutive poses) */
} InetNrParams;

/* One scheduled slot of the control step (host-built per TDD key, device resident). */
typedef struct InetNrRow {
    int32_t rel;          /* slot index inside the control step */
    int32_t nsym_idx;     /* index into the LA tables (-1: no UL data symbols) */
    int32_t flags;        /* 1 SR opportunity, 2 UL data, 4 fading evolves, 8 fading state needed, 16 proactive grant */
    float re_prb;         /* data REs per PRB of the UL slot */
    float rho, c1;        /* AR(1) coefficients rho^(dt slot_ms) and sqrt(1 - rho^2), as float32 (params.doppler:
                             rho = the exponent dt slot_ms, c1 unused) */
    uint32_t salt_fade;   /* salt((FADING << 16) | rel) */
    uint32_t salt_bler;   /* salt((BLER_UL << 16) | rel) */
} InetNrRow;

/* Step outputs. out_ref = 1: reference dtypes and layout; 0: compact form (flags/delay/cap/cls of every frame). */
typedef struct InetNrOutputs {
    uint8_t *delivered, *timed_out, *dropped;   /* [E][R][F] bool (out_ref = 1); flags bit 0/1/2 in delivered (0) */
    int64_t *cap, *cls;                          /* [E][R][F] int64 (out_ref = 1) */
    int32_t *cap32;                              /* [E][R][F] int32 (out_ref = 0) */
    uint8_t *cls8;                               /* [E][R][F] uint8 (out_ref = 0) */
    float *delay;                                /* [E][R][F] float32 */
    int64_t *newest, *queue_len, *serving_cell;  /* [E][R] int64 */
    float *queue_bytes, *sinr_db;                /* [E][R] float32 */
    uint8_t *det_env;                            /* [E] bool */
    int64_t *t;                                  /* [E] int64 */
} InetNrOutputs;

/* The downlink of NRConfig(dl=True) (DlMac, isaac_net/core/mac_dl.py:19-49, on MacLink, mac.py:65-616): the DL
   link's MAC state and frame queue (the same fields and layouts as the UL link's in InetNrState), its step outputs
   and constants. The state both links share (fading h_re / h_im, Rician spectrum, RNG words, epoch, clock, radio
   fields) stays in InetNrState: the DL step reads it and never writes it. */
typedef struct InetNrDlState {
    int32_t *sent, *floor_, *last_tx;   /* [E][R] */
    float *olla, *avg;                  /* [E][R] */
    int32_t *enq, *qlen;                /* [E][R] */
    float *csi;                         /* [E][S][R] the gNB's estimate from the last CQI report (dB) */
    uint32_t *h_meta;                   /* [E][P][R] state (0 free, 1 undecoded, 2 decoded awaiting HARQ-ACK) | ... */
    int32_t *h_lo, *h_hi, *h_ready, *h_tbs;
    float *h_comb, *h_lexp, *h_nrb;
    int32_t *q_cap, *q_start, *q_end, *q_fin;   /* [E][F][R] */
    uint32_t *q_meta;                   /* [E][F][R] lost | cls << 8 */
    int32_t *newest;                    /* [E][R] capture step (engine clock, absolute) of the newest DL frame
                                           delivered in the last step, -1 if none (NRNet.dl_newest) */
    int64_t *ctr, *hist;                /* [E][INET_NR_NCTR], [E][3][max_tx + 1]: as InetNrState's, for the DL */
    int64_t *out_newest, *out_queue_len;        /* [E][R] step outputs dl_newest (env clock) and dl_queue_len */
    float *out_delay;                   /* [E][R][F] or NULL: per frame slot of the queue before compaction, the delivery
                                           time minus the capture step of a frame delivered in this step (fin - cap,
                                           control steps), NaN otherwise (the DL frames NRNet._log_dl records,
                                           nr_engine.py:906-907) */
    const float *cqi_thr;               /* [15] SINR from which CQI k + 1 is reported (cqi_table = "38214"), */
    const int32_t *cqi_mcs;             /* [16] MCS of each CQI; both NULL for cqi_table = "mcs" */
    int64_t *base;                      /* [E][R] the DL byte-stream base, as InetNrState.base for the UL */
    int32_t gnb_proc;                   /* gNB processing slots after the HARQ-ACK */
    int32_t snr_offset;                 /* 1: SNR input plus snr_off (dl_snr_offset_db); 0: the DL SNR as given */
    float ref_off, noise_prb, snr_off;  /* pose input: dl_ref = (pg + ref_off) - noise_prb (gNB PSD, UE noise) */
    int32_t pad;
} InetNrDlState;

/* The arrivals of one control step for inet_nr_submit_step: the counts form of inet_nr_submit. */
typedef struct InetNrArrivals {
    const uint8_t *counts;              /* [E][R][n_cls] messages per class, enqueued class by class (device) */
    const float *sizes;                 /* [n_cls] message bytes (device) */
    int32_t *accepted;                  /* [E][R] messages accepted, or NULL (device) */
    int32_t n_cls, discard_pdcp, pkt_payload, pkt_overhead;
} InetNrArrivals;

/* Several cells per env (NRConfig(n_cells > 1), NRNet.step_cells, nr_engine.py:718-788): the association of every
   robot (CellAssociation, radio.py:303-453, without radio link failure), each gNB's N+I estimate and the constants
   of association, A3 handover, power control and interference. */
typedef struct InetNrCells {
    int32_t *serv, *a3_cand, *a3_cnt, *ho_end, *n_ho;   /* [E][R] serving cell, A3 candidate / count, end slot of
                                                           the handover interruption, handovers */
    int32_t *pending;                   /* [E] 1: associate to the max-RSRP cell at the next step (after a reset) */
    float *ni_ul;                       /* [E][C][S] each gNB's N+I estimate per PRB (mW, EWMA of the measurements) */
    float *ion;                         /* [E] sum of interference over thermal over gNB-RBG-slots */
    float gnb_xy[2 * INET_NR_MAX_C];    /* gNB positions (x, y) */
    int32_t C;                          /* cells (must equal the params' n_cells) */
    int32_t ttt, ho_int;                /* A3 time-to-trigger and handover interruption, slots */
    int32_t ho_flush;                   /* 1: ho_rlc = "flush" (queued frames are dropped at a handover) */
    int32_t use_int;                    /* 1: same-slot UL interference (noise_model "thermal", ul_interference) */
    int32_t pc_on;                      /* 1: fractional UL power control */
    int32_t has_floor;                  /* 1: A3 target admission floor (a3_min_target_rsrp_dbm) */
    float a3_off, a3_hyst, floor_rx;    /* A3: best > (serving + a3_off) + a3_hyst; floor on the rx scale */
    float noise_mw;                     /* gNB noise per PRB (mW) */
    float ref_db;                       /* 10 log10(snr_ref_prbs) */
    float li_a, li_b;                   /* N+I EWMA: li_a * now + li_b * estimate (li_b = 0: the measurement) */
    float pc_p0, pc_alpha;              /* power control: backoff = ue_tx - (p0 + alpha (ue_tx - rx_serving)) */
    /* Radio link failure (cfg.rlf; CellAssociation, radio.py:456-531, NRNet._rlf_events / _rlf_links,
       nr_engine.py:684-707; ABI 15). Per robot [E][R]: in RLF, out-of-sync / in-sync counts, the slots at which
       T310, T311 and the re-establishment end (-1: not running), the re-establishment cell, RLFs since the reset.
       Once per step, at its first slot, before the A3 plan: T311 expiry (the robot goes idle: its queue is flushed),
       the cell search of the robots in RLF, the indications of the connected ones (serving SINR < qout:
       out-of-sync, > qin: in-sync) and T310 start (n310 out-of-sync in a row) / stop (n311 in-sync). At every
       scheduled slot and after the last one: T310 expiries (RLF: unschedulable, T311 starts, the search runs, the
       link's MAC restarts as at a handover, flushed with rlf_flush) unless a handover precedes them, then the
       re-establishments due (the robot attaches to the selected cell, the MAC restarts unflushed). A handover stops
       T310. The search takes the max-RSRP cell with SINR estimate >= qin (and RSRP above the floor when set); the
       re-establishment completes reest slots later. Counters [E][5] int64 (rlf, reest, rlf_idle, t310_start,
       t310_stop), cleared by a full reset only; out_rlf [E][R] uint8: in RLF after the step (the "rlf" output). */
    int32_t *rlf_active, *oos_cnt, *is_cnt, *t310_end, *t311_end, *reest_end, *reest_cell, *n_rlf;
    int64_t *rlf_ctr;
    uint8_t *out_rlf;
    int32_t rlf, rlf_flush, n310, n311, t310, t311, reest;
    float qout, qin;
    int32_t pad_r;
} InetNrCells;

/* Library version (INET_NR_ABI_VERSION) and a short build string. */
int32_t inet_nr_abi_version(void);
const char *inet_nr_build_info(void);

/* One control step T (the engine's global control-step counter; T < 0: *st->clock, read on the device) over
   rows[0..n_rows) (device buffer).
   x: poses [E][R][2] (input_kind 0), SNR [E][R] (1) or per-subband SNR [E][R][S] (2), float32, device.
   cur_hid: [E] int64 hazard ids for det_env (device). first_evolve_dt is folded into rows[0] by the host. */
int32_t inet_nr_step(const InetNrState *st, const InetNrTables *tab, const InetNrParams *prm, const InetNrRow *rows,
                     int32_t n_rows, int64_t T, const float *x, const int64_t *cur_hid, const InetNrOutputs *out,
                     void *stream);

/* inet_nr_submit (counts form, arr) and inet_nr_step of the same control step in one launch: every lane enqueues its
   robot's arrivals at the start of the step kernel (NRNet.add_frames, nr_engine.py:466-487, one message at a time in
   class order), then runs the step. Same results as the two calls. */
int32_t inet_nr_submit_step(const InetNrState *st, const InetNrTables *tab, const InetNrParams *prm,
                            const InetNrRow *rows, int32_t n_rows, int64_t T, const float *x, const int64_t *cur_hid,
                            const InetNrOutputs *out, const InetNrArrivals *arr, void *stream);

/* Enqueue at control step T (T < 0: *st->clock on the device). Single form (counts == NULL): send [E][R] int64 class index (0 = none), det [E][R]
   uint8 or NULL, hid [E] int64 or NULL; accepted [E][R] uint8. Counts form (send == NULL): counts [E][R][NC]
   uint8 messages per class, enqueued class by class; accepted [E][R] int32 = messages accepted.
   sizes [NC] float32 message bytes; discard_pdcp: 1 = refuse while the head frame is stale (timeout_steps). */
int32_t inet_nr_submit(const InetNrState *st, const InetNrParams *prm, int64_t T, const int64_t *send,
                       const uint8_t *det, const int64_t *hid, const uint8_t *counts, int32_t n_cls,
                       const float *sizes, int32_t discard_pdcp, int32_t pkt_payload, int32_t pkt_overhead,
                       void *accepted, void *stream);

/* Reset the envs of mask [E] uint8 (device; NULL = every env, full reset). T: control step of the reset (the
   epoch of the reset envs). k_lin0: Rician K (linear) of a reset link. dcorr[3]: correlation distances of the
   shadowing fields (tr38901: sf LOS, sf NLOS, LOS state; log_distance: shadow_dcorr_m), spectrum: 0 sos, 1 exp. */
int32_t inet_nr_reset(const InetNrState *st, const InetNrParams *prm, const uint8_t *mask, int64_t T, float k_lin0,
                      const float *dcorr, int32_t spectrum, void *stream);

/* The downlink part of control step T (NRNet.step / step_rx with dl=True, nr_engine.py:613-668: DlMac.cqi_report at
   the CQI rows, MacLink.slot with the DlMac hooks at the DL data rows, and the DL half of _finish, nr_engine.py:866-
   881). Launch it before inet_nr_step of the same step, on the same stream: both read the fading state and RNG words
   of the step start, which inet_nr_step then advances. rows: the DL rows of the step (flags 1 CQI report, 2 DL data,
   4 / 8 fading as for the UL rows, bits 8..23 the HARQ-ACK slot of the row relative to the step's first slot;
   salt_bler = salt((BLER_DL << 16) | rel)). tab: the PHY tables with the DL MCS cap. x: as inet_nr_step's (poses,
   SNR [E][R] or per-subband SNR [E][R][S]; with SNR, dl->snr_offset says whether dl_snr_offset_db is added).
   No counterpart launch in the reference's triton backend: there the DL runs inside its one fused kernel
   (nr_triton.py:938-989, the DL flag of _mac_slot). */
int32_t inet_nr_dl_step(const InetNrState *st, const InetNrDlState *dl, const InetNrTables *tab,
                        const InetNrParams *prm, const InetNrRow *rows, int32_t n_rows, int64_t T, const float *x,
                        void *stream);

/* Enqueue one DL frame per robot at control step T (T < 0: *st->clock): NRNet.add_dl_frames (nr_engine.py:489-497)
   with FrameQueue.add (queues.py:87-103). nbytes [E][R] float32 application bytes (0 = none), cls [E][R] int64 or
   NULL (the slot then keeps the class it held, as the reference's meta field); accepted [E][R] uint8. Frames of more
   than 2^22 bytes (after the packet overhead) are refused, which keeps a full queue inside the int32 offsets. */
int32_t inet_nr_dl_submit(const InetNrState *st, const InetNrDlState *dl, const InetNrParams *prm, int64_t T,
                          const float *nbytes, const int64_t *cls, int32_t discard_pdcp, int32_t pkt_payload,
                          int32_t pkt_overhead, uint8_t *accepted, void *stream);

/* Reset the DL link of the envs of mask [E] uint8 (NULL = every env, which also clears the DL counters):
   MacLink.reset / FrameQueue.reset of NRNet.dl and dl_newest (nr_engine.py:256-274). */
int32_t inet_nr_dl_reset(const InetNrDlState *dl, const InetNrParams *prm, const uint8_t *mask, void *stream);

/* One control step T with several cells (NRNet.step_cells, nr_engine.py:718-788, uplink): per robot the path gain to
   every cell from its pose (input_kind 0, x: poses [E][R][2]) or as given (input_kind 3, x: path gain [E][R][C] dB,
   step(pathgain_db=), engine.py:909-915: no radio, so no LOS state and no motion), the max-RSRP association of the envs flagged pending, the A3 plan of
   the step (the slot at which a handover fires); per scheduled slot the handovers due by that slot (CellAssociation
   switch, UlMac.handover: mac_ul.py:238-247, mac.py:557-581), AR(1) fading on every robot-cell link, one scheduler
   per cell over the same RBGs (mac.py:278-379 with member masks), the robots in a handover interruption left out,
   the UL reference against the serving gNB's N+I estimate, fractional power control (nr_engine.py:671-675,
   mac_ul.py:154-180) and the same-slot interference of the other cells' transmissions (_ul_ici, nr_engine.py:799-816);
   then the handovers due after the last slot and the end of step as inet_nr_step. sinr_db is the serving link's
   full-power SINR against the serving gNB's estimate (serving_sinr_db, nr_engine.py:709-713); serving_cell the
   serving cell. arr: this step's arrivals as inet_nr_submit_step, or NULL. Needs prm->n_cells == cells->C > 1,
   input_kind 0 or 3 and F <= 64. No counterpart in the reference's triton backend, which
   runs one cell (nr_fast.py:538-554 refuses n_cells > 1); the reference path is the eager NRNet.step_cells. */
int32_t inet_nr_step_cells(const InetNrState *st, const InetNrCells *cells, const InetNrTables *tab,
                           const InetNrParams *prm, const InetNrRow *rows, int32_t n_rows, int64_t T, const float *x,
                           const int64_t *cur_hid, const InetNrOutputs *out, const InetNrArrivals *arr, void *stream);

/* Reset the association and the N+I estimates of the envs of mask [E] uint8 (NULL = every env, which also clears
   the interference statistic): CellAssociation.reset and NRNet._reset_cells (radio.py:402-408,
   nr_engine.py:424-438). inet_nr_reset with prm->n_cells = C redraws the fading state of every link and the
   shadowing fields of every cell. */
int32_t inet_nr_cells_reset(const InetNrCells *cells, const InetNrParams *prm, const uint8_t *mask, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* INET_NR_H */

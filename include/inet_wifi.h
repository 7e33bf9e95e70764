/*
 * inet_wifi.h -- C ABI of the MI355X-native engine of isaac-net's level "WIFI" (libinet_nr.so, HIP kernels for
 * gfx950): the mean-field 802.11 uplink of a robot fleet at one access point.
 *
 * Drop-in boundary for the Wi-Fi level's hot path. The reference runs it as torch ops, captured in two CUDA graphs
 * (backend "graph") or eagerly (backend "reference"):
 *     step region    LevelNet._step_region (isaac_net/core/levels/base.py:301-316): WifiNet._serve
 *                    (isaac_net/core/wifi/engine.py:292-403: K sub-steps of meanfield.solve, wifi/meanfield.py:187-209,
 *                    poisson_icdf :57-63, serve_fifo proto/netsim.py:86-92, the retry-limit loss) and finish_body
 *                    (proto/netsim_fast.py:185-206), preceded by the eager association and radio
 *                    (WifiNet._snr_from, wifi/engine.py:227-259; RadioMC.rx_dbm, core/radio.py:238-272);
 *     enqueue region LevelNet._add_region (base.py:290-299): add_body (proto/netsim_fast.py:136-160);
 *     reset          LevelNet.reset (base.py:142-157), WifiNet._reset_rows (wifi/engine.py:179-186), RadioMC.reset
 *                    (radio.py:200-219).
 * This library replaces them with three entry points:
 *
 *   inet_wifi_step    one control step of every env: SNR from poses / SNR / received power, MCS, the K sub-steps
 *                     (mean-field fixed point, access counts, FIFO service, finish times, retry-limit loss), the end of
 *                     step (delivered, timed out, newest, det_env, stable compaction) and the step outputs.
 *   inet_wifi_submit  enqueue one message per robot (send form, one LevelNet.submit call) or several per robot in
 *                     class order (counts form, the harness's per-class calls in one launch).
 *   inet_wifi_reset   reset an env mask: FIFO, clock, mean-field state, counter-RNG episode, radio plane waves.
 *
 * Conventions (as inet_nr.h): the caller owns every device buffer; state is updated in place; nothing is allocated
 * and the host never waits; work goes on `stream`; every entry point returns 0 or a negative INET_WIFI_E* code,
 * checked before any launch. Layout: per-robot [E][R], per-frame state [E][F][R] (robot-minor), step outputs in the
 * reference's [E][R][F] layout and dtypes.
 */
#ifndef INET_WIFI_H
#define INET_WIFI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define INET_WIFI_ABI_VERSION 7
#define INET_WIFI_MAX_R 64        /* robots per env (one wavefront segment) */
#define INET_WIFI_MAX_F 64        /* frame buffer */
#define INET_WIFI_MAX_M 16        /* MCS table entries */
#define INET_WIFI_MAX_L 16        /* transmission attempts per frame (max_tx) */
#define INET_WIFI_MAX_CLS 16      /* message classes */
#define INET_WIFI_MAX_NACC 128    /* support of the Poisson access count */
#define INET_WIFI_MAX_KF 16       /* plane waves per shadowing field */
#define INET_WIFI_MAX_A 8
#define INET_WIFI_MAX_Z 6         /* AIFS zones (AIFSN 2 .. 7) */         /* access points per env (on one channel: one collision domain) */

#define INET_WIFI_OK 0
#define INET_WIFI_EINVAL (-1)
#define INET_WIFI_EUNSUPPORTED (-2)
#define INET_WIFI_ELAUNCH (-3)

/* Per-env engine state (device pointers). */
typedef struct InetWifiState {
    /* frames [E][F][R]: capture step (-1 = empty slot), class, det flag, hazard id, bytes left, and the features
       recorded at enqueue (robots with a queued frame in the env, SNR of the last step, frames queued before) */
    int32_t *cap, *cls;
    uint8_t *det;
    int32_t *hid;
    float *rem;
    int32_t *f_nact;
    float *f_snr;
    int32_t *f_own;
    /* per robot [E][R]: frames queued (the valid prefix of the FIFO), SNR of the last step, roaming interruption
       (sub-steps), serving AP, the backlogged period's contending sub-steps and log failure sum, renewal credit */
    int32_t *qlen;
    float *last_snr;
    int32_t *roam_left, *serv;
    float *att_n, *att_logp, *credit;
    /* mean-field attempt probability [E][R + A]: the robots, then one background station per AP */
    float *tau;
    /* per env [E]: clock, hazard id of the last submit, association pending, counter-RNG key and call counters */
    int64_t *clock, *last_hid;
    uint8_t *pending;
    int32_t *env_id, *episode, *ctr_step, *ctr_submit;
    /* radio plane waves [E][A][n_fields][n_modes][3] = (kx, ky, phase), one set per AP */
    float *field;
    /* [1]: the counts form's global submit calls (each advances every env's SUBMIT counter alike): env e's counter
       is ctr_submit[e] + calls[0]; a reset sets ctr_submit[e] = -calls[0] */
    int32_t *calls;
} InetWifiState;

/* Config constants (derived on the host from NRConfig + WifiConfig; float32 values of the reference's tensors). */
typedef struct InetWifiParams {
    int32_t E, R, F, K, M, L;        /* envs, robots, frame buffer, sub-steps, MCS entries, max_tx */
    int32_t n_cls, n_acc_max, fp_iters, timeout;
    int32_t access_noise;            /* 0 poisson, 1 mean */
    int32_t rts_cts, coll_ack, per_class_ac, no_aggr;
    int32_t radio_model, n_fields, n_modes, seed_key, roam_sub, bg_ac, envs_per_wave, spectrum, pad0;
    float noise_dbm, roam_hyst, damp, fer1, dt_us, tau0, slot_us, sifs_us;
    float pre, tsym, ovh1, t_ack, t_rts, t_cts, hs, ampdu_lim, msdu_payload, ppdu_max, bg_w, bg_rate, bg_B;
    float dcorr[3];
    float rates[INET_WIFI_MAX_M], thr[INET_WIFI_MAX_M];
    int32_t mcs_ids[INET_WIFI_MAX_M];
    float ac_W0[5], ac_Wmax[5], ac_aifsn[5], ac_txop[5];
    int32_t cls_ac[INET_WIFI_MAX_CLS + 1];
    float sizes[INET_WIFI_MAX_CLS];
    float lgamma[INET_WIFI_MAX_NACC];   /* lgamma(k + 1) of the reference's float32 torch.lgamma */
    /* radio of the AP (same meaning as in InetNrParams) */
    float gnb_x, gnb_y, hh2, dbp, pl_a, pl_n1, pl_c20, pl_c2, nl_b1, nl_b0, nl_c, nl_d, sig, amp, pl_const, pl_exp10,
          ue_tx;
    int32_t los_sto;                 /* TR 38.901 stochastic LOS state of every robot-AP link (as InetNrParams) */
    int32_t plos_scn;                /* los_sto: the Pr_LOS formula, 0 UMi, 1 UMa (h_UT <= 13 m), 2 InH */
    float sig_nlos;                  /* los_sto: NLOS shadow-fading sigma (dB); sig is the LOS one */
    int32_t A;                       /* access points (1 .. INET_WIFI_MAX_A), all on one channel: the robots associate to
                                        the strongest after a reset and roam to an AP stronger by roam_hyst dB, with
                                        roam_sub sub-steps without channel access (wifi/engine.py:245-257) */
    const float *los_cdf;            /* los_sto: [65536] sorted samples of a unit sum of cosines */
    float ap_xy[2 * INET_WIFI_MAX_A]; /* AP positions (x, y); gnb_x, gnb_y repeat AP 0 */
    /* The control step's enqueue in the step launch (inet_wifi_step, inet_wifi_dcf_step; NULL elsewhere): with
       step_counts set, the step first enqueues step_counts [E][R][step_n_cls] uint8 (device) exactly as
       inet_wifi_submit's counts form does (the same FIFO entries, submit counters and last hazard ids) and writes the
       messages accepted per robot to step_accepted [E][R] int32 (device, or NULL). One launch in place of three. */
    const uint8_t *step_counts;
    int32_t *step_accepted;
    int32_t step_n_cls;
    /* APs on several channels (wifi/engine.py:117-166, 300-305): n_dom collision domains, one per distinct channel,
       and each AP's domain (the index of its channel among the sorted distinct channels). A robot contends in its
       serving AP's domain, an AP's background station in the AP's. n_dom = 1: one domain. n_dom > 1 needs
       R + A <= 64 and (R + A) n_dom < 400 (else INET_WIFI_EUNSUPPORTED). */
    int32_t n_dom;
    int32_t ap_dom[INET_WIFI_MAX_A];
    /* AIFS zones (wifi/meanfield.py:106-209, wifi/engine.py:344-348): 1 + the largest AIFSN difference among the
       access categories in use (robots' and background stations'), 1 .. INET_WIFI_MAX_Z. Z > 1: each station's
       offset from the smallest AIFSN among the contending stations of its domain, per-zone sums and the stationary
       zone distribution; needs R + A <= 64 (else INET_WIFI_EUNSUPPORTED); level WIFI_DCF needs Z = 1. */
    int32_t Z;
    /* Hidden nodes (wifi/engine.py:260-282, wifi/meanfield.py:92-103, 161-178): each station senses the stations of
       its domain, and a robot the robots whose power at it reaches cca_dbm (sta_c0 - sta_c1 log10(max(d, 1 m)):
       sta_c0 = sta_tx_dbm - PL(1 m), sta_c1 = 10 n as float32; or sense[E][R][R] uint8, robot i senses robot j,
       device, per call; or every robot with an SNR or received-power input). An unsensed robot of the domain whose
       power at the robot's AP reaches cca_dbm is hidden; the failure probability gains the hidden-collision term.
       Needs (R + A)^2 < 400 (else INET_WIFI_EUNSUPPORTED); level WIFI_DCF refuses it. */
    int32_t hidden;
    float cca_dbm, sta_c0, sta_c1;
    const uint8_t *sense;
} InetWifiParams;

/* Step outputs, the reference's keys, layouts and dtypes (bool as uint8). */
typedef struct InetWifiOutputs {
    uint8_t *delivered, *timed_out;                      /* [E][R][F] */
    int64_t *cap, *cls;                                  /* [E][R][F] */
    float *delay;                                        /* [E][R][F] */
    int64_t *newest, *queue_len, *serving_cell, *mcs;    /* [E][R] */
    float *queue_bytes, *sinr_db, *rate_mbps, *access_ms, *p_fail, *busy;   /* [E][R] */
    uint8_t *det_env;                                    /* [E] */
    int64_t *t;                                          /* [E] */
} InetWifiOutputs;

/* Level WIFI_DCF (this build's per-slot CSMA/CA access with integer backoff counters, following the semantics of
   the reference's validation simulator isaac_net/core/wifi/eventsim.py:56-186, behind the same LevelNet API):
   the per-station counter state and the per-env end of the last busy period. */
typedef struct InetDcfState {
    int32_t *b;          /* [E][R] backoff counter (slots) */
    int32_t *stage;      /* [E][R] retry stage of the current access */
    uint8_t *had;        /* [E][R] contending (bytes queued, usable MCS) at the end of the last step */
    int32_t *t_idle;     /* [E] end of the last busy period, ns relative to the start of the next step (<= 0) */
} InetDcfState;

/* Integer timing of the DCF level (ns) and its EDCA set. */
typedef struct InetDcfParams {
    int32_t ndbps[INET_WIFI_MAX_M];   /* data bits per OFDM symbol of each MCS entry */
    int32_t T;                        /* control step, ns (<= 2^30) */
    int32_t tsym, pre, sifs, slot, t_ack, t_rts, t_cts;
    int32_t W0, Wmax, aifsn;          /* CWmin + 1, CWmax + 1, AIFSN of the access category */
    int32_t ovh, payload;             /* per-MSDU overhead bytes and MSDU payload bytes */
    float fer;                        /* residual frame error rate (float32) */
} InetDcfParams;

int32_t inet_wifi_abi_version(void);

/* One control step. t: [E] int64 step of each env (device) or NULL for st->clock. input_kind: 0 poses [E][R][2],
   1 SNR [E][R] dB, 2 received power [E][R][A] dBm (float32, device). cur_hid: [E] int64 or NULL for st->last_hid.
   Replaces the step region of LevelNet.step (levels/base.py:252-316) with WifiNet._snr_from / _serve
   (wifi/engine.py:227-403), and with prm->step_counts set also the enqueue region before it (the harness's
   per-class LevelNet.submit calls, base.py:290-299): the env's own FIFO entries in the env's wavefront (a call
   changes nothing of an env in which no robot sends), the global call count in one extra workgroup. */
int32_t inet_wifi_step(const InetWifiState *st, const InetWifiParams *prm, const int64_t *t, int32_t input_kind,
                       const float *x, const int64_t *cur_hid, const InetWifiOutputs *out, void *stream);

/* Enqueue (LevelNet.submit / add_body, levels/base.py:223-246, proto/netsim_fast.py:136-160). t: [E] or NULL
   (clock). snr: [E][R] float32 SNR recorded with the frames, or NULL for st->last_snr. Send form (counts == NULL):
   send [E][R] int64 class (0 = none; classes above n_cls take the last class's size), det [E][R] uint8 or NULL,
   hid [E] int64 or NULL; accepted [E][R] uint8. Counts form (send == NULL): counts [E][R][n_cls] uint8, the calls of
   class 1 first, one call per message index up to the class's largest count over every env (a call is global, as
   LevelNet.submit is); accepted [E][R] int32 = messages accepted; every env's submit counter advances by the number
   of calls (st->calls[0]) and its last hazard id becomes 0 (a second, one-workgroup launch reduces the counts). */
int32_t inet_wifi_submit(const InetWifiState *st, const InetWifiParams *prm, const int64_t *t, const int64_t *send,
                         const uint8_t *det, const int64_t *hid, const float *snr, const uint8_t *counts,
                         int32_t n_cls, void *accepted, void *stream);

/* Reset the envs of mask [E] uint8 (device; NULL = every env) (LevelNet.reset, levels/base.py:142-157). */
int32_t inet_wifi_reset(const InetWifiState *st, const InetWifiParams *prm, const uint8_t *mask, void *stream);

/* Level WIFI_DCF: one control step with the per-slot CSMA/CA access in place of the mean-field sub-steps (same
   arguments and outputs as inet_wifi_step; wifi_access_ms, wifi_p_fail and wifi_busy are the step's measured access
   time, failure share and busy share). No counterpart in the reference's engines: its integer-backoff semantics
   exist only in the validation simulator (wifi/eventsim.py:56-186). Refused (INET_WIFI_EUNSUPPORTED): per-class
   access categories and background stations; refused (INET_WIFI_EINVAL): message sizes above 2^24 bytes, T above
   2^30 ns, non-positive symbol, slot, RTS or CTS times. */
int32_t inet_wifi_dcf_step(const InetWifiState *st, const InetDcfState *ds, const InetWifiParams *prm,
                           const InetDcfParams *dp, const int64_t *t, int32_t input_kind, const float *x,
                           const int64_t *cur_hid, const InetWifiOutputs *out, void *stream);

/* Level WIFI_DCF reset: inet_wifi_reset plus the initial backoff counters of the new episode. */
int32_t inet_wifi_dcf_reset(const InetWifiState *st, const InetDcfState *ds, const InetWifiParams *prm,
                            const InetDcfParams *dp, const uint8_t *mask, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* INET_WIFI_H */

// MI355X (gfx950) kernels of isaac-net's per-control-step NR uplink engine, behind the C ABI of include/inet_nr.h.
//
// nr_step_kernel<S, P> runs one whole control step per env: the radio prologue (TR 38.901 / log-distance path gain
// of the pose, isaac_net/core/radio.py:238-277), every scheduled slot of the step (AR(1) Rician / Rayleigh fading,
// nr_engine.py:570-611; SR opportunities, mac_ul.py:66-71; UL data slots, mac.py:228-508 with the UlMac hooks of
// mac_ul.py:140-236) and the end of step (nr_engine.py:843-888, mac.py:585-616, queues.py:105-110), reading and
// writing HBM once per step.
//
// Work decomposition: one robot per lane; the RB = next_pow2(R) lanes of an env form one aligned segment of a
// 64-lane wavefront, so a wavefront carries 64 / RB envs and every cross-robot step of the scheduler (retransmission
// admission, RBG-by-RBG argmax, lexicographic masking) is a segment butterfly or a ballot, with no LDS and no
// barrier. Per-robot state (HARQ processes, subband CSI and fading, MAC scalars) stays in VGPRs across the slots;
// the frame FIFO is touched only in the epilogue, which replays the per-slot in-order pointer (recorded in
// registers) over the queued frames, so the slot loop never reads the queue.
//
// Float arithmetic follows the reference's torch op order (no contraction, ATen reduction order) so that only the
// transcendental functions (logf, expf, powf, log10f, cosf) differ from the CPU path by rounding.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/inet_nr.h"
#include "inet_nr_dev.h"

using namespace inet;

namespace {

constexpr int BLOCK = 256;
constexpr uint32_t CH_STEP = 2, CH_RESET = 3;
constexpr uint32_t SITE_H0 = 4, SITE_KPHI = 6;
constexpr uint32_t LOG_DISTANCE_STREAM = 10;
constexpr uint32_t TR38901_STREAM = (0x52u << 16) + 16u;
constexpr int MAX_ROWS_UL = 64;   // UL data slots per control step whose in-order pointer the epilogue replays

DEV int hm_state(uint32_t m) { return (int)(m & 0xffu); }
DEV int hm_ntx(uint32_t m) { return (int)((m >> 8) & 0xffu); }
DEV int hm_mcs(uint32_t m) { return (int)((m >> 16) & 0xffu); }
DEV int hm_nsb(uint32_t m) { return (int)((m >> 24) & 0xffu); }
DEV uint32_t hm_pack(int st, int ntx, int mcs, int nsb) {
    return (uint32_t)st | ((uint32_t)ntx << 8) | ((uint32_t)mcs << 16) | ((uint32_t)nsb << 24);
}

// runtime-length ATen row sum for the shadowing modes (n <= 16)
DEV float aten_sum_rt(const float* x, int n) {
    if (n >= 8) {
        float lane[8];
        for (int l = 0; l < 8; ++l) lane[l] = x[l];
        float fin = 0.f;
        for (int k = 8; k < n; ++k) fin += x[k];
        for (int l = 0; l < 8; ++l) fin += lane[l];
        return fin;
    }
    float q[4] = {0.f, 0.f, 0.f, 0.f};
    int si = n / 4;
    for (int i = 0; i < si; ++i)
        for (int k = 0; k < 4; ++k) q[k] += x[i * 4 + k];
    for (int i = si * 4; i < n; ++i) q[0] += x[i];
    return ((q[0] + q[1]) + q[2]) + q[3];
}

// Bilinear BLER at (table row base, SINR dB) with the code-block interpolation weight wi (phy.bler_lookup)
DEV float bler_at(const float* __restrict__ tab, int base0, int G, float s0, float ds, float sinr, float wi) {
    float xs = sinr != sinr ? -30.0f : sinr;
    float xg = clampf((xs - s0) / ds, 0.0f, (float)(G - 1));
    float j0f = clamp_max(floorf(xg), (float)(G - 2));
    int j0 = (int)j0f;
    float wj = xg - j0f;
    const float* p = tab + base0 + j0;
    float lo = p[0] * (1.0f - wj) + p[1] * wj;
    float hi = p[G] * (1.0f - wj) + p[G + 1] * wj;
    return lo * (1.0f - wi) + hi * wi;
}

// code-block segmentation (phy.segment) of TBS tbs at code rate r (float32 rate, float64 math) -> (cbs f32, ncb f32)
DEV void segment_f(int tbs, float r32, float& cbs, float& ncb) {
    double t = (double)tbs, r = (double)r32;
    bool bg2 = (t <= 292.0) || ((t <= 3824.0) && (r <= 0.67)) || (r <= 0.25);
    double kcb = bg2 ? 3840.0 : 8448.0;
    double b = t + (t > 3824.0 ? 24.0 : 16.0);
    double c = b <= kcb ? 1.0 : ceil(b / (kcb - 24.0));
    double bp = c > 1.0 ? b + 24.0 * c : b;
    cbs = (float)(bp / c);
    ncb = (float)c;
}

}  // namespace

// ======================================================================================= step kernel
template <int S, int P>
__global__ __launch_bounds__(BLOCK) void nr_step_kernel(InetNrState st, InetNrTables tb, InetNrParams pm,
                                                        const InetNrRow* __restrict__ rows, int n_rows, int64_t T,
                                                        const float* __restrict__ xin,
                                                        const int64_t* __restrict__ cur_hid, InetNrOutputs out,
                                                        int rb) {
    const int lane = threadIdx.x & 63;
    const int envs_pb = BLOCK / rb;
    const int e = blockIdx.x * envs_pb + (int)threadIdx.x / rb;
    const int r = (int)threadIdx.x & (rb - 1);
    const int R = pm.R, E = pm.E, F = pm.F, N = pm.N;
    if (blockIdx.x * envs_pb + ((int)threadIdx.x & ~63) / rb >= E) return;     // the whole wavefront is idle
    const bool act = (e < E) && (r < R);
    const int ee = e < E ? e : E - 1;
    const size_t ir = (size_t)ee * R + (r < R ? r : 0);
    const float* __restrict__ w = tb.w;

    // ---------------- load per-robot state ----------------
    int sent = 0, floor_ = 0, bsr = 0, sr_t = -1, last_tx = -1, enq = 0, qlen = 0;
    float olla = 0.f, avg = 100.f;
    float csi[S], hr[S], hi[S], ref[S];
    uint32_t hmeta[P];
    int hlo[P], hhi[P], hrdy[P], htbs[P];
    float hcomb[P], hlexp[P], hnrb[P];
    const bool ir_comb = pm.comb == 2;
    bool read_h = pm.fading && !(n_rows > 0 && (rows[0].flags & 4) && rows[0].rho == 0.0f);
    if (act) {
        sent = st.sent[ir]; floor_ = st.floor_[ir]; bsr = st.bsr[ir]; sr_t = st.sr_t[ir];
        last_tx = st.last_tx[ir]; enq = st.enq[ir]; qlen = st.qlen[ir]; olla = st.olla[ir]; avg = st.avg[ir];
        qlen = qlen < 0 ? 0 : (qlen > F ? F : qlen);
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
        size_t is = ((size_t)ee * S + s) * R + r;
        csi[s] = act ? st.csi[is] : 0.f;
        hr[s] = (act && read_h) ? st.h_re[is] : 0.f;
        hi[s] = (act && read_h) ? st.h_im[is] : 0.f;
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
        size_t ip = ((size_t)ee * P + p) * R + r;
        hmeta[p] = act ? st.h_meta[ip] : 0u;
        hlo[p] = act ? st.h_lo[ip] : 0;
        hhi[p] = act ? st.h_hi[ip] : 0;
        hrdy[p] = act ? st.h_ready[ip] : 0;
        htbs[p] = act ? st.h_tbs[ip] : 0;
        hcomb[p] = act ? st.h_comb[ip] : 0.f;
        hlexp[p] = (act && ir_comb) ? st.h_lexp[ip] : -INFINITY;
        hnrb[p] = (act && ir_comb) ? st.h_nrb[ip] : 0.f;
    }
    float sp_re = 0.f, sp_im = 0.f, kk = 0.f;
    if (pm.rician && act) { sp_re = st.spec_re[ir]; sp_im = st.spec_im[ir]; kk = st.k_lin[ir]; }
    // rician gain coefficients (nr_engine.py:608-611): inv = 1 / (K + 1), sqrt(K inv), sqrt(inv)
    const float kinv = 1.0f / (kk + 1.0f);
    const float ka = sqrtf(kk * kinv), kb = sqrtf(kinv);

    // ---------------- inputs: SINR reference per subband and the reported SNR ----------------
    float snr_out = 0.f;
    if (pm.input_kind == 0) {                      // poses -> path gain (radio prologue)
        float px = 0.f, py = 0.f;
        if (act) { px = xin[ir * 2]; py = xin[ir * 2 + 1]; }
        float dx = px - pm.gnb_x, dy = py - pm.gnb_y;
        float d2 = clamp_min(sqrtf(dx * dx + dy * dy), 1.0f);
        // once per robot and step: the transcendental functions of the radio are evaluated in double precision and
        // rounded once (correctly rounded float results; the field arguments k . x reach 1e4 rad)
        int fi = 0;
        float pl;
        if (pm.radio_model == 1) {                 // TR 38.901 (tr38901.py:162-203), deterministic LOS state
            float d3 = sqrtf(d2 * d2 + pm.hh2);
            float lg = (float)log10((double)d3);
            float pl1 = (pm.pl_a + pm.pl_n1 * lg) + pm.pl_c20;
            float pl2 = ((pm.pl_a + 40.0f * lg) + pm.pl_c20) - pm.pl_c2;
            pl = d2 <= pm.dbp ? pl1 : pl2;
            if (pm.nl_b1 != 0.0f) {                // NLOS: max(PL_LOS, PL'_NLOS)
                float pn = ((pm.nl_b1 * lg + pm.nl_b0) + pm.nl_c) - pm.nl_d;
                pl = pn > pl ? pn : pl;
                fi = 1;
            }
        } else {
            pl = pm.pl_const + pm.pl_exp10 * (float)log10((double)d2);
        }
        const float* fld = st.field + ((size_t)ee * pm.n_fields + fi) * pm.n_modes * 3;
        float cs[INET_NR_MAX_KF];
        for (int k = 0; k < pm.n_modes; ++k) {
            float arg = (px * fld[k * 3 + 0] + py * fld[k * 3 + 1]) + fld[k * 3 + 2];
            cs[k] = (float)cos((double)arg);
        }
        float field = pm.amp * aten_sum_rt(cs, pm.n_modes);
        float pg;
        if (pm.radio_model == 1) {
            float loss = pl + pm.sig * field;
            pg = (pm.ue_tx + (-loss)) - pm.ue_tx;
        } else {
            pg = ((pm.ue_tx - pl) - field) - pm.ue_tx;
        }
        float ru = (pg + pm.ref_off) - pm.noise_prb;
#pragma unroll
        for (int s = 0; s < S; ++s) ref[s] = ru;
        snr_out = (pg + pm.ue_tx) - pm.subband_noise;
    } else if (pm.input_kind == 1) {
        float v = act ? xin[ir] : 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) ref[s] = v;
        snr_out = v;
    } else {
#pragma unroll
        for (int s = 0; s < S; ++s) ref[s] = act ? xin[ir * S + s] : 0.f;
        snr_out = aten_sum<S>(ref) / (float)S;
    }
    // PHR cap n_max (mac_ul.py:165-168): ref.mean(-1) -> snr_ref_prbs 10^((ref - phr_min) / 10) / w0
    int n_max = S;
    if (pm.phr_cap) {
        float mref = aten_sum<S>(ref) / (float)S;
        float nmp = pm.snr_ref_prbs * from_db(mref - pm.phr_min);
        float f = floorf(nmp / pm.w0);
        f = clampf(f, 1.0f, (float)S);
        n_max = (int)f;
    }

    // ---------------- counter RNG key of this env and step ----------------
    uint32_t base0 = 0;
    if (e < E) {
        uint32_t h = mix32((uint32_t)pm.seed_key ^ salt32((uint32_t)st.env_id[e]));
        h = mix32(h ^ salt32((uint32_t)st.episode[e]));
        h = mix32(h ^ salt32(CH_STEP));
        base0 = mix32(h ^ salt32((uint32_t)st.ctr_step[e]));
    }

    // per-env counters (summed over the segment at the end)
    int c_new = 0, c_retx = 0, c_ok = 0, c_fail = 0, c_exh = 0, c_new_pend = 0;
    int64_t c_bytes_ok = 0, c_bytes_new = 0, c_prb = 0;
    const int HB = pm.max_tx + 1;
    int h_ok[INET_NR_MAX_P + 1], h_tx[INET_NR_MAX_P + 1], h_fl[INET_NR_MAX_P + 1];
    for (int k = 0; k <= INET_NR_MAX_P; ++k) { h_ok[k] = 0; h_tx[k] = 0; h_fl[k] = 0; }

    // in-order pointer after every UL slot, and (RLC UM) the byte range of a TB that exhausted its HARQ
    int ack_hist[MAX_ROWS_UL];
    int exh_lo[MAX_ROWS_UL], exh_hi[MAX_ROWS_UL];
    int n_ul = 0;
    auto ack_ptr = [&]() {
        int a = sent;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            bool own = hm_state(hmeta[p]) == 1 && hhi[p] > floor_;
            int lo = hlo[p] > floor_ ? hlo[p] : floor_;
            if (own && lo < a) a = lo;
        }
        return a;
    };

    const int g0 = (int)(T * (int64_t)N);
    // ================================================================ slot loop
    for (int k = 0; k < n_rows; ++k) {
        const InetNrRow row = rows[k];
        const int g = g0 + row.rel;
        const bool need_h = (row.flags & 8) != 0;
        if ((row.flags & 4) && need_h) {           // AR(1) fading innovation of this slot (nr_engine.py:575-589)
            const uint32_t bf = mix32(base0 ^ row.salt_fade);
#pragma unroll
            for (int s = 0; s < S; ++s) {
                uint32_t j = (uint32_t)((r * S + s) * 2);
                float zr = normal_at(bf, j), zi = normal_at(bf, j + 1u);
                hr[s] = row.rho * hr[s] + (row.c1 * zr) / (float)1.4142135623730951;
                hi[s] = row.rho * hi[s] + (row.c1 * zi) / (float)1.4142135623730951;
            }
        }
        if (row.flags & 1) {                       // SR opportunity (UlMac.sr_step, lumped)
            if ((enq - sent) > 0 && bsr <= 0 && sr_t < 0) sr_t = g;
        }
        if (!(row.flags & 2)) continue;
        // ============================ UL data slot (MacLink.slot) ============================
        float gain[S];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (!pm.fading) { gain[s] = 0.f; continue; }
            float p;
            if (pm.rician) {
                float xr = ka * sp_re + kb * hr[s];
                float xi = ka * sp_im + kb * hi[s];
                p = xr * xr + xi * xi;
            } else {
                p = hr[s] * hr[s] + hi[s] * hi[s];
            }
            gain[s] = 10.0f * log10f(clamp_min(p, 1e-6f));
        }
        const int unsent = enq - sent;
        // grants (UlMac._pre_slot_lumped)
        if (row.flags & 16) bsr = bsr > 1 ? bsr : 1;
        if (sr_t >= 0 && g - sr_t >= pm.sr_delay) { bsr = bsr > 1 ? bsr : 1; sr_t = -1; }
        // candidates
        int rx_p = 0, p_new = 0;
        int best_rdy = 0x7fffffff;
        bool has_rx = false, any_free = false, pending = false;
#pragma unroll
        for (int p = P - 1; p >= 0; --p) {
            int stp = hm_state(hmeta[p]);
            if (stp == 1 && hrdy[p] <= g && hrdy[p] <= best_rdy) { best_rdy = hrdy[p]; rx_p = p; has_rx = true; }
            if (stp == 0) { any_free = true; p_new = p; }
            if (stp == 1) pending = true;
        }
        const int need = bsr < unsent ? bsr : unsent;
        bool new_el = any_free && need > 0 && !has_rx && act;
        has_rx = has_rx && act;
        const int rx_nsb = hm_nsb(hmeta[rx_p]);
        // scheduler estimate, OLLA, rate and metric per RBG (mac_ul.py:154-171, mac.py:256-275)
        float rate[S], metric[S];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            float est = (ref[s] - tb.wdb[s]) + csi[s];
            float eo = pm.olla ? est + olla : est;
            int mi = 0;
            if (tb.thr_monotone) {
                int lo = 0, hi_ = tb.mcs_max;            // highest m <= mcs_max with eo >= thr[m]
                if (!(eo >= tb.thr_ref[0])) { mi = 0; }
                else {
                    while (lo < hi_) { int mid = (lo + hi_ + 1) >> 1; if (eo >= tb.thr_ref[mid]) lo = mid; else hi_ = mid - 1; }
                    mi = lo;
                }
            } else {
                for (int m = 0; m <= tb.mcs_max; ++m) if (eo >= tb.thr_ref[m]) mi = m;
            }
            rate[s] = ((tb.se[mi] * row.re_prb) * w[s]) / 8.0f;
            if (pm.sched == 0) metric[s] = rate[s] / clamp_min(avg, 1e-9f);
            else if (pm.sched == 1) metric[s] = rate[s];
            else metric[s] = (float)(g - last_tx);
        }
        // retransmission admission (mac.py:300-304): rank by the metric sum, admit while the RBG counts fit
        if (seg_any(has_rx, rb, lane)) {
            int val = has_rx ? rx_nsb : 0;
            int tot = seg_sum_i(val, rb);
            if (tot > S) {
                float rkey = has_rx ? aten_sum<S>(metric) : -1.0f;
                int cum = 0;
                const int sb = lane & ~(rb - 1);
                for (int j = 0; j < rb; ++j) {
                    float kj = __shfl(rkey, sb + j, 64);
                    int vj = __shfl(val, sb + j, 64);
                    bool before = (kj > rkey) || (kj == rkey && j <= r);
                    cum += before ? vj : 0;
                }
                has_rx = has_rx && cum <= S;
            }
        }
        const int want_cnt = has_rx ? rx_nsb : (new_el ? n_max : 0);
        const float prio = pm.retx_prio ? (has_rx ? 1e9f : 0.0f) : 0.0f;
        // RBG-by-RBG allocation (mac.py:322-352)
        int cnt = 0;
        float left = (float)need;
        uint32_t won = 0;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            bool want = (cnt < want_cnt) && (has_rx || left > 0.0f);
            float m = want ? metric[s] + prio : -1.0f;
            if (pm.retx_prio) {
                bool wr = want && has_rx;
                if (seg_any(wr, rb, lane) && !wr) m = -1.0f;
            }
            float bv = m;
            int bi = r;
            seg_argmax(bv, bi, rb);
            bool sel = (bi == r) && bv >= 0.0f;
            if (sel) { won |= 1u << s; ++cnt; }
            left = left - ((sel && !has_rx) ? rate[s] : 0.0f);
        }
        if (!pm.retx_prio) {                          // release short retransmissions (mac.py:353-379)
            bool short_ = has_rx && (__popc(won) != rx_nsb);
            uint32_t rel_rs = short_ ? won : 0u;
            if (short_) won = 0u;
            cnt = __popc(won);
#pragma unroll
            for (int s = 0; s < S; ++s) {
                bool avs = seg_any((rel_rs >> s) & 1u, rb, lane);
                bool want = (cnt < want_cnt) && new_el && (left > 0.0f);
                float m = want ? metric[s] : -1.0f;
                float bv = m;
                int bi = r;
                seg_argmax(bv, bi, rb);
                bool sel = (bi == r) && bv >= 0.0f && avs;
                if (sel) { won |= 1u << s; ++cnt; }
                left = left - (sel ? rate[s] : 0.0f);
            }
        }
        const int n_sb = __popc(won);
        float n_prb = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) n_prb += ((won >> s) & 1u) ? w[s] : 0.0f;
        const bool tx_rx = has_rx && n_sb == rx_nsb && n_sb > 0;
        const bool tx_new = new_el && n_sb > 0;
        const bool tx = tx_rx || tx_new;
        // power split (mac_ul.py:173-180) and the per-subband estimate of link adaptation / decoding
        const float sp = 10.0f * log10f(clamp_min(n_prb / pm.snr_ref_prbs, 1e-3f));
        float lw[S];
#pragma unroll
        for (int s = 0; s < S; ++s) lw[s] = ((won >> s) & 1u) ? tb.logw[s] : -INFINITY;
        const float lnw = aten_lse<S>(lw);
        // ---- link adaptation for new TBs (phy.select_mcs): the highest MCS meeting the BLER target ----
        int mcs_new = 0, tbs_new = 0;
        if (__ballot(tx_new) != 0ull) {
            float lin[S];
#pragma unroll
            for (int s = 0; s < S; ++s) lin[s] = from_db(clampf((ref[s] - sp) + csi[s], -30.0f, 60.0f));
            float eff_md = 0.f;
            if (!pm.eesm) {                               // mean_db: PRB-weighted mean of the dB values
                float v[S];
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    float t = ((ref[s] - sp) + csi[s]) * expf(lw[s] - lnw);
                    v[s] = nan_to_num(t, 0.0f, 3.4028234663852886e38f, -3.4028234663852886e38f);
                }
                eff_md = aten_sum<S>(v);
            }
            const int np = (int)n_prb;
            const int toff = (row.nsym_idx * (tb.NPRB + 1) + np) * tb.M;
            bool found = false;
            if (tx_new) {
                for (int m = tb.mcs_max; m >= 0 && !found; --m) {
                    int tbs_m = tb.la_tbs[toff + m];
                    if (tbs_m <= 0) continue;
                    float eff;
                    if (pm.eesm) {
                        const float beta = tb.beta[m];
                        float xv[S];
#pragma unroll
                        for (int s = 0; s < S; ++s) xv[s] = (-lin[s]) / beta + lw[s];
                        eff = db_of((-beta) * (aten_lse<S>(xv) - lnw));
                    } else {
                        eff = eff_md;
                    }
                    eff = eff + (pm.olla ? olla : 0.0f);
                    const int base0m = (m * tb.C + tb.la_ci0[toff + m]) * tb.G;
                    float b = bler_at(tb.bler, base0m, tb.G, tb.s0, tb.ds, eff, tb.la_cwi[toff + m]);
                    float tbler = 1.0f - powf(1.0f - b, tb.la_ncb[toff + m]);
                    if (tbler <= pm.target) { mcs_new = m; tbs_new = tbs_m; found = true; }
                }
                if (!found) { mcs_new = 0; tbs_new = tb.la_tbs[toff]; }
            }
        }
        int cap_b = tbs_new / 8 - pm.tb_oh;
        cap_b = cap_b > 1 ? cap_b : 1;
        const int byt_new = cap_b < unsent ? cap_b : unsent;
        // ---- bind TBs to HARQ processes (mac.py:407-426) ----
        const int p_tx = tx_rx ? rx_p : p_new;
        int mcs = 0, tbs = 0, ntx = 1, lo_tx = 0, hi_tx = 0;
        float comb_p = 0.f, lexp_p = -INFINITY, nrb_p = 0.f;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (p == p_tx) {
                if (tx_new) {
                    hlo[p] = sent; hhi[p] = sent + byt_new; htbs[p] = tbs_new;
                    hmeta[p] = hm_pack(1, 0, mcs_new, n_sb);
                    hcomb[p] = 0.f; hlexp[p] = -INFINITY; hnrb[p] = 0.f;
                }
                mcs = hm_mcs(hmeta[p]); tbs = htbs[p]; ntx = hm_ntx(hmeta[p]) + 1;
                mcs = mcs < tb.M ? mcs : tb.M - 1;
                comb_p = hcomb[p]; lexp_p = hlexp[p]; nrb_p = hnrb[p]; lo_tx = hlo[p]; hi_tx = hhi[p];
            }
        }
        if (tx_new) sent = sent + byt_new;
        // ---- decoding on the actual channel (mac.py:428-454, mac_ul.py:185-192) ----
        bool ok = false, fail = false, exh = false;
        float comb = comb_p, lexp = lexp_p, nrb = nrb_p;
        if (__ballot(tx) != 0ull) {
            const float beta = tb.beta[mcs];
            float act_s[S];
#pragma unroll
            for (int s = 0; s < S; ++s) act_s[s] = (ref[s] - sp) + gain[s];
            float eff_used;
            int m_look = mcs;
            if (pm.comb == 2) {
                float xv[S];
#pragma unroll
                for (int s = 0; s < S; ++s) xv[s] = (-from_db(clampf(act_s[s], -30.0f, 60.0f))) / beta + lw[s];
                float lse = aten_lse<S>(xv);
                // torch.logaddexp: equal infinities stay, else max + log1p(exp(-|a - b|))
                if (isinf(lexp_p) && lexp_p == lse) lexp = lexp_p;
                else { float mx = lexp_p > lse ? lexp_p : lse; lexp = mx + log1pf(expf(-fabsf(lexp_p - lse))); }
                nrb = nrb_p + n_prb;
                float v = (-beta) * (lexp - logf(clamp_min(nrb, 1.0f)));
                eff_used = nan_to_num(10.0f * log10f(clamp_min(v, 1e-6f)), -30.0f, 60.0f, -30.0f);
                int nt = ntx < tb.EQW - 1 ? ntx : tb.EQW - 1;
                m_look = tb.mcs_eq[mcs * tb.EQW + nt];
                comb = comb_p;
            } else {
                float eff;
                if (pm.eesm) {
                    float xv[S];
#pragma unroll
                    for (int s = 0; s < S; ++s) xv[s] = (-from_db(clampf(act_s[s], -30.0f, 60.0f))) / beta + lw[s];
                    eff = db_of((-beta) * (aten_lse<S>(xv) - lnw));
                } else {
                    float v[S];
#pragma unroll
                    for (int s = 0; s < S; ++s) {
                        float t = act_s[s] * expf(lw[s] - lnw);
                        v[s] = nan_to_num(t, 0.0f, 3.4028234663852886e38f, -3.4028234663852886e38f);
                    }
                    eff = aten_sum<S>(v);
                }
                float lin_e = from_db(eff);
                comb = pm.comb == 1 ? comb_p + lin_e : lin_e;
                eff_used = 10.0f * log10f(clamp_min(comb, 1e-9f));
            }
            float cbs, ncb;
            segment_f(tbs, tb.rate[mcs], cbs, ncb);
            float xc = clampf((cbs - tb.c0) / tb.dc, 0.0f, (float)(tb.C - 1));
            float i0f = clamp_max(floorf(xc), (float)(tb.C - 2));
            float wi = xc - i0f;
            float b = bler_at(tb.bler, (m_look * tb.C + (int)i0f) * tb.G, tb.G, tb.s0, tb.ds, eff_used, wi);
            float p_err = 1.0f - powf(1.0f - b, ncb);
            float u = uniform_bits(elem_hash(mix32(base0 ^ row.salt_bler), (uint32_t)r));
            ok = tx && (u >= p_err);
            fail = tx && !ok;
            exh = fail && ntx >= pm.max_tx;
        }
        // ---- HARQ state update (mac.py:456-477, mac_ul.py:218-219) ----
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (p == p_tx && tx) {
                int stp = hm_state(hmeta[p]);
                int ntxp = ntx;
                if (ok) { stp = 0; hrdy[p] = g; }
                hcomb[p] = comb;
                if (pm.comb == 2) { hlexp[p] = lexp; hnrb[p] = nrb; }
                if (fail) hrdy[p] = g + pm.ul_rtt;
                if (exh) {
                    if (pm.harq_drop) stp = 0;
                    else {
                        ntxp = 0; hcomb[p] = 0.f; hlexp[p] = -INFINITY; hnrb[p] = 0.f;
                        hrdy[p] = g + pm.rlc_retx;
                    }
                }
                hmeta[p] = hm_pack(stp, ntxp, hm_mcs(hmeta[p]), hm_nsb(hmeta[p]));
            }
        }
        // ---- OLLA, BSR, CSI, PF average, RR (mac.py:479-485, mac_ul.py:229-236, mac.py:534-554) ----
        if (pm.olla) olla = clampf((olla + pm.olla_up * (ok ? 1.0f : 0.0f)) - pm.olla_dn * (fail ? 1.0f : 0.0f),
                                   -10.0f, 10.0f);
        const int served = ok ? hi_tx - lo_tx : 0;
        if (tx) bsr = enq - sent;
#pragma unroll
        for (int s = 0; s < S; ++s) csi[s] = gain[s];
        avg = clamp_min(pm.pf_a * avg + pm.pf_b * (float)served, 1e-9f);
        if (pm.sched == 2 && tx) last_tx = g;
        // ---- counters ----
        c_new += tx_new; c_retx += tx_rx; c_ok += ok; c_fail += fail; c_exh += exh;
        c_bytes_ok += served; c_bytes_new += tx_new ? byt_new : 0; c_new_pend += (tx_new && pending);
        c_prb += tx ? (int)n_prb : 0;
        {
            int kh = ntx < pm.max_tx ? ntx : pm.max_tx;
            for (int q = 0; q < HB; ++q) {
                h_ok[q] += (q == kh) && ok;
                h_tx[q] += (q == kh) && tx;
                h_fl[q] += (q == kh) && fail;
            }
        }
        // ---- RLC in-order pointer of this slot (completion replayed in the epilogue) ----
        if (n_ul < MAX_ROWS_UL) {
            ack_hist[n_ul] = ack_ptr();
            exh_lo[n_ul] = (exh && pm.harq_drop) ? lo_tx : 0;
            exh_hi[n_ul] = (exh && pm.harq_drop) ? hi_tx : 0;
        }
        ++n_ul;
    }

    // ================================================================ end of step (NRNet._finish)
    const int t = (int)T;
    const int ack_end = ack_ptr();
    const int ep0 = act ? st.epoch[ee] : 0;
    int newest = -1, kept = 0, lost_new = 0;
    bool det_hit = false;
    int new_floor = enq;
    const int64_t hid_cur = (act && cur_hid) ? cur_hid[ee] : 0;
    const double po = (double)pm.proc_off_hi + (double)pm.proc_off_lo;
    // per-row slot offsets of the UL slots (for completion times)
    int ul_rel[MAX_ROWS_UL];
    {
        int j = 0;
        for (int k = 0; k < n_rows && j < MAX_ROWS_UL; ++k)
            if (rows[k].flags & 2) ul_rel[j++] = rows[k].rel;
    }
    const size_t ob = ((size_t)ee * R + r) * F;     // output row of this robot [E][R][F]
    for (int f = 0; f < F; ++f) {
        bool valid = act && f < qlen;
        int cap = -1, qs = 0, qe = 0, fin = FIN_NONE;
        uint32_t meta = 0;
        size_t iq = ((size_t)ee * F + f) * R + r;
        if (valid) {
            cap = st.q_cap[iq]; qs = st.q_start[iq]; qe = st.q_end[iq]; fin = st.q_fin[iq]; meta = st.q_meta[iq];
        }
        bool lost = meta & 1u;
        if (valid) {
            // replay the slots: lost marking (RLC UM) first, then in-order completion (mac.py:474-477, 500-503)
            for (int j = 0; j < n_ul && j < MAX_ROWS_UL; ++j) {
                if (pm.harq_drop && exh_hi[j] > exh_lo[j] && qs < exh_hi[j] && qe > exh_lo[j]) {
                    if (!lost) ++lost_new;
                    lost = true;
                }
                if (fin == FIN_NONE && !lost && qe <= ack_hist[j]) fin = g0 + ul_rel[j];
            }
        }
        bool delivered = false, timed = false, dropped = false;
        float delay = NAN;
        if (valid) {
            double fin_d = INFINITY;
            if (fin != FIN_NONE) {
                int tf = fin / N, rel = fin - tf * N;
                fin_d = ((double)tf + (double)(rel + 1) / (double)N) + po;
            }
            delivered = fin_d <= ((double)t + 1.0) + 1e-9;
            timed = pm.purge && fin == FIN_NONE && (t + 1 - cap) >= pm.timeout;
            dropped = lost && qe <= ack_end && !timed;
            if (delivered) {
                delay = (float)(fin_d - (double)cap);
                newest = cap > newest ? cap : newest;
                if ((meta & 2u) && st.q_hid[iq] == (int32_t)hid_cur) det_hit = true;
            }
        }
        if (act) {
            int cap_rel = cap >= 0 ? cap - ep0 : -1;
            int cls = valid ? (int)((meta >> 8) & 0xffu) : 0;
            if (pm.out_ref) {
                out.delivered[ob + f] = delivered;
                out.timed_out[ob + f] = timed;
                out.dropped[ob + f] = dropped;
                out.cap[ob + f] = cap_rel;
                out.cls[ob + f] = cls;
            } else {
                out.delivered[ob + f] = (uint8_t)(delivered | (timed << 1) | (dropped << 2));
                out.cap32[ob + f] = cap_rel;
                out.cls8[ob + f] = (uint8_t)cls;
            }
            out.delay[ob + f] = delay;
        }
        // compaction: the frames that stay move to the front, in order (queues.py:105-110)
        if (valid && !(delivered || timed || dropped)) {
            if (kept == 0) new_floor = qs;
            if (kept != f) {
                size_t iw = ((size_t)ee * F + kept) * R + r;
                st.q_cap[iw] = cap; st.q_start[iw] = qs; st.q_end[iw] = qe;
                st.q_meta[iw] = (meta & ~1u) | (lost ? 1u : 0u);
                st.q_hid[iw] = st.q_hid[iq];
                st.q_fin[iw] = fin;
            } else {
                st.q_meta[iq] = (meta & ~1u) | (lost ? 1u : 0u);
                st.q_fin[iq] = fin;
            }
            ++kept;
        }
    }
    if (act) {
        for (int f = kept; f < qlen; ++f) st.q_cap[((size_t)ee * F + f) * R + r] = -1;
    }
    // compact(): floor, sent, dead processes, BSR (mac.py:610-616, mac_ul.py:255-257)
    floor_ = new_floor;
    sent = sent > floor_ ? sent : floor_;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        if (hm_state(hmeta[p]) == 1 && hhi[p] <= floor_ && hhi[p] > hlo[p]) {
            hmeta[p] = hm_pack(0, 0, hm_mcs(hmeta[p]), hm_nsb(hmeta[p]));
            hrdy[p] = 0; hcomb[p] = 0.f; hlexp[p] = -INFINITY; hnrb[p] = 0.f;
        }
    }
    {
        int un = enq - sent;
        bsr = bsr < un ? bsr : un;
    }
    const int ack_new = ack_ptr();
    // ---------------- store state and per-robot outputs ----------------
    if (act) {
        st.sent[ir] = sent; st.floor_[ir] = floor_; st.bsr[ir] = bsr; st.sr_t[ir] = sr_t;
        st.last_tx[ir] = last_tx; st.qlen[ir] = kept; st.olla[ir] = olla; st.avg[ir] = avg;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            size_t is = ((size_t)ee * S + s) * R + r;
            st.csi[is] = csi[s];
            if (pm.fading) { st.h_re[is] = hr[s]; st.h_im[is] = hi[s]; }
        }
#pragma unroll
        for (int p = 0; p < P; ++p) {
            size_t ip = ((size_t)ee * P + p) * R + r;
            st.h_meta[ip] = hmeta[p]; st.h_lo[ip] = hlo[p]; st.h_hi[ip] = hhi[p]; st.h_ready[ip] = hrdy[p];
            st.h_tbs[ip] = htbs[p]; st.h_comb[ip] = hcomb[p];
            if (ir_comb) { st.h_lexp[ip] = hlexp[p]; st.h_nrb[ip] = hnrb[p]; }
        }
        out.newest[ir] = newest >= 0 ? newest - ep0 : -1;
        out.queue_len[ir] = kept;
        int qb = enq - ack_new;
        out.queue_bytes[ir] = (float)(qb > 0 ? qb : 0);
        out.sinr_db[ir] = snr_out;
        if (out.serving_cell) out.serving_cell[ir] = 0;
    }
    // per-env outputs and counters (segment reductions, written by robot 0)
    const bool det_any = seg_any(det_hit, rb, lane);
    int v[10] = {c_new, c_retx, c_ok, c_fail, c_exh, 0, 0, lost_new, c_new_pend, 0};
    for (int q = 0; q < 10; ++q) v[q] = seg_sum_i(act ? v[q] : 0, rb);
    int64_t b_ok = seg_sum_l(act ? c_bytes_ok : 0, rb), b_new = seg_sum_l(act ? c_bytes_new : 0, rb);
    int64_t prb = seg_sum_l(act ? c_prb : 0, rb);
    int hs[3 * (INET_NR_MAX_P + 1)];
    for (int q = 0; q < HB; ++q) {
        hs[q] = seg_sum_i(act ? h_ok[q] : 0, rb);
        hs[HB + q] = seg_sum_i(act ? h_tx[q] : 0, rb);
        hs[2 * HB + q] = seg_sum_i(act ? h_fl[q] : 0, rb);
    }
    if (r == 0 && e < E) {
        out.det_env[e] = det_any;
        out.t[e] = (int64_t)t - (int64_t)st.epoch[e];
        st.ctr_step[e] = st.ctr_step[e] + 1;                 // rng.tick_step (nr_engine.py:847-848)
        int64_t* c = st.ctr + (size_t)e * INET_NR_NCTR;
        c[0] += v[0]; c[1] += v[1]; c[2] += v[2]; c[3] += v[3]; c[4] += v[4];
        c[5] += b_ok; c[6] += b_new; c[7] += v[7]; c[8] += v[8]; c[9] += prb;
        int64_t* h = st.hist + (size_t)e * 3 * HB;
        for (int q = 0; q < 3 * HB; ++q) h[q] += hs[q];
    }
}

// ======================================================================================= submit kernel
// FrameQueue.add + NRNet.add_frames (queues.py:87-103, nr_engine.py:451-487): one frame per message at the tail.
__global__ void nr_submit_kernel(InetNrState st, int E, int R, int F, int T, const int64_t* __restrict__ send,
                                 const uint8_t* __restrict__ det, const int64_t* __restrict__ hid,
                                 const uint8_t* __restrict__ counts, int n_cls, const float* __restrict__ sizes,
                                 int discard_pdcp, int timeout, int pkt_payload, int pkt_overhead, void* accepted) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= E * R) return;
    int e = i / R, r = i - e * R;
    int qlen = st.qlen[i], enq = st.enq[i];
    int n_acc = 0;
    int n_msgs = counts ? 0 : 1;
    if (counts) for (int c = 0; c < n_cls; ++c) n_msgs += counts[(size_t)i * n_cls + c];
    int cls_i = 0, left_in_cls = counts ? 0 : 1;
    for (int k = 0; k < n_msgs; ++k) {
        int cls;
        if (counts) {
            while (left_in_cls == 0) { left_in_cls = counts[(size_t)i * n_cls + cls_i]; ++cls_i; }
            cls = cls_i;
            --left_in_cls;
        } else {
            cls = (int)send[i];
        }
        bool want = cls > 0;
        bool adm = want;
        if (discard_pdcp && qlen > 0) {
            int cap0 = st.q_cap[((size_t)e * F + 0) * R + r];
            if (T - cap0 >= timeout) adm = false;
        }
        float size = sizes[(cls > 0 ? cls : 1) - 1];
        if (pkt_overhead) size = size + ceilf(size / (float)pkt_payload) * (float)pkt_overhead;
        bool acc = adm && qlen < F && size > 0.0f;
        if (acc) {
            int nb = (int)rintf(size);
            size_t iq = ((size_t)e * F + qlen) * R + r;
            st.q_cap[iq] = T; st.q_start[iq] = enq; st.q_end[iq] = enq + nb; st.q_fin[iq] = FIN_NONE;
            uint32_t dm = (det && det[i]) ? 2u : 0u;
            st.q_meta[iq] = dm | ((uint32_t)cls << 8);
            st.q_hid[iq] = hid ? (int32_t)hid[e] : 0;
            enq += nb;
            ++qlen;
            ++n_acc;
        }
        if (!counts) ((uint8_t*)accepted)[i] = acc;
    }
    if (counts && accepted) ((int32_t*)accepted)[i] = n_acc;
    st.qlen[i] = qlen;
    st.enq[i] = enq;
}

// ======================================================================================= reset kernel
// One block per env. NRNet.reset / MacLink.reset / FrameQueue.reset / NRRng.reset_mask and the reset draws: H0 of
// the fading state, the Rician phase (KPHI) and the radio's plane-wave fields (channels/fields.py:38-58,
// radio.py:185-219); the fields' cos / sin / sqrt are evaluated in double precision and rounded once (correctly rounded
// float32), since the step multiplies each wave vector by positions of hundreds of metres.
__global__ void nr_reset_kernel(InetNrState st, InetNrParams pm, const uint8_t* __restrict__ mask, int T, float k_lin0,
                                float dc0, float dc1, float dc2, int spectrum, int full) {
    const int e = blockIdx.x;
    if (e >= pm.E) return;
    if (!full && !mask[e]) return;
    const int R = pm.R, S = pm.S, P = pm.P, F = pm.F;
    __shared__ int ep_new;
    if (threadIdx.x == 0) ep_new = st.episode[e] + 1;
    __syncthreads();
    const uint32_t s0 = (uint32_t)pm.seed_key, env = (uint32_t)st.env_id[e], ep = (uint32_t)ep_new;
    for (int r = threadIdx.x; r < R; r += blockDim.x) {
        size_t ir = (size_t)e * R + r;
        st.sent[ir] = 0; st.floor_[ir] = 0; st.bsr[ir] = 0; st.sr_t[ir] = -1; st.last_tx[ir] = -1;
        st.olla[ir] = 0.f; st.avg[ir] = 100.f; st.enq[ir] = 0; st.qlen[ir] = 0;
        for (int s = 0; s < S; ++s) st.csi[((size_t)e * S + s) * R + r] = 0.f;
        for (int p = 0; p < P; ++p) {
            size_t ip = ((size_t)e * P + p) * R + r;
            st.h_meta[ip] = 0u; st.h_lo[ip] = 0; st.h_hi[ip] = 0; st.h_ready[ip] = 0; st.h_tbs[ip] = 0;
            st.h_comb[ip] = 0.f; st.h_lexp[ip] = -INFINITY; st.h_nrb[ip] = 0.f;
        }
        for (int f = 0; f < F; ++f) {
            size_t iq = ((size_t)e * F + f) * R + r;
            st.q_cap[iq] = -1; st.q_start[iq] = 0; st.q_end[iq] = 0; st.q_fin[iq] = FIN_NONE;
            st.q_meta[iq] = 0u; st.q_hid[iq] = 0;
        }
        // H0: N(0, 1) / sqrt 2 per element (r, s, re/im) of the per-env draw (nr_engine.py:262-263)
        const uint32_t bh = base_key(s0, env, ep, CH_RESET, 0u, SITE_H0 << 16);
        for (int s = 0; s < S; ++s) {
            uint32_t j = (uint32_t)((r * S + s) * 2);
            size_t is = ((size_t)e * S + s) * R + r;
            st.h_re[is] = normal_at(bh, j) / (float)1.4142135623730951;
            st.h_im[is] = normal_at(bh, j + 1u) / (float)1.4142135623730951;
        }
        if (pm.rician) {                                   // phi = 2 pi u (KPHI), nr_engine.py:293-299
            const uint32_t bk = base_key(s0, env, ep, CH_RESET, 0u, SITE_KPHI << 16);
            float phi = (float)6.283185307179586 * uniform_bits(elem_hash(bk, (uint32_t)r));
            st.spec_re[ir] = cosf(phi);
            st.spec_im[ir] = sinf(phi);
            st.k_lin[ir] = k_lin0;
        }
    }
    // env-level: radio fields (draw_plane_waves) of the new episode
    const int K = pm.n_modes;
    const float dcs[3] = {dc0, dc1, dc2};
    for (int q = threadIdx.x; q < pm.n_fields * K; q += blockDim.x) {
        int fi = q / K, kk = q - fi * K;
        uint32_t st0 = pm.radio_model == 1 ? TR38901_STREAM + 3u * fi : LOG_DISTANCE_STREAM;
        float u0 = uniform_bits(elem_hash(base_key(s0, env, ep, CH_RESET, 0u, st0 + 0u), (uint32_t)kk));
        float u1 = uniform_bits(elem_hash(base_key(s0, env, ep, CH_RESET, 0u, st0 + 1u), (uint32_t)kk));
        float u2 = uniform_bits(elem_hash(base_key(s0, env, ep, CH_RESET, 0u, st0 + 2u), (uint32_t)kk));
        float ang = (u0 * 2.0f) * (float)3.141592653589793;          // rand * 2 * pi, in that order
        float kmag;
        if (spectrum == 0) {                                          // "sos": wavelengths 20..60 m
            float wl = 20.0f + 40.0f * u1;
            if (dcs[fi] != 10.3f) wl = wl * (float)((double)dcs[fi] / 10.3);
            kmag = (1.0f / wl) * (float)6.283185307179586;            // 2 pi / wl = reciprocal(wl) * 2 pi
        } else {                                                      // "exp": inverse CDF of the radial spectrum
            float u = clamp_max(u1, (float)(1.0 - 1e-6));
            float a = 1.0f - u;
            kmag = sqrtf(1.0f / (a * a) - 1.0f) / dcs[fi];
        }
        float* fp = st.field + (((size_t)e * pm.n_fields + fi) * K + kk) * 3;
        fp[0] = (float)cos((double)ang) * kmag;
        fp[1] = (float)sin((double)ang) * kmag;
        fp[2] = (u2 * 2.0f) * (float)3.141592653589793;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        st.episode[e] = ep_new;
        st.ctr_step[e] = 0;
        st.ctr_submit[e] = 0;
        st.epoch[e] = T;
        if (full) {
            for (int q = 0; q < INET_NR_NCTR; ++q) st.ctr[(size_t)e * INET_NR_NCTR + q] = 0;
            for (int q = 0; q < 3 * (pm.max_tx + 1); ++q) st.hist[(size_t)e * 3 * (pm.max_tx + 1) + q] = 0;
        }
    }
}

// ======================================================================================= C ABI
namespace {

typedef void (*StepFn)(dim3, hipStream_t, const InetNrState&, const InetNrTables&, const InetNrParams&,
                       const InetNrRow*, int, int64_t, const float*, const int64_t*, const InetNrOutputs&, int);

template <int S, int P>
void launch_step(dim3 grid, hipStream_t s, const InetNrState& st, const InetNrTables& tb, const InetNrParams& pm,
                 const InetNrRow* rows, int n_rows, int64_t T, const float* x, const int64_t* hid,
                 const InetNrOutputs& out, int rb) {
    hipLaunchKernelGGL((nr_step_kernel<S, P>), grid, dim3(BLOCK), 0, s, st, tb, pm, rows, n_rows, T, x, hid, out, rb);
}

StepFn pick_step(int S, int P) {
#define INET_CASE(SS, PP) if (S == SS && P == PP) return &launch_step<SS, PP>;
    INET_CASE(13, 2) INET_CASE(13, 4) INET_CASE(13, 8) INET_CASE(13, 16)
    INET_CASE(8, 2) INET_CASE(8, 4) INET_CASE(8, 8) INET_CASE(8, 16)
#undef INET_CASE
    return nullptr;
}

int next_pow2(int v) { int p = 1; while (p < v) p <<= 1; return p; }

}  // namespace

extern "C" {

int32_t inet_nr_abi_version(void) { return INET_NR_ABI_VERSION; }

const char* inet_nr_build_info(void) {
    return "inet_nr gfx950: step<S in {8,13}, P in {2,4,8,16}>, wave64 segments, ATen-order reductions";
}

int32_t inet_nr_step(const InetNrState* st, const InetNrTables* tab, const InetNrParams* prm, const InetNrRow* rows,
                     int32_t n_rows, int64_t T, const float* x, const int64_t* cur_hid, const InetNrOutputs* out,
                     void* stream) {
    if (!st || !tab || !prm || !out || !x) return INET_NR_EINVAL;
    const InetNrParams& p = *prm;
    if (p.E <= 0 || p.R <= 0 || p.R > INET_NR_MAX_R || p.F <= 0 || p.N <= 0) return INET_NR_EINVAL;
    if (p.S > INET_NR_MAX_S || p.P > INET_NR_MAX_P || p.max_tx + 1 > INET_NR_MAX_P + 1) return INET_NR_EINVAL;
    if (n_rows < 0 || (n_rows > 0 && !rows) || p.n_modes > INET_NR_MAX_KF) return INET_NR_EINVAL;
    if (T < 0 || T * (int64_t)p.N > (int64_t)0x3fffffff) return INET_NR_EINVAL;
    StepFn fn = pick_step(p.S, p.P);
    if (!fn) return INET_NR_EUNSUPPORTED;
    int rb = next_pow2(p.R);
    int envs_pb = BLOCK / rb;
    dim3 grid((p.E + envs_pb - 1) / envs_pb);
    fn(grid, (hipStream_t)stream, *st, *tab, p, rows, n_rows, T, x, cur_hid, *out, rb);
    return hipGetLastError() == hipSuccess ? INET_NR_OK : INET_NR_ELAUNCH;
}

int32_t inet_nr_submit(const InetNrState* st, const InetNrParams* prm, int64_t T, const int64_t* send,
                       const uint8_t* det, const int64_t* hid, const uint8_t* counts, int32_t n_cls,
                       const float* sizes, int32_t discard_pdcp, int32_t pkt_payload, int32_t pkt_overhead,
                       void* accepted, void* stream) {
    if (!st || !prm || !sizes || (!send && !counts) || (send && counts)) return INET_NR_EINVAL;
    if (!counts && !accepted) return INET_NR_EINVAL;
    if (counts && n_cls <= 0) return INET_NR_EINVAL;
    if (T < 0 || T > 0x7fffffff || (pkt_overhead && pkt_payload <= 0)) return INET_NR_EINVAL;
    const InetNrParams& p = *prm;
    int n = p.E * p.R;
    hipLaunchKernelGGL(nr_submit_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, *st, p.E, p.R,
                       p.F, (int)T, send, det, hid, counts, n_cls, sizes, discard_pdcp, p.timeout, pkt_payload,
                       pkt_overhead, accepted);
    return hipGetLastError() == hipSuccess ? INET_NR_OK : INET_NR_ELAUNCH;
}

int32_t inet_nr_reset(const InetNrState* st, const InetNrParams* prm, const uint8_t* mask, int64_t T, float k_lin0,
                      const float* dcorr, int32_t spectrum, void* stream) {
    if (!st || !prm || !dcorr) return INET_NR_EINVAL;
    const InetNrParams& p = *prm;
    if (p.E <= 0 || p.R <= 0 || p.n_fields < 0 || p.n_fields > 3 || p.n_modes > INET_NR_MAX_KF) return INET_NR_EINVAL;
    if (T < 0 || T > 0x7fffffff) return INET_NR_EINVAL;
    hipLaunchKernelGGL(nr_reset_kernel, dim3(p.E), dim3(64), 0, (hipStream_t)stream, *st, p, mask, (int)T, k_lin0,
                       dcorr[0], dcorr[1], dcorr[2], spectrum, mask ? 0 : 1);
    return hipGetLastError() == hipSuccess ? INET_NR_OK : INET_NR_ELAUNCH;
}

}  // extern "C"

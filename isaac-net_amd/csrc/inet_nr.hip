// MI355X (gfx950) kernels of isaac-net's NR uplink engine other than the control step (nr_step.h), and the C ABI of
// include/inet_nr.h: the enqueue kernel (FrameQueue.add / NRNet.add_frames), the reset kernel (NRNet.reset and the
// reset draws of the fading state, Rician phase and shadowing fields) and the entry points that check their
// arguments and launch.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "../../include/inet_nr.h"
#include "inet_nr_dev.h"

#include "nr_step.h"

using namespace inet;

namespace {

constexpr uint32_t CH_RESET = 3;
constexpr uint32_t SITE_H0 = 4, SITE_KFAC = 5, SITE_KPHI = 6, SITE_DSPR = 7;

}  // namespace

// ======================================================================================= submit kernel
// FrameQueue.add + NRNet.add_frames (queues.py:87-103, nr_engine.py:451-487): one frame per message at the tail.
__global__ void nr_submit_kernel(InetNrState st, int E, int R, int F, int64_t T_arg, const int64_t* __restrict__ send,
                                 const uint8_t* __restrict__ det, const int64_t* __restrict__ hid,
                                 const uint8_t* __restrict__ counts, int n_cls, const float* __restrict__ sizes,
                                 int discard_pdcp, int timeout, int pkt_payload, int pkt_overhead, void* accepted) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= E * R) return;
    const int T = (int)(T_arg >= 0 ? T_arg : st.clock[0]);
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

// ======================================================================================= DL submit kernel
// NRNet.add_dl_frames (nr_engine.py:489-497) with FrameQueue.add (queues.py:87-103): one DL frame of nbytes at the
// tail. The class is a meta field that add does not reset: without cls the slot keeps the class it held.
__global__ void nr_dl_submit_kernel(InetNrState st, InetNrDlState dl, int E, int R, int F, int64_t T_arg,
                                    const float* __restrict__ nbytes, const int64_t* __restrict__ cls,
                                    int discard_pdcp, int timeout, int pkt_payload, int pkt_overhead,
                                    uint8_t* __restrict__ accepted) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= E * R) return;
    const int T = (int)(T_arg >= 0 ? T_arg : st.clock[0]);
    const int e = i / R, r = i - e * R;
    int qlen = dl.qlen[i];
    const int enq = dl.enq[i];
    float size = nbytes[i];
    bool adm = size > 0.0f;
    if (discard_pdcp && qlen > 0) {
        int cap0 = dl.q_cap[((size_t)e * F + 0) * R + r];
        if (T - cap0 >= timeout) adm = false;
    }
    if (pkt_overhead) size = size + ceilf(size / (float)pkt_payload) * (float)pkt_overhead;
    // (frames above 2^22 bytes are refused: F of them stay inside the int32 offsets between two rebases)
    const bool acc = adm && qlen < F && size > 0.0f && size <= 4194304.0f;
    if (acc) {
        const int nb = (int)rintf(size);
        const size_t iq = ((size_t)e * F + qlen) * R + r;
        dl.q_cap[iq] = T; dl.q_start[iq] = enq; dl.q_end[iq] = enq + nb; dl.q_fin[iq] = FIN_NONE;
        const uint32_t c = cls ? ((uint32_t)cls[i] & 0xffu) << 8 : dl.q_meta[iq] & 0xff00u;
        dl.q_meta[iq] = c;
        dl.enq[i] = enq + nb;
        dl.qlen[i] = qlen + 1;
    }
    accepted[i] = acc;
}

// ======================================================================================= DL reset kernel
// MacLink.reset / FrameQueue.reset of NRNet.dl and dl_newest = -1 (nr_engine.py:256-274) for the envs of the mask;
// a full reset (mask NULL) also clears the DL counters.
__global__ void nr_dl_reset_kernel(InetNrDlState dl, InetNrParams pm, const uint8_t* __restrict__ mask, int full) {
    const int e = blockIdx.x;
    if (e >= pm.E) return;
    if (!full && !mask[e]) return;
    const int R = pm.R, S = pm.S, P = pm.P, F = pm.F;
    for (int r = threadIdx.x; r < R; r += blockDim.x) {
        size_t ir = (size_t)e * R + r;
        dl.sent[ir] = 0; dl.floor_[ir] = 0; dl.last_tx[ir] = -1; dl.olla[ir] = 0.f; dl.avg[ir] = 100.f;
        if (dl.base) dl.base[ir] = 0;
        dl.enq[ir] = 0; dl.qlen[ir] = 0; dl.newest[ir] = -1;
        for (int s = 0; s < S; ++s) dl.csi[((size_t)e * S + s) * R + r] = 0.f;
        for (int p = 0; p < P; ++p) {
            size_t ip = ((size_t)e * P + p) * R + r;
            dl.h_meta[ip] = 0u; dl.h_lo[ip] = 0; dl.h_hi[ip] = 0; dl.h_ready[ip] = 0; dl.h_tbs[ip] = 0;
            dl.h_comb[ip] = 0.f; dl.h_lexp[ip] = -INFINITY; dl.h_nrb[ip] = 0.f;
        }
        for (int f = 0; f < F; ++f) {
            size_t iq = ((size_t)e * F + f) * R + r;
            dl.q_cap[iq] = -1; dl.q_start[iq] = 0; dl.q_end[iq] = 0; dl.q_fin[iq] = FIN_NONE; dl.q_meta[iq] = 0u;
        }
    }
    if (full && threadIdx.x == 0) {
        for (int q = 0; q < INET_NR_NCTR; ++q) dl.ctr[(size_t)e * INET_NR_NCTR + q] = 0;
        for (int q = 0; q < 3 * (pm.max_tx + 1); ++q) dl.hist[(size_t)e * 3 * (pm.max_tx + 1) + q] = 0;
    }
}

// ======================================================================================= cells reset kernel
// CellAssociation.reset and NRNet._reset_cells (radio.py:402-408, nr_engine.py:424-438) of the envs of the mask: serving
// cell 0 until the next step's association, no A3 candidate, no interruption, no handovers, no radio link failure
// state; every gNB's N+I estimate back to the noise; a full reset (mask NULL) also clears the interference statistic
// and the RLF counters.
__global__ void nr_cells_reset_kernel(InetNrCells cl, int E, int R, int S, const uint8_t* __restrict__ mask, int full) {
    const int e = blockIdx.x;
    if (e >= E) return;
    if (!full && !mask[e]) return;
    for (int r = threadIdx.x; r < R; r += blockDim.x) {
        size_t ir = (size_t)e * R + r;
        cl.serv[ir] = 0; cl.a3_cand[ir] = -1; cl.a3_cnt[ir] = 0; cl.ho_end[ir] = 0; cl.n_ho[ir] = 0;
        if (cl.rlf) {
            cl.rlf_active[ir] = 0; cl.oos_cnt[ir] = 0; cl.is_cnt[ir] = 0; cl.t310_end[ir] = -1; cl.t311_end[ir] = -1;
            cl.reest_end[ir] = -1; cl.reest_cell[ir] = 0; cl.n_rlf[ir] = 0;
        }
    }
    for (int q = threadIdx.x; q < cl.C * S; q += blockDim.x) cl.ni_ul[(size_t)e * cl.C * S + q] = cl.noise_mw;
    if (threadIdx.x == 0) {
        cl.pending[e] = 1;
        if (full) cl.ion[e] = 0.f;
        if (full && cl.rlf)
            for (int k = 0; k < 5; ++k) cl.rlf_ctr[(size_t)e * 5 + k] = 0;
    }
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
    const int NC = pm.n_cells > 1 ? pm.n_cells : 1;
    __shared__ int ep_new;
    if (threadIdx.x == 0) {
        ep_new = st.episode[e] + 1;
        if (pm.rician && pm.k_from_los) st.k_fresh[e] = 1;      // waiting for the env's first LOS state
    }
    __syncthreads();
    const uint32_t s0 = (uint32_t)pm.seed_key, env = (uint32_t)st.env_id[e], ep = (uint32_t)ep_new;
    for (int r = threadIdx.x; r < R; r += blockDim.x) {
        size_t ir = (size_t)e * R + r;
        st.sent[ir] = 0; st.floor_[ir] = 0; st.bsr[ir] = 0; st.sr_t[ir] = -1; st.last_tx[ir] = -1;
        if (st.base) st.base[ir] = 0;
        if (st.last_nprb) st.last_nprb[ir] = 0.f;
        if (pm.doppler) st.has_prev[ir] = 0;          // (radio.py:218: no last pose; rho_ms is kept)
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
        // H0: N(0, 1) / sqrt 2 per element (r, c, s, re/im) of the per-env draw (nr_engine.py:262-263), for every
        // robot-cell link q = c S + s
        const uint32_t bh = base_key(s0, env, ep, CH_RESET, 0u, SITE_H0 << 16);
        const int CS = NC * S;
        for (int q = 0; q < CS; ++q) {
            uint32_t j = (uint32_t)((r * CS + q) * 2);
            size_t is = ((size_t)e * CS + q) * R + r;
            st.h_re[is] = div_const(normal_at(bh, j), SQRT2_F, INV_SQRT2_F);
            st.h_im[is] = div_const(normal_at(bh, j + 1u), SQRT2_F, INV_SQRT2_F);
        }
        if (pm.fc_on) {
            // frequency-correlated fading: the initial state correlated across the subbands too, h0 <- L h0 per link
            // (nr_engine.py:264-266), the products accumulated in subband order; rows from the last down, so each
            // reads the uncorrelated values of the rows above it. One delay spread: L = fc_L, fused multiply-adds (a
            // float32 matrix product). Per-link delay spreads: the link's NLOS and LOS grid indices from two normals
            // of reset site DSPR (elements 2 r, 2 r + 1; nr_engine.py:341-363), L = fc_tab[NLOS index], and the
            // batched product's order: separate multiplies and adds while S S 2 < 400, fused above
            // (several cells: every robot-cell link c has its own two normals, elements 2 (r NC + c) + {0, 1}, and
            // its own indices, state [E][NC][R])
            const float* L = pm.fc_L;
            const bool seq = pm.fc_on == 2 && S * S * 2 < 400;
            const uint32_t bd = base_key(s0, env, ep, CH_RESET, 0u, SITE_DSPR << 16);
            for (int c = 0; c < NC; ++c) {
                if (pm.fc_on == 2) {
                    const uint32_t j = 2u * (uint32_t)(r * NC + c);
                    const size_t ic = ((size_t)e * NC + c) * R + r;
                    const int idn = ds_index(pm.ds_mu_n, pm.ds_sig_n, normal_at(bd, j), pm.ds_c1, pm.ds_c2, pm.fc_G);
                    const int idl = ds_index(pm.ds_mu_l, pm.ds_sig_l, normal_at(bd, j + 1u), pm.ds_c1, pm.ds_c2,
                                             pm.fc_G);
                    st.fc_idn[ic] = idn; st.fc_idl[ic] = idl; st.fc_idx[ic] = idn;
                    L = pm.fc_tab + (size_t)idn * S * S;
                }
                const size_t i0 = ((size_t)e * CS + c * S) * R + r;
                for (int i = S - 1; i >= 0; --i) {
                    float ar = 0.f, ai = 0.f;
                    for (int jj = 0; jj <= i; ++jj) {
                        const float l = L[i * S + jj];
                        const float xr = st.h_re[i0 + (size_t)jj * R], xi = st.h_im[i0 + (size_t)jj * R];
                        if (seq) { ar = ar + l * xr; ai = ai + l * xi; }
                        else { ar = fmaf(l, xr, ar); ai = fmaf(l, xi, ai); }
                    }
                    st.h_re[i0 + (size_t)i * R] = ar;
                    st.h_im[i0 + (size_t)i * R] = ai;
                }
            }
        }
        if (pm.rician) {                                   // phi = 2 pi u (KPHI), nr_engine.py:293-299
            // every robot-cell link c: element j = r NC + c of the per-env draws, state [E][NC][R]
            const uint32_t bk = base_key(s0, env, ep, CH_RESET, 0u, SITE_KPHI << 16);
            const uint32_t bz = base_key(s0, env, ep, CH_RESET, 0u, SITE_KFAC << 16);
            for (int c = 0; c < NC; ++c) {
                const uint32_t j = (uint32_t)(r * NC + c);
                const size_t ic = ((size_t)e * NC + c) * R + r;
                float phi = (float)6.283185307179586 * uniform_bits(elem_hash(bk, j));
                st.spec_re[ic] = cosf(phi);
                st.spec_im[ic] = sinf(phi);
                st.k_lin[ic] = k_lin0;
                if (pm.k_from_los) {
                    // K from the LOS state (nr_engine.py:300-303): k_los = 10^((mu_K + sigma_K z) / 10), z the link's
                    // KFAC normal; K = 0 until the link is reported LOS. 10^x in double, rounded once.
                    const float x = (pm.k_mu + pm.k_sigma * normal_at(bz, j)) / 10.0f;
                    st.k_los[ic] = (float)exp10((double)x);
                    st.k_lin[ic] = 0.0f;
                    st.k_from[ic] = 0.0f;
                    st.k_g0[ic] = 0;
                }
            }
        }
    }
    // env-level: radio fields (draw_plane_waves) of the new episode, one per cell: wave kk of cell c is element
    // c K + kk of the field's draws
    const int K = pm.n_modes;
    const float dcs[3] = {dc0, dc1, dc2};
    for (int q = threadIdx.x; q < NC * pm.n_fields * K; q += blockDim.x) {
        int c = q / (pm.n_fields * K), rem = q - c * pm.n_fields * K;
        int fi = rem / K, kk = rem - fi * K;
        draw_plane_wave(s0, env, ep, pm.radio_model, fi, c * K + kk, dcs[fi], spectrum,
                        st.field + ((((size_t)e * NC + c) * pm.n_fields + fi) * K + kk) * 3);
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

// the radio link failure state and constants of a cells struct with rlf set (step: with the rlf output)
bool rlf_ok(const InetNrCells& c, bool step) {
    return c.rlf_active && c.oos_cnt && c.is_cnt && c.t310_end && c.t311_end && c.reest_end && c.reest_cell && c.n_rlf &&
           c.rlf_ctr && (c.out_rlf || !step) && c.n310 >= 1 && c.n311 >= 1 && c.t310 >= 0 && c.t311 >= 0 &&
           c.reest >= 0;
}

int next_pow2(int v) { int p = 1; while (p < v) p <<= 1; return p; }

// the argument checks and the launch of one step kernel (UL: dl NULL)
int32_t launch_step_kernel(const InetNrState* st, const InetNrDlState* dl, const InetNrTables* tab,
                           const InetNrParams* prm, const InetNrRow* rows, int32_t n_rows, int64_t T, const float* x,
                           const int64_t* cur_hid, const InetNrOutputs* out, const InetNrArrivals* arr,
                           void* stream, const InetNrCells* cells = nullptr) {
    const InetNrParams& p = *prm;
    const InetNrTables& t = *tab;
    if (p.E <= 0 || p.R <= 0 || p.R > INET_NR_MAX_R || p.F <= 0 || p.N <= 0) return INET_NR_EINVAL;
    if (p.S > INET_NR_MAX_S || p.P > INET_NR_MAX_P || p.max_tx < 1 || p.max_tx + 1 > INET_NR_MAX_P + 1)
        return INET_NR_EINVAL;
    if (n_rows < 0 || n_rows > INET_NR_MAX_ROWS || (n_rows > 0 && !rows) || p.n_modes > INET_NR_MAX_KF)
        return INET_NR_EINVAL;
    if (t.M <= 0 || t.M > inet::MAX_M || t.EQW <= 0 || t.EQW > inet::MAX_EQW || t.mcs_max >= t.M) return INET_NR_EINVAL;
    if (p.input_kind < 0 || p.input_kind > 3 || (p.input_kind == 3 && !cells)) return INET_NR_EINVAL;
    if ((T < 0 && !st->clock) || T * (int64_t)p.N > (int64_t)0x3fffffff) return INET_NR_EINVAL;
    if (p.n_data < 0 || p.n_data > n_rows) return INET_NR_EINVAL;
    if (p.amc_prev && !st->last_nprb) return INET_NR_EINVAL;     // (the UL link's last PUSCH PRBs are state)
    if (p.fc_on < 0 || p.fc_on > 2 || (p.fc_on == 1 && !p.fc_L)) return INET_NR_EINVAL;
    if (p.fc_on == 2 && (!p.fc_tab || p.fc_G < 1 || !st->fc_idx || !st->fc_idl || !st->fc_idn))
        return INET_NR_EINVAL;
    if (p.k_from_los && (!p.rician || !st->k_los || !st->k_from || !st->k_g0 || !st->k_fresh || p.k_ramp < 0))
        return INET_NR_EINVAL;
    if (p.los_sto && (!p.los_cdf || p.radio_model != 1 || p.n_fields != 3 || p.plos_scn < 0 || p.plos_scn > 2))
        return INET_NR_EINVAL;
    if (p.doppler && (!st->prev_pos || !st->has_prev || !st->rho_ms || !(p.dop_dt > 0.0f)))
        return INET_NR_EINVAL;
    const int n_data = p.n_data > 0 ? p.n_data : n_rows;
    const bool ir = p.comb == 2, vref = p.input_kind == 2;
    const int rb = next_pow2(p.R);
    // the single-cell entry points run one cell; inet_nr_step_cells several
    if ((cells != nullptr) != (p.n_cells > 1)) return INET_NR_EINVAL;
    inet::StepFn fn;
    // the builds with the common switches fixed at compile time (INET_NR_GENERIC=1 keeps the general build, for
    // comparing the two)
    const char* gen = getenv("INET_NR_GENERIC");
    const int fx = (gen && gen[0] == '1') ? 0 : inet::fx_profile(p);
    if (cells) {
        const InetNrCells& c = *cells;
        if (c.C != p.n_cells || c.C > INET_NR_MAX_C || (p.input_kind != 0 && p.input_kind != 3) || p.F > 64 || dl)
            return INET_NR_EINVAL;
        if (!c.serv || !c.a3_cand || !c.a3_cnt || !c.ho_end || !c.n_ho || !c.pending || !c.ni_ul || !c.ion)
            return INET_NR_EINVAL;
        if (c.ttt < 0 || c.ho_int < 0 || !(c.noise_mw > 0.0f)) return INET_NR_EINVAL;
        if (c.rlf && !rlf_ok(c, true)) return INET_NR_EINVAL;
        fn = inet::pick_step_mc(p.S, c.C, p.P, ir, fx, rb);
    } else if (rb > inet::STEP_WAVE) {          // 65..128 / 129..256 robots: two / four wavefronts per env (the DL: two)
        if (vref || (dl && rb > 2 * inet::STEP_WAVE)) return INET_NR_EUNSUPPORTED;
        fn = rb == 2 * inet::STEP_WAVE ? inet::pick_step_two_waves(p.S, p.P, ir, fx) : inet::pick_step_w4(p.S, p.P, ir);
    } else {
        fn = inet::pick_step_one_cell(p.S, p.P, ir, vref, rb, fx);
    }
    if (!fn) return INET_NR_EUNSUPPORTED;
    const int envs_pw = rb > inet::STEP_WAVE ? 1 : inet::STEP_WAVE / rb;
    InetNrArrivals none{};
    if (arr && (!arr->counts || !arr->sizes || arr->n_cls <= 0 || (arr->pkt_overhead && arr->pkt_payload <= 0)))
        return INET_NR_EINVAL;
    // the DL link resolves frame completion in the slot loop: no per-slot history in LDS
    const int n_hist = dl ? 0 : n_data;
    inet::StepArgs a{*st, dl, cells, t, p, rows, n_rows, n_hist, arr ? *arr : none, T, x, cur_hid, *out, rb,
                     (unsigned)((p.E + envs_pw - 1) / envs_pw),
                     inet::step_lds_bytes(n_hist, p.harq_drop, rb, p.max_tx, cells ? cells->C : 1, p.S),
                     (hipStream_t)stream};
    // several cells: the static LDS grows with the cells (each lane's fading normals, 2 NC S floats, the
    // interference pairs and every robot's PSD at each cell; under 16 KiB besides) and must fit the CU's 160 KiB
    // with the dynamic part
    if (cells) {
        const size_t nc = (size_t)cells->C, ns = (size_t)p.S;
        const size_t stat = sizeof(float) * (2 * nc * ns * inet::STEP_WAVE + nc * ns * (1 + 2 * nc) +
                                             nc * inet::STEP_WAVE) + 16384;
        if (a.lds + stat > 160 * 1024) return INET_NR_EUNSUPPORTED;
    }
    fn(a);
    return hipGetLastError() == hipSuccess ? INET_NR_OK : INET_NR_ELAUNCH;
}

}  // namespace

extern "C" {

int32_t inet_nr_abi_version(void) { return INET_NR_ABI_VERSION; }

#ifndef INET_SRC_HASH
#define INET_SRC_HASH "unknown"
#endif
// "<description>; src=<sha256 of the sources the library was built from>" (build.py passes the hash; the loader
// refuses a library whose hash is not the tree's)
const char* inet_nr_build_info(void) {
    return "inet_nr gfx950: one-cell step<S in {8,10,11,12,13,14,16,17,18}, P in {2,4,8,16}, IR, per-subband SNR> "
           "for envs of up to 64 robots (UL and DL), two-wave step (R <= 128, every S), four-wave step (R <= 256, "
           "S in {8,13}), multi-cell step<C in {2,3}, S in {8,13,14}, P, IR>, common-configuration builds (FX 1, 2), "
           "radio link failure, per-robot Doppler, wideband PF, DPP segment reductions, ATen-order sums; Wi-Fi "
           "mean-field (one AP or up to 8 on one channel) and DCF steps, each with or without the enqueue in the "
           "step launch; src=" INET_SRC_HASH;
}

int32_t inet_nr_step(const InetNrState* st, const InetNrTables* tab, const InetNrParams* prm, const InetNrRow* rows,
                     int32_t n_rows, int64_t T, const float* x, const int64_t* cur_hid, const InetNrOutputs* out,
                     void* stream) {
    if (!st || !tab || !prm || !out || !x) return INET_NR_EINVAL;
    return launch_step_kernel(st, nullptr, tab, prm, rows, n_rows, T, x, cur_hid, out, nullptr, stream);
}

int32_t inet_nr_submit_step(const InetNrState* st, const InetNrTables* tab, const InetNrParams* prm,
                            const InetNrRow* rows, int32_t n_rows, int64_t T, const float* x, const int64_t* cur_hid,
                            const InetNrOutputs* out, const InetNrArrivals* arr, void* stream) {
    if (!st || !tab || !prm || !out || !x || !arr) return INET_NR_EINVAL;
    return launch_step_kernel(st, nullptr, tab, prm, rows, n_rows, T, x, cur_hid, out, arr, stream);
}

int32_t inet_nr_step_cells(const InetNrState* st, const InetNrCells* cells, const InetNrTables* tab,
                           const InetNrParams* prm, const InetNrRow* rows, int32_t n_rows, int64_t T, const float* x,
                           const int64_t* cur_hid, const InetNrOutputs* out, const InetNrArrivals* arr, void* stream) {
    if (!st || !cells || !tab || !prm || !out || !x) return INET_NR_EINVAL;
    return launch_step_kernel(st, nullptr, tab, prm, rows, n_rows, T, x, cur_hid, out, arr, stream, cells);
}

int32_t inet_nr_cells_reset(const InetNrCells* cells, const InetNrParams* prm, const uint8_t* mask, void* stream) {
    if (!cells || !prm) return INET_NR_EINVAL;
    const InetNrParams& p = *prm;
    const InetNrCells& c = *cells;
    if (p.E <= 0 || p.R <= 0 || p.S <= 0 || p.S > INET_NR_MAX_S || c.C < 2 || c.C > INET_NR_MAX_C || c.C != p.n_cells)
        return INET_NR_EINVAL;
    if (!c.serv || !c.a3_cand || !c.a3_cnt || !c.ho_end || !c.n_ho || !c.pending || !c.ni_ul || !c.ion)
        return INET_NR_EINVAL;
    if (c.rlf && !rlf_ok(c, false)) return INET_NR_EINVAL;
    hipLaunchKernelGGL(nr_cells_reset_kernel, dim3(p.E), dim3(64), 0, (hipStream_t)stream, c, p.E, p.R, p.S, mask,
                       mask ? 0 : 1);
    return hipGetLastError() == hipSuccess ? INET_NR_OK : INET_NR_ELAUNCH;
}

int32_t inet_nr_dl_step(const InetNrState* st, const InetNrDlState* dl, const InetNrTables* tab,
                        const InetNrParams* prm, const InetNrRow* rows, int32_t n_rows, int64_t T, const float* x,
                        void* stream) {
    if (!st || !dl || !tab || !prm || !x) return INET_NR_EINVAL;
    if (!dl->sent || !dl->q_cap || !dl->newest || !dl->out_newest || !dl->out_queue_len || !dl->ctr || !dl->hist)
        return INET_NR_EINVAL;
    if ((dl->cqi_thr == nullptr) != (dl->cqi_mcs == nullptr) || dl->gnb_proc < 0) return INET_NR_EINVAL;
    InetNrOutputs none{};
    return launch_step_kernel(st, dl, tab, prm, rows, n_rows, T, x, nullptr, &none, nullptr, stream);
}

int32_t inet_nr_dl_submit(const InetNrState* st, const InetNrDlState* dl, const InetNrParams* prm, int64_t T,
                          const float* nbytes, const int64_t* cls, int32_t discard_pdcp, int32_t pkt_payload,
                          int32_t pkt_overhead, uint8_t* accepted, void* stream) {
    if (!st || !dl || !prm || !nbytes || !accepted) return INET_NR_EINVAL;
    if ((T < 0 && !st->clock) || T > 0x7fffffff || (pkt_overhead && pkt_payload <= 0)) return INET_NR_EINVAL;
    const InetNrParams& p = *prm;
    if (p.E <= 0 || p.R <= 0 || p.F <= 0) return INET_NR_EINVAL;
    int n = p.E * p.R;
    hipLaunchKernelGGL(nr_dl_submit_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, *st, *dl, p.E,
                       p.R, p.F, T, nbytes, cls, discard_pdcp, p.timeout, pkt_payload, pkt_overhead, accepted);
    return hipGetLastError() == hipSuccess ? INET_NR_OK : INET_NR_ELAUNCH;
}

int32_t inet_nr_dl_reset(const InetNrDlState* dl, const InetNrParams* prm, const uint8_t* mask, void* stream) {
    if (!dl || !prm) return INET_NR_EINVAL;
    const InetNrParams& p = *prm;
    if (p.E <= 0 || p.R <= 0 || p.S > INET_NR_MAX_S || p.P > INET_NR_MAX_P) return INET_NR_EINVAL;
    hipLaunchKernelGGL(nr_dl_reset_kernel, dim3(p.E), dim3(64), 0, (hipStream_t)stream, *dl, p, mask, mask ? 0 : 1);
    return hipGetLastError() == hipSuccess ? INET_NR_OK : INET_NR_ELAUNCH;
}

int32_t inet_nr_submit(const InetNrState* st, const InetNrParams* prm, int64_t T, const int64_t* send,
                       const uint8_t* det, const int64_t* hid, const uint8_t* counts, int32_t n_cls,
                       const float* sizes, int32_t discard_pdcp, int32_t pkt_payload, int32_t pkt_overhead,
                       void* accepted, void* stream) {
    if (!st || !prm || !sizes || (!send && !counts) || (send && counts)) return INET_NR_EINVAL;
    if (!counts && !accepted) return INET_NR_EINVAL;
    if (counts && n_cls <= 0) return INET_NR_EINVAL;
    if ((T < 0 && !st->clock) || T > 0x7fffffff || (pkt_overhead && pkt_payload <= 0)) return INET_NR_EINVAL;
    const InetNrParams& p = *prm;
    int n = p.E * p.R;
    hipLaunchKernelGGL(nr_submit_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, *st, p.E, p.R,
                       p.F, T, send, det, hid, counts, n_cls, sizes, discard_pdcp, p.timeout, pkt_payload,
                       pkt_overhead, accepted);
    return hipGetLastError() == hipSuccess ? INET_NR_OK : INET_NR_ELAUNCH;
}

int32_t inet_nr_reset(const InetNrState* st, const InetNrParams* prm, const uint8_t* mask, int64_t T, float k_lin0,
                      const float* dcorr, int32_t spectrum, void* stream) {
    if (!st || !prm || !dcorr) return INET_NR_EINVAL;
    const InetNrParams& p = *prm;
    if (p.E <= 0 || p.R <= 0 || p.n_fields < 0 || p.n_fields > 3 || p.n_modes > INET_NR_MAX_KF) return INET_NR_EINVAL;
    if (p.n_cells > INET_NR_MAX_C) return INET_NR_EINVAL;
    if (p.fc_on < 0 || p.fc_on > 2 || (p.fc_on == 1 && !p.fc_L) ||
        (p.fc_on == 2 && (!p.fc_tab || p.fc_G < 1 || !st->fc_idx || !st->fc_idl || !st->fc_idn)))
        return INET_NR_EINVAL;
    if (T < 0 || T > 0x7fffffff ||
        (p.k_from_los && (!st->k_los || !st->k_from || !st->k_g0 || !st->k_fresh || !p.rician)))
        return INET_NR_EINVAL;
    if (p.doppler && !st->has_prev) return INET_NR_EINVAL;
    hipLaunchKernelGGL(nr_reset_kernel, dim3(p.E), dim3(64), 0, (hipStream_t)stream, *st, p, mask, (int)T, k_lin0,
                       dcorr[0], dcorr[1], dcorr[2], spectrum, mask ? 0 : 1);
    return hipGetLastError() == hipSuccess ? INET_NR_OK : INET_NR_ELAUNCH;
}

}  // extern "C"

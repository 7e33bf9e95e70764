// MI355X (gfx950) kernels of isaac-net's level "WIFI" (the mean-field 802.11 uplink at one access point) and the C
// ABI of include/inet_wifi.h.
//
// wifi_step_kernel runs one whole control step per env: the SNR of each robot (poses through the AP's radio, or the
// SNR / received power given), its MCS, the K sub-steps of WifiNet._serve (isaac_net/core/wifi/engine.py:292-403) and
// the end of step of finish_body (proto/netsim_fast.py:185-206), reading and writing each env's state once.
//
// Work decomposition: one workgroup is one wavefront; one robot per lane; the RB = next_pow2(R) lanes of an env form
// an aligned segment, and a wave holds G envs (G RB <= 64; a launch parameter: fewer envs per wave give more waves,
// which hides the latency of the serial sub-step chain). The AP's background station is segment-uniform: every lane
// of the env computes it. The mean-field sums over the stations of the domain (meanfield.SingleView.sum) run over
// an LDS row in torch's CPU summation order (aten_row_sum), so that only the transcendental functions differ from
// the CPU path; those are evaluated in double precision and rounded once. The FIFO of each robot lives in LDS
// columns during the step ([F][64] floats).
//
// Per sub-step and lane: q = sum of the FIFO bytes; contention flag; AC parameters and the access's bytes B; the
// channel times Ts, Tc (wifi/phy.py:141-155); fp_iters + 1 evaluations of the failure probability (one LDS row sum
// each) and the damped update of tau (tau(p) of meanfield.py:55-62 over the max_tx backoff stages); the slot time
// (four row sums); the access count (Poisson inverse CDF over a double-precision running sum, or the renewal credit);
// the FIFO service with each frame's finish time and retry-limit loss draw.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/inet_wifi.h"
#include "inet_nr_dev.h"

using namespace inet;

namespace {

constexpr int WAVE = 64;
constexpr uint32_t CH_STEP = 2;

// transcendental functions evaluated in double precision and rounded once to float32
DEV float exp_r(float x) { return (float)exp((double)x); }
DEV float log_r(float x) { return (float)log((double)x); }
DEV float log1p_r(float x) { return (float)log1p((double)x); }
DEV float pow_r(float x, float y) { return (float)pow((double)x, (double)y); }
// x ** n for a Python int exponent n (torch pow with a scalar: 1 copies, 2 and 3 multiply, others pow)
DEV float pow_int_torch(float x, int n) {
    if (n == 1) return x;
    if (n == 2) return x * x;
    if (n == 3) return (x * x) * x;
    return pow_count(x, (float)n);
}
// p ** k of tau(p) (torch pow of two float tensors) for an integer k >= 0: double-precision binary powering,
// rounded once
DEV float pow_k(float p, int k) { return pow_count(p, (float)k); }
DEV float fminn(float a, float b) { return a != a ? a : (b != b ? b : (a < b ? a : b)); }   // torch.minimum

// AccessTiming.cap_bytes (wifi/phy.py:130-139): application bytes one access carries
DEV float cap_bytes(const InetWifiParams& pm, float rate, float txop) {
    if (pm.no_aggr) return pm.msdu_payload;
    float tmax = txop > 0.f ? clamp_max(txop, pm.ppdu_max) : pm.ppdu_max;
    float by_time = (((tmax - pm.pre) * rate) / 8.0f) / pm.ovh1;
    return clamp_min(clamp_max(by_time, pm.ampdu_lim), pm.msdu_payload);
}
// AccessTiming.times (wifi/phy.py:141-155): (Ts, Tc) in us of an access of B bytes at rate after AIFSN aifsn
DEV void access_times(const InetWifiParams& pm, float B, float rate, float aifsn, float& ts, float& tc) {
    float aifs = aifsn * pm.slot_us + pm.sifs_us;
    float nsym = ceilf(((B * pm.ovh1) * 8.0f + 22.0f) / (rate * pm.tsym));
    float tdata = pm.tsym * nsym + pm.pre;
    if (pm.rts_cts) {
        ts = (((aifs + pm.hs) + tdata) + pm.sifs_us) + pm.t_ack;
        tc = ((aifs + pm.t_rts) + pm.sifs_us) + pm.t_cts;
    } else {
        ts = ((aifs + tdata) + pm.sifs_us) + pm.t_ack;
        tc = pm.coll_ack ? ts : aifs + tdata;
    }
}
// the vulnerable period Tv of a hidden-node collision (wifi/phy.py:150, 154): the RTS, or the data PPDU
DEV float vuln_time(const InetWifiParams& pm, float B, float rate) {
    if (pm.rts_cts) return pm.t_rts;
    const float nsym = ceilf(((B * pm.ovh1) * 8.0f + 22.0f) / (rate * pm.tsym));
    return pm.tsym * nsym + pm.pre;
}
// tau(p) of meanfield.tau_from_p: sum_k p^k / sum_k p^k (W_k + 1) / 2 over the L stages, W_k = min(2^k W0, Wmax),
// both sums in torch's CPU order. p^k is the double-precision running product rounded once (the correctly rounded
// power unless p^k lies within ~k 2^-53 relative of a float rounding boundary). Under 8 stages the CPU order adds
// stages 0..3 into four partial sums and the later stages into the first, so one pass over k in order suffices.
// the stage weights (W_k + 1) / 2, W_k = min(2^k W0, Wmax), of the first 7 stages (2^k W0 by doubling, exact)
struct TauW {
    float c[7];
};
DEV TauW tau_weights(float W0, float Wm) {
    TauW t;
    float wk = W0;
#pragma unroll
    for (int k = 0; k < 7; ++k) {
        t.c[k] = (fminn(wk, Wm) + 1.0f) * 0.5f;
        wk = wk * 2.0f;
    }
    return t;
}
DEV float tau_of_p(float p, float W0, float Wm, int L, const TauW& tw) {
    if (L < 8) {
        // (unrolled to the 7-stage bound; the stage terms are the running product's, and the four partial sums take
        // stages 0..3 one each and the later ones into the first when L >= 4, every stage into the first below 4)
        const double pd = (double)p;
        float pk[7], tk[7];
        double pw = 1.0;
#pragma unroll
        for (int k = 0; k < 7; ++k) {
            pk[k] = (float)pw;
            pw *= pd;
            tk[k] = pk[k] * tw.c[k];
        }
        float n0, n1 = 0.f, n2 = 0.f, n3 = 0.f, d0, d1 = 0.f, d2 = 0.f, d3 = 0.f;
        if (L >= 4) {
            n0 = pk[0]; n1 = pk[1]; n2 = pk[2]; n3 = pk[3];
            d0 = tk[0]; d1 = tk[1]; d2 = tk[2]; d3 = tk[3];
#pragma unroll
            for (int k = 4; k < 7; ++k)
                if (k < L) { n0 += pk[k]; d0 += tk[k]; }
        } else {
            n0 = pk[0]; d0 = tk[0];
#pragma unroll
            for (int k = 1; k < 3; ++k)
                if (k < L) { n0 += pk[k]; d0 += tk[k]; }
        }
        return (((n0 + n1) + n2) + n3) / (((d0 + d1) + d2) + d3);
    }
    float num = aten_row_sum(L, [&](int k) { return pow_k(p, k); });
    float den = aten_row_sum(L, [&](int k) {
        float wk = fminn(W0 * exp2f((float)k), Wm);
        return pow_k(p, k) * ((wk + 1.0f) * 0.5f);
    });
    return num / den;
}

// U{0..W-1} from an element hash: ((h >> 8) W) >> 24
DEV int draw_int(uint32_t h, int W) { return (int)(((uint64_t)(h >> 8) * (uint64_t)W) >> 24); }
// channel time (ns) of an access of B bytes: the busy period of a lone transmission (success or FER loss) and of a
// collision (wifi/eventsim.py:140-152 with the AccessTiming exchange of wifi/phy.py:141-155, integer nanoseconds)
DEV void dcf_busy(const InetWifiParams& pm, const InetDcfParams& dp, int B, int nd, int& succ, int& coll) {
    const int nmsdu = (B + dp.payload - 1) / dp.payload;
    const int bits = 22 + 8 * B + 8 * dp.ovh * nmsdu;
    const int tdata = dp.pre + dp.tsym * ((bits + nd - 1) / nd);
    if (pm.rts_cts) {
        succ = dp.t_rts + dp.sifs + dp.t_cts + dp.sifs + tdata + dp.sifs + dp.t_ack;
        coll = dp.t_rts + dp.sifs + dp.t_cts;
    } else {
        succ = tdata + dp.sifs + dp.t_ack;
        coll = pm.coll_ack ? succ : tdata;
    }
}

// One submit call of class cls (0: none) by each robot lane (add_body, proto/netsim_fast.py:136-160): the message
// takes FIFO slot qlen unless the FIFO is full; f_nact records how many robots of the env hold a message after the
// call. Convergent over the env's segment (a ballot).
DEV bool fifo_call(const InetWifiState& st, const InetWifiParams& pm, bool rob, int cls, int& qlen, size_t fo,
                   int64_t t, bool dt, int64_t hid, float snr, int rb, int lane) {
    const bool nw = rob && cls > 0 && qlen < pm.F;
    const int nact = __builtin_popcountll(__ballot(rob && (qlen + (nw ? 1 : 0)) > 0) & seg_bits(rb, lane));
    if (nw) {
        const size_t o = fo + (size_t)qlen * pm.R;
        const int c = cls < pm.n_cls ? cls : pm.n_cls;
        st.cap[o] = (int32_t)t;
        st.cls[o] = cls;
        st.det[o] = dt;
        st.hid[o] = (int32_t)hid;
        st.rem[o] = pm.sizes[c - 1];
        st.f_nact[o] = nact;
        st.f_snr[o] = snr;
        st.f_own[o] = qlen;
        ++qlen;
    }
    return nw;
}

// The counts form's calls as seen by the env of this lane's segment: class 1 first, one call per message index up to
// the env's largest count of the class (the later calls change nothing of the env). Returns the messages accepted for
// this robot; calls = the env's number of calls (segment-uniform).
DEV int fifo_counts(const InetWifiState& st, const InetWifiParams& pm, const uint8_t* __restrict__ counts, int n_cls,
                    bool rob, size_t ir, int& qlen, size_t fo, int64_t t, bool dt, int64_t hid, float snr, int rb,
                    int lane, int& calls) {
    int n_acc = 0;
    calls = 0;
    for (int c = 0; c < n_cls; ++c) {
        const int mine = rob ? counts[ir * n_cls + c] : 0;
        const int most = seg_max_i(mine, rb);
        for (int i = 0; i < most; ++i)
            n_acc += fifo_call(st, pm, rob, mine > i ? c + 1 : 0, qlen, fo, t, dt, hid, snr, rb, lane) ? 1 : 0;
        calls += most;
    }
    return n_acc;
}

// The sum over the stations of one collision domain as the reference's DomainView.sum forms it
// (wifi/meanfield.py:76-89: onehot^T x, then onehot times that, two batched products small enough for ATen's CPU
// kernel, which accumulates products in index order): the members' values added in station order. (Each product is
// 1 x or 0 x, exact, and adding a zero leaves a non-zero sum unchanged.)
DEV float dom_seq_sum(const float* row, const uint8_t* dom, int n, int d) {
    float acc = 0.f;
    for (int i = 0; i < n; ++i) acc = dom[i] == d ? acc + row[i] : acc;
    return acc;
}

// the sum over the stations of a mask (MatrixView.sum, meanfield.py:98-99: V @ x with V of 0 / 1, added in index
// order by ATen's CPU product kernel at (R + A)^2 < 400)
DEV float mask_seq_sum(const float* row, uint64_t mask, int n) {
    float acc = 0.f;
    for (int i = 0; i < n; ++i) acc = ((mask >> i) & 1ull) ? acc + row[i] : acc;
    return acc;
}

// bytewise maximum of two words of four uint8
DEV uint32_t max_u8x4(uint32_t a, uint32_t b) {
    uint32_t m = 0;
#pragma unroll
    for (int k = 0; k < 32; k += 8) {
        const uint32_t x = (a >> k) & 0xffu, y = (b >> k) & 0xffu;
        m |= (x > y ? x : y) << k;
    }
    return m;
}

// The global part of the counts form, run by one workgroup: the calls of every class number its largest count over
// every env and robot, and each call advances every env's SUBMIT call counter (the global word st.calls) and, with
// set_hid, sets its last hazard id to 0. s_max: n_cls ints of LDS. 16-byte loads, sixteen in flight per lane; with
// n_cls dividing 16 each byte position of a load holds one class, so every lane keeps a running maximum per byte
// position; at the end each class's maximum is reduced over the lane's positions and over the wave (shuffles), and
// lane 0 takes one LDS maximum per class (LDS atomics of every lane on one word serialize).
DEV void submit_calls(const InetWifiState& st, int E, const uint8_t* __restrict__ counts, size_t n, int n_cls,
                      int* s_max, bool set_hid) {
    const int tid = threadIdx.x, nt = blockDim.x;
    if (tid < n_cls) s_max[tid] = 0;
    __syncthreads();
    const bool vec = ((uintptr_t)counts & 15u) == 0u && 16 % n_cls == 0;
    const size_t n16 = vec ? n / 16 : 0;
    const uint4* c4 = reinterpret_cast<const uint4*>(counts);
    uint32_t m0 = 0, m1 = 0, m2 = 0, m3 = 0;
    constexpr int U = 16;
    size_t j = tid;
    for (; j + (size_t)(U - 1) * nt < n16; j += (size_t)U * nt) {
        uint4 w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) w[u] = c4[j + (size_t)u * nt];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            m0 = max_u8x4(m0, w[u].x); m1 = max_u8x4(m1, w[u].y); m2 = max_u8x4(m2, w[u].z); m3 = max_u8x4(m3, w[u].w);
        }
    }
    for (; j < n16; j += nt) {
        const uint4 w = c4[j];
        m0 = max_u8x4(m0, w.x); m1 = max_u8x4(m1, w.y); m2 = max_u8x4(m2, w.z); m3 = max_u8x4(m3, w.w);
    }
    if (n16) {
        const uint32_t ws[4] = {m0, m1, m2, m3};
        for (int c = 0; c < n_cls; ++c) {
            int v = 0;
#pragma unroll
            for (int b = 0; b < 16; ++b) {
                const int x = (int)((ws[b >> 2] >> (8 * (b & 3))) & 0xffu);
                v = (b % n_cls == c && x > v) ? x : v;
            }
#pragma unroll
            for (int o = WAVE / 2; o > 0; o >>= 1) {
                const int w = __shfl_xor(v, o, WAVE);
                v = w > v ? w : v;
            }
            if ((tid & (WAVE - 1)) == 0 && v > 0) atomicMax(&s_max[c], v);
        }
    }
    for (size_t i = 16 * n16 + tid; i < n; i += nt) {
        const int v = counts[i];
        if (v > 0) atomicMax(&s_max[i % (size_t)n_cls], v);
    }
    __syncthreads();
    int tot = 0;
    for (int c = 0; c < n_cls; ++c) tot += s_max[c];
    if (tot > 0 && tid == 0) st.calls[0] += tot;
    if (tot > 0 && set_hid)
        for (int e = tid; e < E; e += nt) st.last_hid[e] = 0;
}

}  // namespace

// ======================================================================================= step kernel
// DCF = false: the mean-field level (WifiNet._serve); true: the per-slot CSMA/CA level (integer backoff counters).
// MA: several APs (pm.A > 1); the one-AP build fixes A = 1, which keeps the station count R + 1 a compile-time
// offset of R (measured: the general count costs a fifth of the one-AP step through register allocation).
// CNT: the launch enqueues pm.step_counts first (a build of its own, so that the step without it keeps its register
// allocation). ZN: AIFS zones (pm.Z > 1; with MA, every station in a lane of its own).
template <bool DCF, bool MA = false, bool CNT = false, bool ZN = false>
__global__ __launch_bounds__(WAVE) void wifi_step_kernel(InetWifiState st, InetWifiParams pm,
                                                         const int64_t* __restrict__ tin, int input_kind,
                                                         const float* __restrict__ xin,
                                                         const int64_t* __restrict__ hid_in, InetWifiOutputs out,
                                                         int rb, InetDcfState ds, InetDcfParams dp) {
    extern __shared__ float dyn[];
    __shared__ __align__(16) float s_red[WAVE];
    __shared__ __align__(16) float s_red4[DCF ? 1 : 3 * WAVE];          // three more rows of station values (dom_sum4)
    __shared__ uint8_t s_hid0[CNT ? WAVE : 1];            // per env: the enqueue's calls clear the last hazard id
    __shared__ int s_cmax[CNT ? INET_WIFI_MAX_CLS : 1];   // the largest count of every class (workgroup 0)
    __shared__ uint8_t s_dom[MA ? WAVE : 1];              // APs on several channels: each station's domain
    __shared__ float s_rxa[ZN ? WAVE * INET_WIFI_MAX_A : 1];   // hidden nodes: every robot's power at every AP
    __shared__ float s_pos[ZN ? 2 * WAVE : 1];                  // hidden nodes: every robot's position
    const int R = pm.R, F = pm.F, K = pm.K, L = pm.L, G = pm.envs_per_wave;
    float* s_rem = dyn;                                   // [F][64] bytes left of every frame slot
    float* s_fin = dyn + F * WAVE;                        // [F][64] finish time, then the compaction staging row
    uint8_t* s_cls = (uint8_t*)(dyn + 2 * F * WAVE);      // [F][64] class of every frame slot
    uint8_t* s_src = s_cls + F * WAVE;                    // [F][64] source slot of every compacted slot
    int32_t* s_stage = (int32_t*)s_fin;

    const int lane = threadIdx.x;
    const int g = lane / rb, r = lane - g * rb;
    const int e = blockIdx.x * G + g;
    const bool env_ok = g < G && e < pm.E;
    const bool rob = env_ok && r < R;
    const int ec = env_ok ? e : 0, rc = rob ? r : 0;
    const int gseg = g < G ? g : 0;
    const size_t ir = (size_t)ec * R + rc;                 // [E][R]
    const size_t fo = (size_t)ec * F * R + rc;             // [E][F][R] slot f at fo + f R

    const int64_t t = env_ok ? (tin ? tin[ec] : st.clock[ec]) : 0;
    // ---------------- the control step's enqueue (the counts form of submit, before anything else is live) ----------
    if constexpr (CNT) {
        int qlen = rob ? st.qlen[ir] : 0, calls;
        const int na = fifo_counts(st, pm, pm.step_counts, pm.step_n_cls, rob, ir, qlen, fo, t, false, 0,
                                   rob ? st.last_snr[ir] : 0.f, rb, lane, calls);
        if (rob) {
            st.qlen[ir] = qlen;
            if (pm.step_accepted) pm.step_accepted[ir] = na;
        }
        // the calls clear every env's last hazard id: known from the env's own calls, else (an env with a hazard id
        // and nothing to send) from a scan of every count for any message
        bool any = calls > 0;
        if (!any && env_ok && st.last_hid[ec] != 0) {
            const size_t n = (size_t)pm.E * R * pm.step_n_cls;
            bool mine = false;
            for (size_t j = r; j < n && !mine; j += rb) mine = pm.step_counts[j] != 0;
            any = seg_any(mine, rb, lane);
        }
        if (env_ok && r == 0) s_hid0[gseg] = any;
    }

    // ---------------- inputs, association, MCS (wifi/engine.py:227-259, 295-299) ----------------
    // the received power at every AP (poses through the APs' radio, the SNR to the one AP, or rx_dbm [E][R][A]); the
    // strongest AP after a reset, else a roam to an AP stronger than the serving one by roam_hyst (the first of equal
    // maxima), which starts the roaming interruption
    const int A = MA ? pm.A : 1;
    float rx = 0.f;
    int sv = 0;
    bool roamed = false;
    if (rob) {
        const int s0 = st.serv[ir];
        const bool pend = st.pending[ec] != 0;
        float bv = 0.f, cur = 0.f;
        int best = 0;
        const float px = input_kind == 0 ? xin[ir * 2] : 0.f, py = input_kind == 0 ? xin[ir * 2 + 1] : 0.f;
        if constexpr (ZN) { s_pos[2 * lane] = px; s_pos[2 * lane + 1] = py; }
        const StoLos sto{pm.los_cdf, pm.plos_scn, pm.sig_nlos, pm.los_sto != 0};
        for (int c = 0; c < A; ++c) {
            float v;
            if (input_kind == 0)
                v = radio_rx_dbm(pm, px, py, pm.ap_xy[2 * c], pm.ap_xy[2 * c + 1],
                                 st.field + ((size_t)ec * A + c) * pm.n_fields * pm.n_modes * 3, sto);
            else if (input_kind == 1)
                v = xin[ir] + pm.noise_dbm;
            else
                v = xin[ir * A + c];
            if (c == 0 || v > bv) { bv = v; best = c; }
            if (c == s0) cur = v;
            if constexpr (ZN) s_rxa[lane * INET_WIFI_MAX_A + c] = v;
        }
        const bool better = bv > cur + pm.roam_hyst;
        roamed = better && !pend && best != s0;
        sv = (pend || roamed) ? best : s0;
        rx = sv == s0 ? cur : bv;
    }
    const float snr = rx - pm.noise_dbm;
    int nm = 0;
    for (int m = 0; m < pm.M; ++m) nm += snr >= pm.thr[m] ? 1 : 0;
    const bool link = nm > 0;
    const int mcs = nm > 0 ? nm - 1 : 0;
    const float rate = pm.rates[mcs];

    // ---------------- state ----------------
    int qlen = rob ? st.qlen[ir] : 0;
    for (int f = 0; f < F; ++f) {
        const int o = f * WAVE + lane;
        s_rem[o] = rob && f < qlen ? st.rem[fo + (size_t)f * R] : 0.f;
        s_cls[o] = rob ? (uint8_t)st.cls[fo + (size_t)f * R] : 0;
        s_fin[o] = INFINITY;
    }
    // counter-RNG keys of this step: the step counter advances before the draws (LevelNet._advance)
    const int ctr = env_ok ? st.ctr_step[ec] + 1 : 0;
    uint32_t hkey = 0;
    if (env_ok) {
        uint32_t h = mix32((uint32_t)pm.seed_key ^ salt32((uint32_t)st.env_id[ec]));
        h = mix32(h ^ salt32((uint32_t)st.episode[ec]));
        h = mix32(h ^ salt32(CH_STEP));
        hkey = mix32(h ^ salt32((uint32_t)ctr));
    }
    const uint32_t key_acc = mix32(hkey ^ salt32(0u)), key_loss = mix32(hkey ^ salt32(1u));
    // EDCA parameters: the class-1 AC for every robot, or the head-of-line message's AC per sub-step
    int ac = pm.cls_ac[1];
    float capB = cap_bytes(pm, rate, pm.ac_txop[ac]);
    float o_acc = NAN, o_pf = NAN, o_busy = 0.0f;       // wifi_access_ms, wifi_p_fail, wifi_busy
    // (the row sums read LDS: aten_row_sum_u issues every read before the first add)
    auto fifo_sum = [&]() -> float {
        auto xf = [&](int f) { return s_rem[f * WAVE + lane]; };
        if (F == 16) return aten_row_sum_u<16>(16, xf);
        if (F <= 16) return aten_row_sum_u<16>(F, xf);
        if (F <= 32) return aten_row_sum_u<32>(F, xf);
        if (F <= 64) return aten_row_sum_u<64>(F, xf);
        return aten_row_sum(F, xf);
    };
    if constexpr (!DCF) {
    // The APs' background stations are stations R .. R + A - 1 of the domain (identical: the same weight, window,
    // times and start, so the same tau). With lanes to spare in the segment (rb >= R + A) each runs in its lane like
    // a robot (nothing else), else every lane evaluates one and the sums count it A times.
    const int NS = R + A;                                  // stations of the domain: robots, one per AP
    const bool bgl = rb >= NS;
    const bool is_bg = bgl && env_ok && r >= R && r < NS;
    // APs on several channels (MA builds): one collision domain per channel. A robot is in its serving AP's channel,
    // an AP's background station in the AP's (each has its own lane: R + A <= 64, checked by the entry points).
    const bool hid = ZN && pm.hidden != 0;
    const bool doms = MA && (pm.n_dom > 1 || hid);
    if (doms) {
        if (env_ok && r < NS) s_dom[lane] = (uint8_t)(r < R ? pm.ap_dom[sv] : pm.ap_dom[r - R]);
        __syncthreads();
    }
    const int mydom = doms && env_ok && r < NS ? s_dom[lane] : 0;
    // hidden nodes (WifiNet._sensing, wifi/engine.py:260-282): this station's row of V (the stations it senses: its
    // domain's, and among robots those whose power at it, robot-robot path loss, reaches the CCA threshold, or
    // pm.sense) and of H (robots of its domain it does not sense whose power at its AP reaches the threshold)
    uint64_t vmask = 0ull, hmask = 0ull;
    if (hid && env_ok && r < NS) {
        const int sb = gseg * rb;
        for (int j = 0; j < NS; ++j) {
            const bool same = s_dom[sb + j] == mydom;
            bool sensed = true;
            if (r < R && j < R && j != r) {
                if (pm.sense) {
                    sensed = pm.sense[((size_t)ec * R + r) * R + j] != 0;
                } else if (input_kind == 0) {
                    const float dx = s_pos[2 * lane] - s_pos[2 * (sb + j)];
                    const float dy = s_pos[2 * lane + 1] - s_pos[2 * (sb + j) + 1];
                    const float dist = fmaxf(sqrtf(fmaf(dy, dy, dx * dx)), 1.0f);        // (torch's norm of two)
                    const float prx = pm.sta_c0 - pm.sta_c1 * (float)log10((double)dist);
                    sensed = prx >= pm.cca_dbm;
                }
                if (same && !sensed && s_rxa[(sb + j) * INET_WIFI_MAX_A + sv] >= pm.cca_dbm) hmask |= 1ull << j;
            }
            if (same && (r >= R || j >= R || sensed)) vmask |= 1ull << j;
        }
    }
    float tau = rob ? st.tau[(size_t)ec * NS + rc] : (is_bg ? st.tau[(size_t)ec * NS + r] : pm.tau0);
    float tau_b = (!bgl && env_ok) ? st.tau[(size_t)ec * NS + R] : pm.tau0;
    int roam = rob ? st.roam_left[ir] : 0;
    if (roamed && pm.roam_sub > 0) roam = pm.roam_sub;
    float att_n = rob ? st.att_n[ir] : 0.f, att_logp = rob ? st.att_logp[ir] : 0.f;
    float credit = rob ? st.credit[ir] : 0.f;

    float W0 = pm.ac_W0[ac], Wm = pm.ac_Wmax[ac], aifsn = pm.ac_aifsn[ac];
    // the background station (segment-uniform)
    const float W0b = pm.ac_W0[pm.bg_ac], Wmb = pm.ac_Wmax[pm.bg_ac];
    float tsb, tcb;
    access_times(pm, pm.bg_B, pm.bg_rate, pm.ac_aifsn[pm.bg_ac], tsb, tcb);
    const float wb = pm.bg_w;
    const bool act_b = wb > 0.f;
    const TauW twb = tau_weights(W0b, Wmb);

    // sum over the R + A stations of the env (robots in lane order, then the APs' background stations, which all hold
    // the same values: lane R's, or vb without a spare lane), torch's CPU order. (dom_sum and dom_sum4 each keep
    // their own copy of the row sum: one shared helper made the compiler spill to scratch.)
    auto dom_sum = [&](float v, float vb) -> float {
        __syncthreads();
        s_red[lane] = v;
        __syncthreads();
        const float* row = s_red + gseg * rb;
        if (hid) return mask_seq_sum(row, vmask, NS);
        if (doms) return dom_seq_sum(row, s_dom + gseg * rb, NS, mydom);
        if (NS == 17 && bgl) {          // (a 32-lane segment: the row is 128-byte aligned, read 16 bytes at a time)
            float v[17];
            const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 q = r4[k];
                v[4 * k] = q.x; v[4 * k + 1] = q.y; v[4 * k + 2] = q.z; v[4 * k + 3] = q.w;
            }
            v[16] = row[16];
            return aten_row_sum_u<17>(17, [&](int i) { return v[i]; });
        }
        auto xr = [&](int i) { return (i < R || bgl) ? row[i] : vb; };
        if (NS == 17) return aten_row_sum_u<17>(17, xr);
        if (NS <= 8) return aten_row_sum_u<8>(NS, xr);
        if (NS <= 16) return aten_row_sum_u<16>(NS, xr);
        if (NS <= 33) return aten_row_sum_u<33>(NS, xr);
        return aten_row_sum_u<65>(NS, xr);                  // (R + A <= 65: checked by the entry points)
    };

    // four such sums at once (one LDS round trip): rows s_red and s_red4[0..2]
    auto dom_sum4 = [&](float v0, float b0, float v1, float b1, float v2, float b2, float v3, float b3, float& o0,
                        float& o1, float& o2, float& o3) {
        __syncthreads();
        s_red[lane] = v0; s_red4[lane] = v1; s_red4[WAVE + lane] = v2; s_red4[2 * WAVE + lane] = v3;
        __syncthreads();
        auto sum_row = [&](const float* base, float vb) -> float {
            const float* row = base + gseg * rb;
            if (hid) return mask_seq_sum(row, vmask, NS);
            if (doms) return dom_seq_sum(row, s_dom + gseg * rb, NS, mydom);
            if (NS == 17 && bgl) {          // (a 32-lane segment: the row is 128-byte aligned, read 16 bytes at a time)
                float v[17];
                const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 q = r4[k];
                    v[4 * k] = q.x; v[4 * k + 1] = q.y; v[4 * k + 2] = q.z; v[4 * k + 3] = q.w;
                }
                v[16] = row[16];
                return aten_row_sum_u<17>(17, [&](int i) { return v[i]; });
            }
            auto xr = [&](int i) { return (i < R || bgl) ? row[i] : vb; };
            if (NS == 17) return aten_row_sum_u<17>(17, xr);
            if (NS <= 8) return aten_row_sum_u<8>(NS, xr);
            if (NS <= 16) return aten_row_sum_u<16>(NS, xr);
            if (NS <= 33) return aten_row_sum_u<33>(NS, xr);
            return aten_row_sum_u<65>(NS, xr);
        };
        o0 = sum_row(s_red, b0);
        o1 = sum_row(s_red4, b1);
        o2 = sum_row(s_red4 + WAVE, b2);
        o3 = sum_row(s_red4 + 2 * WAVE, b3);
    };

    // the smallest value over the stations of this lane's domain (SingleView.min / DomainView.min, meanfield.py:71-73,
    // 86-89: 1e9 stands for excluded stations; exact in any order)
    auto dom_min = [&](float v) -> float {
        __syncthreads();
        s_red[lane] = v;
        __syncthreads();
        const float* row = s_red + gseg * rb;
        float m = 1e9f;
        for (int i = 0; i < NS; ++i)
            if (hid ? ((vmask >> i) & 1ull) != 0ull : (!doms || s_dom[gseg * rb + i] == mydom)) m = fminn(m, row[i]);
        return m;
    };
    // two sums over this station's hidden set (H @ x, meanfield.py:170; rows s_red and s_red4)
    auto hid_sum2 = [&](float v0, float v1, float& o0, float& o1) {
        __syncthreads();
        s_red[lane] = v0;
        s_red4[lane] = v1;
        __syncthreads();
        o0 = mask_seq_sum(s_red + gseg * rb, hmask, NS);
        o1 = mask_seq_sum(s_red4 + gseg * rb, hmask, NS);
    };

    float acc_sum = 0.f, acc_n = 0.f, p_sum = 0.f, busy_sum = 0.f;
    const float tf = (float)t;
    for (int k = 0; k < K; ++k) {
        const float q = fifo_sum();
        const bool act = rob && q > 0.f && link && roam <= 0;
        if (pm.per_class_ac) {
            int hol = 0;
            for (int f = qlen - 1; f >= 0; --f) hol = s_rem[f * WAVE + lane] > 0.f ? f : hol;
            const int ch = s_cls[hol * WAVE + lane];
            ac = pm.cls_ac[ch < pm.n_cls ? ch : pm.n_cls];
            W0 = pm.ac_W0[ac]; Wm = pm.ac_Wmax[ac]; aifsn = pm.ac_aifsn[ac];
            capB = cap_bytes(pm, rate, pm.ac_txop[ac]);
        }
        const float B = act ? fminn(q, capB) : capB;
        const float w = act ? 1.0f : 0.0f;
        float ts, tc;
        // AIFS zones (wifi/engine.py:344-348): each station's offset from the smallest AIFSN among the contending
        // stations of its domain, whose AIFS the channel times then use
        float aif_t = aifsn, d_s = 0.0f, tsbz = tsb, tcbz = tcb;
        float tv_s = 0.0f;
        if constexpr (ZN) {
            const float aif_s = is_bg ? pm.ac_aifsn[pm.bg_ac] : aifsn;
            const bool on = is_bg ? act_b : act;
            aif_t = fminn(dom_min(on ? aif_s : 1e9f), aif_s);
            d_s = aif_s - aif_t;
            if (is_bg) access_times(pm, pm.bg_B, pm.bg_rate, aif_t, tsbz, tcbz);
            if (hid) tv_s = is_bg ? vuln_time(pm, pm.bg_B, pm.bg_rate) : vuln_time(pm, B, rate);
        }
        access_times(pm, B, rate, aif_t, ts, tc);
        // this lane's station in the solve: the robot's, or in lane R the background station's
        const float ws = is_bg ? wb : w, tss = is_bg ? tsbz : ts, tcs = is_bg ? tcbz : tc;
        const float W0s = is_bg ? W0b : W0, Wms = is_bg ? Wmb : Wm;
        const bool acts = is_bg ? act_b : act;
        const TauW tw = tau_weights(W0s, Wms);

        // ---- mean-field fixed point (meanfield.solve, one domain, one AIFS zone)
        float p = 0.f, ok = 0.f, pb = 0.f, S = 0.f;
        // (the iterations' log1p and exp in float32, the device library's, within 2 ulp: the fixed point carries
        // last-bit differences from the CPU's float routines either way, and the tests bound them at 2e-5 relative)
        auto fail = [&]() {
            const float lt = log1pf(-tau), ltb = bgl ? 0.0f : log1pf(-tau_b);
            S = dom_sum(ws * lt, wb * ltb);
            const float own = acts ? lt : 0.0f;
            ok = expf(S - own) * pm.fer1;
            p = 1.0f - ok;
            if (!bgl) {
                const float ownb = act_b ? ltb : 0.0f;
                pb = 1.0f - expf(S - ownb) * pm.fer1;
            }
        };
        // zones (meanfield._zones / _fail, meanfield.py:106-131, 161-178): per zone z the domain sum of w log(1 - tau)
        // over the stations with offset <= z, the stationary zone distribution, and the success and failure
        // probabilities weighted by the zones the station counts down in
        constexpr int ZX = ZN ? INET_WIFI_MAX_Z : 1;
        float Sz[ZX], piz[ZX], num = 0.0f;
        auto failz = [&]() {
            const float lt = log1pf(-tau), wl = ws * lt;
#pragma unroll
            for (int z = 0; z < ZX; ++z)
                if (z < pm.Z) Sz[z] = dom_sum(d_s <= (float)z ? wl : 0.0f, 0.0f);
            float g = 1.0f, raw[ZX], tot = 0.0f;
#pragma unroll
            for (int z = 0; z < ZX; ++z)
                if (z < pm.Z) {
                    const float idle = expf(Sz[z]);
                    raw[z] = z < pm.Z - 1 ? g : g / clamp_min(1.0f - idle, 1e-12f);
                    g = g * idle;
                }
#pragma unroll
            for (int z = 0; z < ZX; ++z) if (z < pm.Z) tot = tot + raw[z];
#pragma unroll
            for (int z = 0; z < ZX; ++z) if (z < pm.Z) piz[z] = raw[z] / tot;
            // hidden nodes: exp(-(Tv_i sum_H rate + sum_H rate Tv)), rate = w tau open / Tslot (meanfield.py:167-170)
            float hf = 1.0f;
            if (hid) {
                const float r_h = (ws * tau) / (1.0f - tau), wt_h = ws * tau;
                float tsl = 0.0f, opn = 0.0f;
#pragma unroll
                for (int z = 0; z < ZX; ++z)
                    if (z < pm.Z) {
                        const bool in = d_s <= (float)z;
                        const float rz = in ? r_h : 0.0f, wtz = in ? wt_h : 0.0f;
                        const float idle = expf(Sz[z]);
                        float a0, a1, gd, gg;
                        dom_sum4(rz, 0.0f, rz * tss, 0.0f, wtz, 0.0f, wtz * tcs, 0.0f, a0, a1, gd, gg);
                        const float p_coll = clamp_min((1.0f - idle) - idle * a0, 0.0f);
                        tsl = tsl + piz[z] * ((pm.slot_us * idle + idle * a1) + p_coll * (gg / clamp_min(gd, 1e-12f)));
                        opn = opn + (in ? piz[z] : 0.0f);
                    }
                const float rate_h = ((ws * tau) * opn) / tsl;
                float h0, h1;
                hid_sum2(rate_h, rate_h * tv_s, h0, h1);
                hf = expf(-(tv_s * h0 + h1));
            }
            float O = 0.0f;
            num = 0.0f;
#pragma unroll
            for (int z = 0; z < ZX; ++z)
                if (z < pm.Z) {
                    const bool in = d_s <= (float)z;
                    const float okz = (expf(Sz[z] - ((acts && in) ? lt : 0.0f)) * hf) * pm.fer1;
                    const float wz = in ? piz[z] : 0.0f;
                    num = num + wz * okz;
                    O = O + wz;
                }
            p = 1.0f - num / clamp_min(O, 1e-12f);
        };
        for (int it = 0; it < pm.fp_iters; ++it) {
            tau = clampf(tau, 1e-7f, 0.999f);
            if (!bgl) tau_b = clampf(tau_b, 1e-7f, 0.999f);
            if constexpr (ZN) failz(); else fail();
            tau = tau + pm.damp * (tau_of_p(p, W0s, Wms, L, tw) - tau);
            if (!bgl) tau_b = tau_b + pm.damp * (tau_of_p(pb, W0b, Wmb, L, twb) - tau_b);
        }
        tau = clampf(tau, 1e-7f, 0.999f);
        if (!bgl) tau_b = clampf(tau_b, 1e-7f, 0.999f);
        if constexpr (ZN) failz(); else fail();
        const float r_o = (ws * tau) / (1.0f - tau), r_b = bgl ? 0.0f : (wb * tau_b) / (1.0f - tau_b);
        const float wt_o = ws * tau, wt_b = wb * tau_b;
        // ---- retry-limit loss inputs (wifi/engine.py:375-381; they need only this sub-step's p, so they are
        // evaluated here, where their latency overlaps the sums below)
        const bool back = q > 0.f;
        att_n = back ? att_n + w : 0.0f;
        const float lp = act ? log_r(clamp_min(p, 1e-12f)) : 0.0f;
        att_logp = back ? att_logp + lp : 0.0f;
        const float p_bar = att_n > 0.f ? exp_r(att_logp / clamp_min(att_n, 1e-12f)) : p;
        const float pbl = pow_int_torch(p_bar, L);
        float tslot = 0.0f, p_idle = 0.0f, succ = ok;
        if constexpr (ZN) {
            // slot_time (meanfield.py:134-158): the four sums and the idle share of every zone, weighted by pi
            succ = num;
#pragma unroll
            for (int z = 0; z < ZX; ++z)
                if (z < pm.Z) {
                    const bool in = d_s <= (float)z;
                    const float rz = in ? r_o : 0.0f, wtz = in ? wt_o : 0.0f;
                    const float idle = exp_r(Sz[z]);
                    float a0, a1, gd, gg;
                    dom_sum4(rz, 0.0f, rz * tss, 0.0f, wtz, 0.0f, wtz * tcs, 0.0f, a0, a1, gd, gg);
                    const float p_coll = clamp_min((1.0f - idle) - idle * a0, 0.0f);
                    const float tcav = gg / clamp_min(gd, 1e-12f);
                    tslot = tslot + piz[z] * ((pm.slot_us * idle + idle * a1) + p_coll * tcav);
                    p_idle = p_idle + piz[z] * idle;
                }
        } else {
            const float idle = exp_r(S);
            float a0, a1, gd, gg;
            dom_sum4(r_o, r_b, r_o * tss, r_b * tsb, wt_o, wt_b, wt_o * tcs, wt_b * tcb, a0, a1, gd, gg);
            const float p_coll = clamp_min((1.0f - idle) - idle * a0, 0.0f);
            const float tcav = gg / clamp_min(gd, 1e-12f);
            tslot = 0.0f + ((pm.slot_us * idle + idle * a1) + p_coll * tcav);
            p_idle = 0.0f + idle;
        }
        const float mu = act ? (tau * succ) / tslot : 0.0f;

        // ---- access count (wifi/engine.py:355-360)
        const float lam = mu * pm.dt_us;
        float n_acc, c1 = 0.f;
        if (pm.access_noise == 0) {
            const float u = uniform_bits(elem_hash(key_acc, (uint32_t)(k * R + rc)));
            const float ll = log_r(clamp_min(lam, 1e-30f));
            double cum = 0.0;
            int n = 0;
            for (int kk = 0; kk < pm.n_acc_max; ++kk) {
                const float lp = ((float)kk * ll - lam) - pm.lgamma[kk];
                cum += (double)exp_r(lp);
                if (!(u > (float)cum)) break;      // the CDF never decreases: the count is the first k with u <= CDF
                ++n;
            }
            n_acc = (float)n;
        } else {
            c1 = credit + lam * w;
            n_acc = floorf(c1);
        }
        const float served = fminn(q, n_acc * B) * w;

        // ---- FIFO service, finish times, loss (serve_fifo, wifi/engine.py:361-383)
        double cacc = 0.0;
        float prev_nc = 0.0f;
        auto serve = [&](int f, float rm, int c) {
            const int o = f * WAVE + lane;
            cacc += (double)rm;
            const float cum = (float)cacc;
            const float nc = clamp_min(cum - served, 0.0f);
            const float nw = nc - prev_nc;
            prev_nc = nc;
            const bool fin = rm > 0.0f && nw <= 1e-3f;
            s_rem[o] = fin ? 0.0f : nw;
            if (fin) {
                const float j = clamp_min(ceilf(cum / B - 1e-6f), 1.0f);
                float frac = pm.access_noise == 0 ? j / (n_acc + 1.0f) : (j - credit) / clamp_min(lam, 1e-9f);
                frac = clampf(frac, 0.0f, 1.0f);
                const float tfin = fminn(tf + ((float)k + frac) / (float)K, (tf + 1.0f) - 1e-6f);
                const float size = pm.sizes[(c > 1 ? (c < pm.n_cls ? c : pm.n_cls) : 1) - 1];
                const float n_frame = clamp_min(ceilf(size / B), 1.0f);
                const float p_lost = 1.0f - pow_count(1.0f - pbl, n_frame);
                const float u = uniform_bits(elem_hash(key_loss, (uint32_t)(rc * F + f)));
                if (!(u < p_lost)) s_fin[o] = tfin;
            }
        };
        {
            // (the next frame's bytes and class are read before this frame is served)
            float rm_n = qlen > 0 ? s_rem[lane] : 0.0f;
            int cl_n = qlen > 0 ? (int)s_cls[lane] : 0;
            for (int f = 0; f < qlen; ++f) {
                const float rm = rm_n;
                const int c = cl_n;
                if (f + 1 < qlen) {
                    rm_n = s_rem[(f + 1) * WAVE + lane];
                    cl_n = (int)s_cls[(f + 1) * WAVE + lane];
                }
                serve(f, rm, c);
            }
        }
        if (pm.access_noise == 1 && act) credit = fifo_sum() > 0.f ? c1 - n_acc : 0.0f;
        roam = roam - 1 > 0 ? roam - 1 : 0;
        acc_sum = acc_sum + (act ? 1.0f / clamp_min(mu, 1e-12f) : 0.0f);
        acc_n = acc_n + w;
        p_sum = p_sum + p * w;
        busy_sum = busy_sum + (1.0f - p_idle);
    }

    // ---------------- per-robot state and outputs of _serve ----------------
    const bool keep = fifo_sum() > 0.f;
    if (rob) {
        st.tau[(size_t)ec * NS + rc] = tau;
        if (r == 0 && !bgl)
            for (int a = 0; a < A; ++a) st.tau[(size_t)ec * NS + R + a] = tau_b;
        st.roam_left[ir] = roam;
        st.credit[ir] = keep ? credit : 0.0f;
        st.att_n[ir] = keep ? att_n : 0.0f;
        st.att_logp[ir] = keep ? att_logp : 0.0f;
    }
    if (is_bg) st.tau[(size_t)ec * NS + r] = tau;
    o_acc = acc_n > 0.f ? (acc_sum / clamp_min(acc_n, 1.0f)) / 1000.0f : NAN;
    o_pf = acc_n > 0.f ? p_sum / clamp_min(acc_n, 1.0f) : NAN;
    o_busy = busy_sum / (float)K;
    } else {
    // ---------------- per-slot CSMA/CA: the next transmission slot, its transmitters, the outcome ----------------
    const int aif = dp.aifsn, slot = dp.slot, sifs = dp.sifs, Tn = dp.T;
    int b = rob ? ds.b[ir] : 0, stage = rob ? ds.stage[ir] : 0;
    const bool had = rob && ds.had[ir] != 0;
    int ti = env_ok ? ds.t_idle[ec] : 0;                  // end of the last busy period, ns from the step start
    const uint32_t kpost = mix32(hkey ^ salt32(2u)), karr = mix32(hkey ^ salt32(3u)), kfer = mix32(hkey ^ salt32(4u));
    const int capi = (int)floorf(capB);
    const int nd = dp.ndbps[mcs];
    int64_t q = 0;                                         // whole bytes queued (sizes rounded up)
    for (int f = 0; f < qlen; ++f) {
        const int o = f * WAVE + lane;
        s_rem[o] = ceilf(s_rem[o]);
        q += (int64_t)s_rem[o];
    }
    // a station that was not contending (empty queue or no usable MCS): it sends at the next slot boundary when its
    // counter has run out during an idle period of at least its AIFS, else it draws a counter first
    // (eventsim.py:113-123)
    if (rob && q > 0 && link && !had) {
        const int el = -ti - sifs;
        const int ka = el >= 0 ? el / slot : -1;
        const int spent = ka - aif > 0 ? ka - aif : 0;
        if (b - spent <= 0) b = ka >= aif ? ka + 1 - aif : draw_int(elem_hash(karr, (uint32_t)rc), dp.W0);
    }
    // serve (lost = false) or drop (lost = true) Bc bytes from the head of this station's FIFO; a message with a
    // dropped byte is discarded whole
    auto consume = [&](int Bc, bool lost, int t_end) {
        const float tfin = (float)((double)t + (double)t_end / (double)Tn);
        for (int f = 0; f < qlen && Bc > 0; ++f) {
            const int o = f * WAVE + lane;
            const int rm = (int)s_rem[o];
            if (rm <= 0) continue;
            const int take = Bc < rm ? Bc : rm;
            Bc -= take;
            if (lost) {
                s_rem[o] = 0.0f;
                q -= rm;
            } else {
                s_rem[o] = (float)(rm - take);
                q -= take;
                if (rm == take) s_fin[o] = tfin;
            }
        }
    };
    int n_ev = 0, n_att = 0, n_fail = 0, n_succ = 0, prev_end = 0, busy_ns = 0;
    double acc_ms = 0.0;
    bool done = !env_ok, idle_end = false;
    while (__ballot(!done) != 0ull) {
        const bool cand = rob && !done && q > 0 && link;
        const int key = cand ? aif + b : 0x3fffffff;
        const int Kc = -seg_max_i(-key, rb);
        const bool tx = cand && key == Kc;
        const int Bv = q < (int64_t)capi ? (int)q : capi;
        int d_succ, d_coll;
        dcf_busy(pm, dp, Bv, nd, d_succ, d_coll);
        const int n_tx = __builtin_popcountll(__ballot(tx) & seg_bits(rb, lane));
        const int dur = n_tx == 1 ? seg_sum_i(tx ? d_succ : 0, rb) : seg_max_i(tx ? d_coll : 0, rb);
        const bool none = Kc >= 0x3fffffff;
        const int t_end = none ? 0 : ti + sifs + Kc * slot + dur;
        const bool stop = none || t_end > Tn;      // the exchange must end within the step
        if (!done && !stop) {
            const int dec = Kc - aif > 0 ? Kc - aif : 0;
            b = b - dec > 0 ? b - dec : 0;
            bool ok = false;
            if (n_tx == 1) ok = !(uniform_bits(elem_hash(kfer, (uint32_t)n_ev)) < dp.fer);
            busy_ns += dur;
            if (tx) {
                ++n_att;
                int W;
                if (ok) {
                    consume(Bv, false, t_end);
                    acc_ms += (double)(t_end - prev_end) * 1e-6;
                    ++n_succ;
                    stage = 0;
                    W = dp.W0;
                } else {
                    ++n_fail;
                    ++stage;
                    if (stage >= L) { consume(Bv, true, t_end); stage = 0; }
                    W = dp.W0 << stage;
                    W = W < dp.Wmax ? W : dp.Wmax;
                }
                b = draw_int(elem_hash(kpost, (uint32_t)(n_ev * R + rc)), W);
                prev_end = t_end;
            }
            ti = t_end;
            ++n_ev;
        }
        if (!done && stop) idle_end = none;
        done = done || stop;
    }
    ti -= Tn;
    if (idle_end && -ti - sifs >= 0) {
        // nobody contends: re-base the idle anchor to AIFS slots before the step end and count the extra idle slots
        // off every counter (the later transmission times and counters are unchanged; the integers stay bounded)
        const int m = (-ti - sifs) / slot - aif;
        if (m > 0) {
            ti += m * slot;
            b = b - m > 0 ? b - m : 0;
        }
    }
    if (rob) { ds.b[ir] = b; ds.stage[ir] = stage; ds.had[ir] = q > 0 && link ? 1 : 0; }
    if (env_ok && r == 0) ds.t_idle[ec] = ti;
    o_acc = n_succ > 0 ? (float)(acc_ms / (double)n_succ) : NAN;
    o_pf = n_att > 0 ? (float)((double)n_fail / (double)n_att) : NAN;
    o_busy = (float)((double)busy_ns / (double)Tn);
    }
    if (rob) {
        st.serv[ir] = sv;
        st.last_snr[ir] = snr;
        out.access_ms[ir] = o_acc;
        out.p_fail[ir] = o_pf;
        out.busy[ir] = o_busy;
        out.mcs[ir] = link ? pm.mcs_ids[mcs] : -1;
        out.rate_mbps[ir] = link ? rate : 0.0f;
        out.sinr_db[ir] = snr;
        out.serving_cell[ir] = sv;
    }

    // ---------------- end of step: finish_body ----------------
    int64_t lhid = env_ok ? st.last_hid[ec] : 0;
    if (CNT && env_ok && s_hid0[gseg] && lhid != 0) {     // (the enqueue's calls clear it)
        lhid = 0;
        if (r == 0) st.last_hid[ec] = 0;
    }
    const int64_t chid = env_ok ? (hid_in ? hid_in[ec] : lhid) : 0;
    int newest = -1;
    bool det_hit = false;
    uint64_t vmask = 0, dmask = 0;                         // slots still queued after the step; their det flags
    const size_t oo = ir * F;                              // [E][R][F] outputs
    for (int f = 0; f < F; ++f) {
        const int o = f * WAVE + lane;
        int cap = -1;
        bool dt = false;
        int hid = 0;
        if (rob) { cap = st.cap[fo + (size_t)f * R]; dt = st.det[fo + (size_t)f * R] != 0; hid = st.hid[fo + (size_t)f * R]; }
        const float fin = s_fin[o];
        const bool dlv = cap >= 0 && fin != INFINITY && fin == fin;
        const bool timed = cap >= 0 && !dlv && ((t + 1 - (int64_t)cap) >= pm.timeout);
        newest = dlv && cap > newest ? cap : newest;
        det_hit = det_hit || (dlv && dt && (int64_t)hid == chid);
        if (rob) {
            out.delivered[oo + f] = dlv;
            out.timed_out[oo + f] = timed;
            out.cap[oo + f] = cap;
            out.cls[oo + f] = s_cls[o];
            out.delay[oo + f] = dlv ? fin - (float)cap : NAN;
        }
        const bool gone = dlv || timed;
        if (gone) s_rem[o] = 0.0f;
        if (!gone && cap >= 0) vmask |= 1ull << f;
        if (dt && !gone) dmask |= 1ull << f;
        s_stage[o] = gone ? -1 : cap;                      // the new cap row, staged for the permutation
    }
    // stable partition (finish_body's cumsum scatter): the queued slots in order, then the others in order
    const int nvalid = __builtin_popcountll(vmask);
    {
        int gv = 0, gi = nvalid;
        for (int f = 0; f < F; ++f) {
            const int dst = ((vmask >> f) & 1ull) ? gv++ : gi++;
            s_src[dst * WAVE + lane] = (uint8_t)f;
        }
    }
    if (rob) {
        // cap (staged above), then every other field through the staging row
        for (int gdst = 0; gdst < F; ++gdst) st.cap[fo + (size_t)gdst * R] = s_stage[s_src[gdst * WAVE + lane] * WAVE + lane];
        for (int f = 0; f < F; ++f) {
            const int o = f * WAVE + lane;
            s_stage[o] = s_cls[o];
        }
        for (int gdst = 0; gdst < F; ++gdst) st.cls[fo + (size_t)gdst * R] = s_stage[s_src[gdst * WAVE + lane] * WAVE + lane];
        for (int gdst = 0; gdst < F; ++gdst) {
            const int sf = s_src[gdst * WAVE + lane];
            st.det[fo + (size_t)gdst * R] = (uint8_t)((dmask >> sf) & 1ull);
        }
        for (int f = 0; f < F; ++f) s_stage[f * WAVE + lane] = st.hid[fo + (size_t)f * R];
        for (int gdst = 0; gdst < F; ++gdst) st.hid[fo + (size_t)gdst * R] = s_stage[s_src[gdst * WAVE + lane] * WAVE + lane];
        for (int f = 0; f < F; ++f) s_stage[f * WAVE + lane] = st.f_nact[fo + (size_t)f * R];
        for (int gdst = 0; gdst < F; ++gdst) st.f_nact[fo + (size_t)gdst * R] = s_stage[s_src[gdst * WAVE + lane] * WAVE + lane];
        for (int f = 0; f < F; ++f) s_stage[f * WAVE + lane] = st.f_own[fo + (size_t)f * R];
        for (int gdst = 0; gdst < F; ++gdst) st.f_own[fo + (size_t)gdst * R] = s_stage[s_src[gdst * WAVE + lane] * WAVE + lane];
        float* s_stf = (float*)s_stage;
        for (int f = 0; f < F; ++f) s_stf[f * WAVE + lane] = st.f_snr[fo + (size_t)f * R];
        for (int gdst = 0; gdst < F; ++gdst) st.f_snr[fo + (size_t)gdst * R] = s_stf[s_src[gdst * WAVE + lane] * WAVE + lane];
        for (int f = 0; f < F; ++f) s_stf[f * WAVE + lane] = s_rem[f * WAVE + lane];
        for (int gdst = 0; gdst < F; ++gdst) {
            const float v = s_stf[s_src[gdst * WAVE + lane] * WAVE + lane];
            st.rem[fo + (size_t)gdst * R] = v;
            s_rem[gdst * WAVE + lane] = v;
        }
        st.qlen[ir] = nvalid;
        out.newest[ir] = newest;
        out.queue_len[ir] = nvalid;
        out.queue_bytes[ir] = fifo_sum();
    }
    // det_env: any delivered detection of the env's current hazard
    const bool any_det = seg_any(det_hit && rob, rb, lane);
    if (env_ok && r == 0) {
        out.det_env[ec] = any_det;
        out.t[ec] = t;
        st.clock[ec] = t + 1;
        st.ctr_step[ec] = ctr;
        st.pending[ec] = 0;
    }
    // the enqueue's global calls, counted by workgroup 0 at its end (a one-wave pass over every count)
    if (CNT && blockIdx.x == 0)
        submit_calls(st, pm.E, pm.step_counts, (size_t)pm.E * R * pm.step_n_cls, pm.step_n_cls, s_cmax, false);
}

// ======================================================================================= submit kernel
// add_body (proto/netsim_fast.py:136-160) for one LevelNet.submit call (send) or the harness's sequence of calls
// (counts: class 1 first, one call per message index).
__global__ __launch_bounds__(WAVE) void wifi_submit_kernel(InetWifiState st, InetWifiParams pm,
                                                           const int64_t* __restrict__ tin,
                                                           const int64_t* __restrict__ send,
                                                           const uint8_t* __restrict__ det,
                                                           const int64_t* __restrict__ hid,
                                                           const float* __restrict__ snr,
                                                           const uint8_t* __restrict__ counts, int n_cls,
                                                           void* accepted, int rb) {
    const int R = pm.R, F = pm.F, G = pm.envs_per_wave;
    const int lane = threadIdx.x;
    const int g = lane / rb, r = lane - g * rb;
    const int e = blockIdx.x * G + g;
    const bool env_ok = g < G && e < pm.E;
    const bool rob = env_ok && r < R;
    const int ec = env_ok ? e : 0, rc = rob ? r : 0;
    const size_t ir = (size_t)ec * R + rc;
    const size_t fo = (size_t)ec * F * R + rc;
    const int64_t t = env_ok ? (tin ? tin[ec] : st.clock[ec]) : 0;
    const int64_t hid_e = env_ok && hid ? hid[ec] : 0;
    int qlen = rob ? st.qlen[ir] : 0;
    const float snr_in = rob ? (snr ? snr[ir] : st.last_snr[ir]) : 0.f;
    const bool dt = rob && det ? det[ir] != 0 : false;
    int n_calls = 0;
    if (!counts) {
        const bool nw = fifo_call(st, pm, rob, rob ? (int)send[ir] : 0, qlen, fo, t, dt, hid_e, snr_in, rb, lane);
        if (rob) ((uint8_t*)accepted)[ir] = nw;
        n_calls = 1;
    } else {
        const int n_acc = fifo_counts(st, pm, counts, n_cls, rob, ir, qlen, fo, t, dt, hid_e, snr_in, rb, lane,
                                      n_calls);
        if (rob) ((int32_t*)accepted)[ir] = n_acc;
    }
    if (rob) st.qlen[ir] = qlen;
    // (the counts form's calls are global: wifi_submit_calls_kernel advances every env's call counter)
    if (!counts && env_ok && r == 0 && n_calls > 0) {
        st.last_hid[ec] = hid_e;
        st.ctr_submit[ec] += n_calls;
    }
}

// The counts form stands for a sequence of global submit calls (class 1 first, one call per message index up to the
// largest count of the class over every env): each call advances every env's SUBMIT call counter and sets its last
// hazard id (0: no hid in this form), including envs with nothing to send. One workgroup.
__global__ __launch_bounds__(1024) void wifi_submit_calls_kernel(InetWifiState st, int E, int R,
                                                                 const uint8_t* __restrict__ counts, int n_cls) {
    __shared__ int s_max[INET_WIFI_MAX_CLS];
    submit_calls(st, E, counts, (size_t)E * R * n_cls, n_cls, s_max, true);
}

// ======================================================================================= reset kernel
// LevelNet.reset (levels/base.py:142-157) + WifiNet._reset_rows (wifi/engine.py:179-186) + the radio's plane waves
// of the new episode (radio.py:200-219; the reference draws them when it makes the radio and at every reset, keyed by
// the env's current episode, so drawing them at every reset gives the same fields). One block per env.
__global__ void wifi_reset_kernel(InetWifiState st, InetWifiParams pm, const uint8_t* __restrict__ mask) {
    const int e = blockIdx.x;
    if (e >= pm.E || (mask && !mask[e])) return;
    const int R = pm.R, F = pm.F;
    const int ep_new = st.episode[e] + 1;
    for (int i = threadIdx.x; i < F * R; i += blockDim.x) {
        const size_t o = (size_t)e * F * R + i;
        st.cap[o] = -1; st.cls[o] = 0; st.det[o] = 0; st.hid[o] = -1; st.rem[o] = 0.f;
        st.f_nact[o] = 0; st.f_snr[o] = 0.f; st.f_own[o] = 0;
    }
    for (int r = threadIdx.x; r < R; r += blockDim.x) {
        const size_t ir = (size_t)e * R + r;
        st.qlen[ir] = 0; st.last_snr[ir] = 0.f; st.roam_left[ir] = 0; st.serv[ir] = 0;
        st.att_n[ir] = 0.f; st.att_logp[ir] = 0.f; st.credit[ir] = 0.f;
    }
    for (int r = threadIdx.x; r < R + pm.A; r += blockDim.x) st.tau[(size_t)e * (R + pm.A) + r] = pm.tau0;
    // the fields of every AP: wave kk of AP c is element c K + kk of the field's draws (as the cells of RadioMC)
    const int Kf = pm.n_modes, A = pm.A;
    for (int q = threadIdx.x; q < A * pm.n_fields * Kf; q += blockDim.x) {
        const int c = q / (pm.n_fields * Kf), rem = q - c * pm.n_fields * Kf;
        const int fi = rem / Kf, kk = rem - fi * Kf;
        draw_plane_wave((uint32_t)pm.seed_key, (uint32_t)st.env_id[e], (uint32_t)ep_new, pm.radio_model, fi,
                        c * Kf + kk, pm.dcorr[fi], pm.spectrum,
                        st.field + ((((size_t)e * A + c) * pm.n_fields + fi) * Kf + kk) * 3);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        st.episode[e] = ep_new;
        st.ctr_step[e] = 0;
        st.ctr_submit[e] = -st.calls[0];
        st.clock[e] = 0;
        st.last_hid[e] = 0;
        st.pending[e] = 1;
    }
}

// ======================================================================================= DCF reset kernel
// the initial backoff counters of the new episode (channel RESET, stream 5, element r), stage 0, idle medium
__global__ void dcf_reset_kernel(InetWifiState st, InetDcfState ds, InetWifiParams pm, InetDcfParams dp,
                                 const uint8_t* __restrict__ mask) {
    const int e = blockIdx.x;
    if (e >= pm.E || (mask && !mask[e])) return;
    const uint32_t key = base_key((uint32_t)pm.seed_key, (uint32_t)st.env_id[e], (uint32_t)st.episode[e], 3u, 0u, 5u);
    for (int r = threadIdx.x; r < pm.R; r += blockDim.x) {
        const size_t ir = (size_t)e * pm.R + r;
        ds.b[ir] = draw_int(elem_hash(key, (uint32_t)r), dp.W0);
        ds.stage[ir] = 0;
        ds.had[ir] = 0;
    }
    if (threadIdx.x == 0) ds.t_idle[e] = 0;
}

// ======================================================================================= C ABI
namespace {

int next_pow2(int v) { int p = 1; while (p < v) p <<= 1; return p; }

int check_params(const InetWifiParams& p) {
    if (p.E <= 0 || p.R <= 0 || p.R > INET_WIFI_MAX_R || p.F <= 0 || p.F > INET_WIFI_MAX_F || p.K <= 0)
        return INET_WIFI_EINVAL;
    if (p.M <= 0 || p.M > INET_WIFI_MAX_M || p.L <= 0 || p.L > INET_WIFI_MAX_L || p.n_cls <= 0 ||
        p.n_cls > INET_WIFI_MAX_CLS || p.n_acc_max <= 0 || p.n_acc_max > INET_WIFI_MAX_NACC || p.fp_iters < 1)
        return INET_WIFI_EINVAL;
    if (p.n_fields < 0 || p.n_fields > 3 || p.n_modes < 0 || p.n_modes > INET_WIFI_MAX_KF) return INET_WIFI_EINVAL;
    if (p.bg_ac < 0 || p.bg_ac > 4 || p.A < 1 || p.A > INET_WIFI_MAX_A || p.R + p.A > 65) return INET_WIFI_EINVAL;
    // several channels: every AP's domain index below n_dom, every station in a lane of its own (R + A <= 64), and
    // (R + A) n_dom < 400 (the size up to which the reference's batched product adds in index order)
    if (p.n_dom < 1 || p.n_dom > p.A) return INET_WIFI_EINVAL;
    for (int a = 0; a < p.A; ++a) if (p.ap_dom[a] < 0 || p.ap_dom[a] >= p.n_dom) return INET_WIFI_EINVAL;
    if (p.n_dom > 1 && (p.R + p.A > 64 || (p.R + p.A) * p.n_dom >= 400)) return INET_WIFI_EUNSUPPORTED;
    // AIFS zones: 1 .. INET_WIFI_MAX_Z, every station in a lane of its own
    if (p.Z < 1 || p.Z > INET_WIFI_MAX_Z) return INET_WIFI_EINVAL;
    if (p.Z > 1 && p.R + p.A > 64) return INET_WIFI_EUNSUPPORTED;
    // hidden nodes: (R + A)^2 < 400 (the size up to which the reference's products add in index order)
    if (p.hidden && (p.R + p.A) * (p.R + p.A) >= 400) return INET_WIFI_EUNSUPPORTED;
    if (p.los_sto && (!p.los_cdf || p.radio_model != 1 || p.n_fields != 3 || p.plos_scn < 0 || p.plos_scn > 2))
        return INET_WIFI_EINVAL;
    for (int c = 0; c <= p.n_cls; ++c) if (p.cls_ac[c] < 0 || p.cls_ac[c] > 4) return INET_WIFI_EINVAL;
    const int rb = next_pow2(p.R);
    if (p.envs_per_wave < 1 || p.envs_per_wave * rb > WAVE) return INET_WIFI_EINVAL;
    return INET_WIFI_OK;
}

// the step's enqueue (step_counts): its class count
int check_step_counts(const InetWifiParams& p) {
    if (p.step_counts && (p.step_n_cls <= 0 || p.step_n_cls > p.n_cls)) return INET_WIFI_EINVAL;
    return INET_WIFI_OK;
}

}  // namespace

extern "C" {

int32_t inet_wifi_abi_version(void) { return INET_WIFI_ABI_VERSION; }

int32_t inet_wifi_step(const InetWifiState* st, const InetWifiParams* prm, const int64_t* t, int32_t input_kind,
                       const float* x, const int64_t* cur_hid, const InetWifiOutputs* out, void* stream) {
    if (!st || !prm || !x || !out) return INET_WIFI_EINVAL;
    const InetWifiParams& p = *prm;
    int rc = check_params(p);
    if (rc) return rc;
    if (input_kind < 0 || input_kind > 2 || (input_kind == 1 && p.A != 1)) return INET_WIFI_EINVAL;
    if (input_kind == 0 && p.n_fields < 1) return INET_WIFI_EINVAL;
    // segments of next_pow2(R + A) lanes, lanes R .. R + A - 1 for the APs' background stations of the mean-field
    // solve (R + A <= 64); as many envs per wave as the submit kernel's segments hold, at most what fits
    const int rb = p.R + p.A <= WAVE ? next_pow2(p.R + p.A) : WAVE;
    InetWifiParams pm = p;
    pm.envs_per_wave = p.envs_per_wave * next_pow2(p.R) / rb > 0 ? p.envs_per_wave * next_pow2(p.R) / rb : 1;
    const int G = pm.envs_per_wave;
    const unsigned grid = (unsigned)((p.E + G - 1) / G);
    if ((rc = check_step_counts(p))) return rc;
    const size_t lds = (size_t)p.F * WAVE * (4 + 4 + 1 + 1);
    auto k = (p.Z > 1 || p.hidden) ? (p.step_counts ? wifi_step_kernel<false, true, true, true>
                                      : wifi_step_kernel<false, true, false, true>)
           : p.A > 1 ? (p.step_counts ? wifi_step_kernel<false, true, true> : wifi_step_kernel<false, true, false>)
                     : (p.step_counts ? wifi_step_kernel<false, false, true> : wifi_step_kernel<false, false, false>);
    hipLaunchKernelGGL(k, dim3(grid), dim3(WAVE), lds, (hipStream_t)stream, *st, pm, t, input_kind, x, cur_hid, *out,
                       rb, InetDcfState{}, InetDcfParams{});
    return hipGetLastError() == hipSuccess ? INET_WIFI_OK : INET_WIFI_ELAUNCH;
}

int32_t inet_wifi_submit(const InetWifiState* st, const InetWifiParams* prm, const int64_t* t, const int64_t* send,
                         const uint8_t* det, const int64_t* hid, const float* snr, const uint8_t* counts,
                         int32_t n_cls, void* accepted, void* stream) {
    if (!st || !prm || !accepted || (!send && !counts) || (send && counts)) return INET_WIFI_EINVAL;
    const InetWifiParams& p = *prm;
    int rc = check_params(p);
    if (rc) return rc;
    if (counts && (n_cls <= 0 || n_cls > p.n_cls)) return INET_WIFI_EINVAL;
    const int rb = next_pow2(p.R);
    const int G = p.envs_per_wave;
    hipLaunchKernelGGL(wifi_submit_kernel, dim3((p.E + G - 1) / G), dim3(WAVE), 0, (hipStream_t)stream, *st, p, t,
                       send, det, hid, snr, counts, n_cls, accepted, rb);
    if (counts)
        hipLaunchKernelGGL(wifi_submit_calls_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, *st, p.E, p.R,
                           counts, n_cls);
    return hipGetLastError() == hipSuccess ? INET_WIFI_OK : INET_WIFI_ELAUNCH;
}

namespace {
int check_dcf(const InetWifiParams& p, const InetDcfParams& d) {
    if (p.Z != 1 || p.hidden) return INET_WIFI_EUNSUPPORTED;
    // every exchange lasts at least one symbol or one control frame, so the event loop ends within the step
    if (d.T <= 0 || d.T > (1 << 30) || d.slot <= 0 || d.sifs < 0 || d.tsym <= 0 || d.pre < 0 || d.t_ack < 0 ||
        d.t_rts <= 0 || d.t_cts <= 0 || d.W0 < 1 || d.Wmax < d.W0 || d.Wmax > 65536 || d.aifsn < 0 ||
        d.aifsn > 64 || d.payload <= 0 || d.ovh < 0)
        return INET_WIFI_EINVAL;
    for (int m = 0; m < p.M; ++m) if (d.ndbps[m] <= 0) return INET_WIFI_EINVAL;
    // whole-byte sizes stay exact in the float32 FIFO
    for (int c = 0; c < p.n_cls; ++c) if (!(p.sizes[c] >= 0.0f && p.sizes[c] <= 16777216.0f)) return INET_WIFI_EINVAL;
    if (p.per_class_ac || p.bg_w != 0.0f || p.A != 1) return INET_WIFI_EUNSUPPORTED;
    return INET_WIFI_OK;
}
}  // namespace

int32_t inet_wifi_dcf_step(const InetWifiState* st, const InetDcfState* ds, const InetWifiParams* prm,
                           const InetDcfParams* dp, const int64_t* t, int32_t input_kind, const float* x,
                           const int64_t* cur_hid, const InetWifiOutputs* out, void* stream) {
    if (!st || !ds || !prm || !dp || !x || !out) return INET_WIFI_EINVAL;
    const InetWifiParams& p = *prm;
    int rc = check_params(p);
    if (!rc) rc = check_dcf(p, *dp);
    if (rc) return rc;
    if (input_kind < 0 || input_kind > 2) return INET_WIFI_EINVAL;
    if (input_kind == 0 && p.n_fields < 1) return INET_WIFI_EINVAL;
    const int rb = next_pow2(p.R);
    const int G = p.envs_per_wave;
    const unsigned grid = (unsigned)((p.E + G - 1) / G);
    if ((rc = check_step_counts(p))) return rc;
    const size_t lds = (size_t)p.F * WAVE * (4 + 4 + 1 + 1);
    auto k = p.step_counts ? wifi_step_kernel<true, false, true> : wifi_step_kernel<true, false, false>;
    hipLaunchKernelGGL(k, dim3(grid), dim3(WAVE), lds, (hipStream_t)stream, *st, p, t, input_kind, x, cur_hid, *out,
                       rb, *ds, *dp);
    return hipGetLastError() == hipSuccess ? INET_WIFI_OK : INET_WIFI_ELAUNCH;
}

int32_t inet_wifi_dcf_reset(const InetWifiState* st, const InetDcfState* ds, const InetWifiParams* prm,
                            const InetDcfParams* dp, const uint8_t* mask, void* stream) {
    if (!st || !ds || !prm || !dp) return INET_WIFI_EINVAL;
    int rc = check_params(*prm);
    if (!rc) rc = check_dcf(*prm, *dp);
    if (rc) return rc;
    hipLaunchKernelGGL(wifi_reset_kernel, dim3(prm->E), dim3(WAVE), 0, (hipStream_t)stream, *st, *prm, mask);
    if (hipGetLastError() != hipSuccess) return INET_WIFI_ELAUNCH;
    hipLaunchKernelGGL(dcf_reset_kernel, dim3(prm->E), dim3(WAVE), 0, (hipStream_t)stream, *st, *ds, *prm, *dp, mask);
    return hipGetLastError() == hipSuccess ? INET_WIFI_OK : INET_WIFI_ELAUNCH;
}

int32_t inet_wifi_reset(const InetWifiState* st, const InetWifiParams* prm, const uint8_t* mask, void* stream) {
    if (!st || !prm) return INET_WIFI_EINVAL;
    int rc = check_params(*prm);
    if (rc) return rc;
    hipLaunchKernelGGL(wifi_reset_kernel, dim3(prm->E), dim3(WAVE), 0, (hipStream_t)stream, *st, *prm, mask);
    return hipGetLastError() == hipSuccess ? INET_WIFI_OK : INET_WIFI_ELAUNCH;
}

}  // extern "C"

// The control-step kernel of the NR uplink engine (gfx950, wave64), instantiated per (subbands S, HARQ processes P,
// IR combining, per-subband SNR input) by nr_step_s*.hip.
//
// nr_step_kernel runs one whole control step per env: the radio prologue (TR 38.901 / log-distance path gain of the
// pose, isaac_net/core/radio.py:238-277), every scheduled slot of the step (AR(1) Rician / Rayleigh fading,
// nr_engine.py:570-611; SR opportunities, mac_ul.py:66-71; UL data slots, mac.py:228-508 with the UlMac hooks of
// mac_ul.py:140-236) and the end of step (nr_engine.py:843-888, mac.py:585-616, queues.py:105-110), reading and
// writing HBM once per step.
//
// Work decomposition: one workgroup is one wavefront; one robot per lane; the RB = next_pow2(R) lanes of an env form
// one aligned segment of the wavefront, so every cross-robot step of the scheduler (retransmission admission,
// RBG-by-RBG argmax, lexicographic masking) is a DPP / lane-swap butterfly or a ballot inside the segment, with no
// barrier. Per-robot state (HARQ processes, subband CSI and fading, MAC scalars) stays in VGPRs across the slots;
// the per-MCS tables live in LDS; the in-order RLC pointer after every UL slot is recorded in LDS and replayed over
// the queued frames in the epilogue, so the slot loop never reads the frame FIFO.
//
// Float arithmetic follows the reference's torch op order (no contraction, ATen reduction order) so that only the
// transcendental functions (logf, expf, powf, log10f, cosf) differ from the CPU path by rounding. Sums over the RBGs
// a robot holds skip the RBGs it does not hold: their terms are exact zeros of the ATen-order sum, so visiting the
// held RBGs in that order gives the same bits (aten_rot).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/inet_nr.h"
#include "aten_sort.h"
#include "doppler.h"
#include "inet_nr_dev.h"

namespace inet {

// Phase clocks (a build option, off in the product library: build.py --phase-clocks writes libinet_nr_phase.so).
// With INET_PHASE_CLOCKS defined, every wavefront of the step kernel adds the shader clock (s_memtime) spent in each
// phase of the step to its own row of g_phase_clk [wave][INET_NPH] (vector stores at the end), read back
// by inet_nr_phase_clocks_<unit> of the translation unit that holds the kernel (each unit has its own array). The
// marks sit at wave-uniform points, so the counts are wave totals; the work is unchanged.
constexpr int INET_NPH = 12;
constexpr int INET_PH_WAVES = 1 << 16;
#ifdef INET_PHASE_CLOCKS
static __device__ uint64_t g_phase_clk[INET_PH_WAVES * INET_NPH];
// the running sums live in one VGPR (lane i holds phase i, a select and an add, no branch) and the
// last mark in one scalar register (the low 32 bits of the clock), so that the build keeps the product kernel's
// register allocation as far as possible
#ifndef INET_PH_MASK
#define INET_PH_MASK 0xfff
#endif
#define INET_PH_DECL                                                                                               \
    uint32_t ph_v = 0u;                                                                                            \
    uint32_t ph_t0 = (uint32_t)__builtin_amdgcn_s_memtime();
#define INET_PH(i)                                                                                                 \
    if (((INET_PH_MASK) >> (i)) & 1) do {                                                                          \
        const uint32_t _t = (uint32_t)__builtin_amdgcn_s_memtime();                                                \
        ph_v += (threadIdx.x & 63) == (i) ? _t - ph_t0 : 0u;                                                       \
        ph_t0 = _t;                                                                                                \
    } while (0)
#define INET_PH_STORE                                                                                              \
    do {                                                                                                           \
        const unsigned wv = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);                                    \
        if ((threadIdx.x & 63) < INET_NPH && wv < (unsigned)INET_PH_WAVES)                                         \
            g_phase_clk[(size_t)wv * INET_NPH + (threadIdx.x & 63)] = ph_v;                                        \
    } while (0)
// copies the first n_waves rows to the host (0, or the HIP error)
#define INET_PHASE_READER(NAME)                                                                                     \
    extern "C" int NAME(uint64_t* out, int n_waves) {                                                              \
        if (n_waves < 0 || n_waves > inet::INET_PH_WAVES) return -1;                                               \
        return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(inet::g_phase_clk),                                        \
                                        sizeof(uint64_t) * inet::INET_NPH * n_waves, 0, hipMemcpyDeviceToHost);     \
    }
#else
#define INET_PH_DECL
#define INET_PH(i) do { } while (0)
#define INET_PH_STORE do { } while (0)
#define INET_PHASE_READER(NAME)
#endif

constexpr int STEP_WAVE = 64;          // one wavefront per workgroup
constexpr int MAX_UL_ROWS = 64;        // UL data slots per control step
constexpr int MAX_M = 32;              // MCS table rows
constexpr int MAX_EQW = INET_NR_MAX_P + 1;
constexpr uint32_t CH_STEP = 2;

// Loads and stores at a uniform base plus a 32-bit per-lane byte offset (global_load ... v_off, s[base]): every
// per-lane address is one 32-bit VGPR, and the row strides of the [E][X][R] arrays stay in scalar registers.
template <class T>
DEV T ldo(const T* base, uint32_t off) { return *(const T*)((const char*)base + off); }
template <class T>
DEV void sto(T* base, uint32_t off, T v) { *(T*)((char*)base + off) = v; }

DEV int hm_state(uint32_t m) { return (int)(m & 0xffu); }
DEV int hm_ntx(uint32_t m) { return (int)((m >> 8) & 0xffu); }
DEV int hm_mcs(uint32_t m) { return (int)((m >> 16) & 0xffu); }
DEV int hm_nsb(uint32_t m) { return (int)((m >> 24) & 0xffu); }
DEV uint32_t hm_pack(int st, int ntx, int mcs, int nsb) {
    return (uint32_t)st | ((uint32_t)ntx << 8) | ((uint32_t)mcs << 16) | ((uint32_t)nsb << 24);
}

// ---------------------------------------------------------------- butterflies inside a power-of-two segment
// Level L combines every lane with a lane of the other half of its 2^(L+1) group: quad_perm [1,0,3,2] and [2,3,0,1],
// row_half_mirror, row_mirror (DPP moves with bound_ctrl, which the compiler folds into the consuming ALU op as a DPP
// source operand), then v_permlane16_swap (16-lane rows 2j and 2j + 1) and v_permlane32_swap (the two 32-lane
// halves): a swap of a value with itself leaves the first register holding the lower row's value and the second the
// upper row's, at every lane of the pair. Used only for commutative reductions whose operands are already uniform
// inside each 2^L group, where any such pairing gives the group result.
template <int L, class Op>
DEV int blevel(int v, Op op) {
    if constexpr (L == 0) return op(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true));
    else if constexpr (L == 1) return op(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true));
    else if constexpr (L == 2) return op(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true));
    else if constexpr (L == 3) return op(v, __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true));
    else if constexpr (L == 4) {
        const auto s = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        return op((int)s[0], (int)s[1]);
    } else {
        const auto s = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
        return op((int)s[0], (int)s[1]);
    }
}
struct OpAdd { DEV int operator()(int a, int b) const { return a + b; } };
struct OpMax { DEV int operator()(int a, int b) const { return a > b ? a : b; } };

DEV int bsum(int v, int rb) {
    if (rb > 1) v = blevel<0>(v, OpAdd{});
    if (rb > 2) v = blevel<1>(v, OpAdd{});
    if (rb > 4) v = blevel<2>(v, OpAdd{});
    if (rb > 8) v = blevel<3>(v, OpAdd{});
    if (rb > 16) v = blevel<4>(v, OpAdd{});
    if (rb > 32) v = blevel<5>(v, OpAdd{});
    return v;
}

template <int L>
DEV int imax_lvl(int v) { return blevel<L>(v, OpMax{}); }
// maximum over the segment, at every lane of the segment. The scheduler's bids are non-negative floats, whose bit
// patterns order like the values, or -1 for no bid, so the argmax runs on integers.
DEV int bmax_i(int v, int rb) {
    if (rb > 1) v = imax_lvl<0>(v);
    if (rb > 2) v = imax_lvl<1>(v);
    if (rb > 4) v = imax_lvl<2>(v);
    if (rb > 8) v = imax_lvl<3>(v);
    if (rb > 16) v = imax_lvl<4>(v);
    if (rb > 32) v = imax_lvl<5>(v);
    return v;
}
// bmax_i of N values at once (independent butterflies, interleaved)
template <int N>
DEV void bmax_n(int (&v)[N], int rb) {
#pragma unroll
    for (int i = 0; i < N; ++i) if (rb > 1) v[i] = imax_lvl<0>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) if (rb > 2) v[i] = imax_lvl<1>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) if (rb > 4) v[i] = imax_lvl<2>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) if (rb > 8) v[i] = imax_lvl<3>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) if (rb > 16) v[i] = imax_lvl<4>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) if (rb > 32) v[i] = imax_lvl<5>(v[i]);
}
// index (inside the segment) of the first lane of this lane's segment whose predicate holds; rb if none
DEV int seg_first(bool p, int rb, int lane) {
    unsigned long long b = __ballot(p) >> (lane & ~(rb - 1));
    if (rb < 64) b &= (1ull << rb) - 1ull;
    return b ? (int)__builtin_ctzll(b) : rb;
}

// bit `lane` of a wave-uniform 64-bit mask, as a lane predicate (one v_cndmask on the mask in scalar registers)
DEV bool lane_bit(unsigned long long m) {
    int v;
    asm volatile("v_cndmask_b32_e64 %0, 0, 1, %1" : "=v"(v) : "s"(m));
    return v != 0;
}
// two 32-lane segments per wavefront (envs of 17..32 robots): per segment, the lowest set bit of a wave-uniform mask
// (scalar ALU), and whether the segment has any bit set, as 64-bit lane masks
DEV unsigned long long seg32_lowest(unsigned long long b) {
    const uint32_t lo = (uint32_t)b, hi = (uint32_t)(b >> 32);
    return (unsigned long long)(lo & (0u - lo)) | ((unsigned long long)(hi & (0u - hi)) << 32);
}
DEV unsigned long long seg32_any(unsigned long long b) {
    return ((uint32_t)b ? 0xffffffffull : 0ull) | ((b >> 32) ? 0xffffffff00000000ull : 0ull);
}

// ---------------------------------------------------------------- ATen-order sums over the RBGs a robot holds
// torch's CPU sum of a row of N (N = 8 or 13 here) adds, from 0, the elements past the last full 8-vector first and
// then the 8 vector lanes in order: for N = 13 the order is 8, 9, ..., 12, 0, 1, ..., 7; for N = 8 it is 0, ..., 7.
// With every other element an exact zero (+0 or -0), adding only the held elements in that order gives the same sum.
template <int S>
DEV uint32_t aten_rot(uint32_t won) {
    if constexpr (S > 8) return (won >> 8) | ((won & 0xffu) << (S - 8));
    else return won;
}
template <int S>
DEV int aten_unrot(int b) {
    if constexpr (S > 8) return b < S - 8 ? b + 8 : b - (S - 8);
    else return b;
}
// torch.logsumexp over a row that is -inf outside the held RBGs (won), as a dense sum over every RBG: the max over the
// held RBGs, then the sum of exp(x_s - max) in ATen order with the RBGs not held adding exact zeros, which gives the
// bits of a sum over the held RBGs only. The loops are unrolled, so the S reads of the row issue together.
// xs(s): the row's value at RBG s (evaluated for every s, used where held).
template <int S, class X>
DEV float lse_held(X xs, uint32_t won) {
    float x[S];
    float mx = -INFINITY;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        x[s] = xs(s);
        const float v = ((won >> s) & 1u) ? x[s] : -INFINITY;
        mx = v > mx ? v : mx;
    }
    if (mx == INFINITY || mx == -INFINITY) mx = 0.f;
    float sum = 0.f;
    // (sum >= 1 when some RBG is held: the max term is exp(0); every term is exp of a finite x <= 0; none held: the
    // log of 0)
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const int s = aten_unrot<S>(i);
        sum += ((won >> s) & 1u) ? exp_nonpos(x[s] - mx) : 0.0f;
    }
    return (sum == 0.0f ? -INFINITY : ln_unit(sum)) + mx;
}
// lse_logw: the row log w_s (the log of the held PRB count, as torch computes it).
template <int S>
DEV float lse_logw(const float* s_logw, uint32_t won) {
    return lse_held<S>([&](int s) { return s_logw[s]; }, won);
}
// lse_eesm: the EESM row x_s = (-lin_s) / beta + log w_s of a robot whose linear SINR at RBG s is lin(s). rbeta =
// RN(1 / beta): the division is div_const, exact for every beta of the MCS tables. `nan` says that some lin_s of the
// full row (held or not) is NaN, which makes torch's result NaN.
template <int S, class L>
DEV float lse_eesm(L lin, const float* s_logw, uint32_t won, float beta, float rbeta, bool nan) {
    const float r = lse_held<S>([&](int s) { return div_const(-lin(s), beta, rbeta) + s_logw[s]; }, won);
    return nan ? NAN : r;
}
// PRB-weighted mean of the per-RBG dB values x_s (s_x[s * CW + lane]) over the held RBGs (mean_db): the ATen-order
// sum of nan_to_num(x_s * exp(log w_s - lnw)); the RBGs not held contribute exact zeros.
template <int S, int CW = STEP_WAVE>
DEV float mean_db_held(const float* s_x, int lane, const float* s_logw, uint32_t won, float lnw) {
    float acc = 0.f;
    for (uint32_t m = aten_rot<S>(won); m; m &= m - 1) {
        int s = aten_unrot<S>(__builtin_ctz(m));
        float t = s_x[s * CW + lane] * exp_nonpos(s_logw[s] - lnw);        // (log w_s - log sum w in [-2.6, 0])
        acc += nan_to_num(t, 0.0f, 3.4028234663852886e38f, -3.4028234663852886e38f);
    }
    return acc;
}

// Bilinear BLER at (table row base, SINR dB) with the code-block interpolation weight wi (phy.bler_lookup); rds =
// RN(1 / ds), the division by the SINR grid step being div_const
DEV float bler_at(const float* __restrict__ tab, int base0, int G, float s0, float ds, float rds, float sinr, float wi) {
    float xs = sinr != sinr ? -30.0f : sinr;
    float xg = clampf(div_const(xs - s0, ds, rds), 0.0f, (float)(G - 1));
    float j0f = clamp_max(floorf(xg), (float)(G - 2));
    int j0 = (int)j0f;
    float wj = xg - j0f;
    const float* p = tab + base0 + j0;
    float lo = p[0] * (1.0f - wj) + p[1] * wj;
    float hi = p[G] * (1.0f - wj) + p[G + 1] * wj;
    return lo * (1.0f - wi) + hi * wi;
}

// code-block segmentation (phy.segment) of TBS tbs at code rate r (float32 rate; the reference's float64 math) ->
// (cbs f32, ncb f32). The block count ceil(B / (Kcb - 24)) is an integer ceiling division: B < 2^31 and the divisor
// is 3816 or 8424, so the float64 quotient never crosses an integer the exact one does not.
DEV void segment_f(int tbs, float r32, float& cbs, float& ncb) {
    const double r = (double)r32;
    const bool bg2 = (tbs <= 292) || ((tbs <= 3824) && (r <= 0.67)) || (r <= 0.25);
    const int kcb = bg2 ? 3840 : 8448;
    const int b = tbs + (tbs > 3824 ? 24 : 16);
    // ceil(b / (kcb - 24)) with each constant divisor written out (a multiply by its reciprocal, not a division)
    const int c = b <= kcb ? 1 : (bg2 ? (b + 3815) / 3816 : (b + 8423) / 8424);
    cbs = c > 1 ? (float)((double)(b + 24 * c) / (double)c) : (float)b;
    ncb = (float)c;
}

// Dynamic LDS of the step kernel, in ints: the in-order pointer after every UL slot [n_ul][64], with RLC drop the
// byte range of a TB that exhausted its HARQ [n_ul][64] x 2, then the per-env HARQ histograms [64 / RB][3][max_tx + 1];
// with several cells (nc > 1) then per env each gNB's N+I estimate and this slot's interference [64 / RB][2][nc S].
inline size_t step_lds_bytes(int n_ul, int harq_drop, int rb, int max_tx, int nc = 1, int S = 0) {
    const size_t cw = rb > STEP_WAVE ? (size_t)rb : (size_t)STEP_WAVE;     // lanes per workgroup
    return sizeof(int) * ((size_t)n_ul * cw * (harq_drop ? 3 : 1) +
                          (cw / rb) * 3 * (max_tx + 1) +
                          (nc > 1 ? (cw / rb) * 2 * nc * S : 0));
}

// v[idx] of a register array indexed by a runtime value (a chain of selects, no scratch memory: the empty asm keeps
// 32-bit elements in registers, where the compiler would otherwise turn the chain into a stack load)
template <int N, class T>
DEV T sel_of(const T (&v)[N], int idx) {
    T r = v[0];
#pragma unroll
    for (int i = 1; i < N; ++i) {
        T x = v[i];
        if constexpr (sizeof(T) == 4) asm volatile("" : "+v"(x));
        r = idx == i ? x : r;
    }
    return r;
}

// RBT: the segment width when it is fixed at compile time (0: the runtime argument rb).
// LS: the link whose MAC state and queue the kernel runs: InetNrState (the UL; lk is st) or InetNrDlState (the DL
// of NRConfig(dl=True): CQI reports and DL data slots with the DlMac hooks; it reads the shared state of st and writes
// only the DL link's).
// NC: cells per env. NC > 1 runs NRNet.step_cells (nr_engine.py:718-788), UL with pose input: association and the A3
// plan in the prologue, the handovers due at every row, fading on every robot-cell link, one scheduler per cell (the
// segment's lanes of one serving cell: ballots masked to the cell, NC interleaved butterflies), fractional power
// control, and the same-slot interference sum of every gNB and RBG over the other cells' robots (each lane's terms in
// LDS, summed by one lane per (cell, RBG) in torch's CPU order); cl holds the association state and constants.
// RBT = 128 / 256: envs of 65..128 / 129..256 robots, one env per workgroup of W = 2 / 4 wavefronts; the env-wide
// collectives then combine the waves' ballots and butterflies through LDS (xchgw), and every cooperative loop runs a
// number of rounds that all waves agree on, so that every barrier is reached by all.
//
// FX = 1 builds the kernel for the common configuration (PF, chase combining, EESM, RLC AM, OLLA, PHR cap, retx
// priority, a fixed Rician phasor, fading; fx_profile), FX = 2 for the same without the Rician phasor: those
// switches become compile-time constants, which removes their tests from the slot loop and the scalar registers that
// hold them.
// Minimum waves per SIMD (the register budget): 2, and 3 for the two-wave FX = 2 build (envs of 65..128 robots at the
// common configuration: 168 VGPRs with 104 B per lane of spills, measured 7% faster than 193 VGPRs at 2 waves on
// 16384 x 128; 4 waves, at 128 VGPRs, spill enough to be 30% slower); 1 with several cells.
template <int S, int P, bool IR, bool VREF, int RBT, class LS, int NC, int FX = 0>
__global__ __launch_bounds__(STEP_WAVE * (RBT > STEP_WAVE ? RBT / STEP_WAVE : 1),
                             NC > 1 ? 1 : ((RBT == 128 && FX == 2) ? 3 : 2)) void nr_step_kernel(
    InetNrState st, LS lk_in, InetNrTables tb_in, InetNrParams pm_in, const InetNrRow* __restrict__ rows, int n_rows,
    int64_t T_arg, const float* __restrict__ xin, const int64_t* __restrict__ cur_hid, InetNrOutputs out, int rb_arg,
    int n_ul_max, InetNrArrivals arr, InetNrCells cl) {
    INET_PH_DECL
    InetNrParams pm = pm_in;
    InetNrTables tb = tb_in;
    if constexpr (FX == 1 || FX == 2) {
        pm.sched = 0; pm.comb = 1; pm.eesm = 1; pm.harq_drop = 0; pm.olla = 1; pm.phr_cap = 1; pm.retx_prio = 1;
        pm.rician = FX == 1 ? 1 : 0; pm.fading = 1;
        pm.pf_rbg = 0; pm.pf_freeze = 0; pm.whole_band = 0; pm.pc1_on = 0; pm.retx_tdma = 0; pm.amc_prev = 0;
        pm.fc_on = 0; pm.los_sto = 0; pm.k_from_los = 0; pm.doppler = 0; pm.pf_wb = 0;
    }
    constexpr bool DL = !std::is_same<LS, InetNrState>::value;
    // the link whose MAC state the kernel runs: the UL link is the shared state itself (one set of pointers)
    const LS& lk = [&]() -> const LS& { if constexpr (DL) return lk_in; else return st; }();
    constexpr bool MC = NC > 1;
    static_assert(!(MC && (DL || VREF)), "several cells: the UL with pose input");
    constexpr int W = RBT > STEP_WAVE ? RBT / STEP_WAVE : 1;   // wavefronts per env (1, 2 or 4)
    static_assert(W == 1 || W == 2 || W == 4, "envs of up to 64, 128 or 256 robots");
    constexpr int CW = STEP_WAVE * W;                   // lanes per workgroup (the LDS column stride)
    static_assert(!(MC && W > 1), "several cells: one wavefront per env");
    constexpr int NCS = NC * S;                        // fading links per robot (cell-major, subband-minor)
    const int rb = RBT ? RBT : rb_arg;
    const int64_t T = T_arg >= 0 ? T_arg : st.clock[0];
    extern __shared__ int dyn[];
    __shared__ __align__(16) float s_thr[MAX_M];
    __shared__ __align__(16) float s_thrs[MAX_M];                // suffix minima of s_thr (the MCS search table)
    __shared__ __align__(16) float s_se[MAX_M];
    __shared__ float s_beta[MAX_M], s_rbeta[MAX_M], s_rate[MAX_M];
    __shared__ float s_w[S], s_logw[S], s_wdb[S], s_lnw[S + 1];
    // frequency-correlated fading: the subband correlation's square root (general build only)
    __shared__ float s_fcl[FX == 0 ? S * S : 1];
    const bool fc = FX == 0 && pm.fc_on != 0;
    const bool fc2 = FX == 0 && pm.fc_on == 2;         // per-link delay spreads: L = fc_tab[the robot's grid index]
    const bool dop = FX == 0 && pm.doppler != 0;       // per-robot Doppler: rho = rho_ms^(row.rho) per robot
    // the batched product of the reference accumulates separately rounded products while S S 2 < 400, fused above
    constexpr bool FC_SEQ = S * S * 2 < 400;
    __shared__ int s_eq[IR ? MAX_M * MAX_EQW : 1];              // HARQ-IR equivalent MCS (IR builds only)
    __shared__ int s_ulrel[MAX_UL_ROWS];
    // per-lane rows: fading normals (2 NC S), RBG SINR in dB (S); several cells: rows S .. S + NC S hold each lane's
    // interference terms at every (cell, RBG) during a UL slot
    __shared__ __align__(16) float s_x[2 * NCS * CW];
    __shared__ float s_lin[S * CW];                              // per-lane rows: linear RBG SINR
    __shared__ int s_la_i[2 * CW], s_la_slot[CW], s_la_top[CW];  // link adaptation work list
    __shared__ float s_la_f[3 * CW];
    // robots that draw fading innovations this slot: (lane, hash offset of the robot's first element, env key)
    __shared__ uint4 s_dlist[CW];
    __shared__ float s_rkey[W > 1 ? CW : 1];                     // W = 2: retransmission ranking keys and RBG counts
    __shared__ int s_rval[W > 1 ? CW : 1];
    __shared__ int s_xw[4 * W];                                  // W > 1: the waves' values of an env collective
    // several cells, one env per wavefront: the interference pairs of a UL slot (robot lane | RBG << 8 | serving cell
    // << 16, then the fading state (re, im) on every cell); at most one holder per (cell, RBG)
    __shared__ float s_ipair[MC ? NC * S * (1 + 2 * NC) : 1];
    __shared__ float s_ipsd[MC ? NC * STEP_WAVE : 1];            // several cells: each robot's PSD at every cell

    const int lane = threadIdx.x;
    const int wbase = lane & ~(STEP_WAVE - 1), wl = lane - wbase;   // this lane's wavefront (base lane) and lane in it
    const int envs_pw = CW / rb;
    const int eloc = lane / rb;
    const int e = blockIdx.x * envs_pw + eloc;
    const int r = lane & (rb - 1);
    const int R = pm.R, E = pm.E, F = pm.F, N = pm.N;
    const bool act = (e < E) && (r < R);
    const int ee = e < E ? e : E - 1;
    const int rr0 = r < R ? r : 0;
    const uint32_t o_r0 = (uint32_t)(ee * R + rr0) * 4u;           // [E][R] element of this robot
    const uint32_t o_sr0 = (uint32_t)(ee * S * R + rr0) * 4u;      // [E][S][R] at s = 0 (row stride R)
    const uint32_t o_pr0 = (uint32_t)(ee * P * R + rr0) * 4u;      // [E][P][R] at p = 0
    const uint32_t o_fr0 = (uint32_t)(ee * F * R + rr0) * 4u;      // [E][F][R] at f = 0
    const uint32_t o_r = o_r0, o_sr = o_sr0, o_pr = o_pr0;
    const int HB = pm.max_tx + 1;
    int* const ack_l = dyn;
    int* const exlo_l = dyn + n_ul_max * CW;
    int* const exhi_l = dyn + 2 * n_ul_max * CW;
    int* const hist_l = dyn + (pm.harq_drop ? 3 : 1) * n_ul_max * CW;
    int* const my_hist = hist_l + eloc * 3 * HB;
    // several cells: each gNB's N+I estimate [NC][S] and this slot's interference [NC][S] of this lane's env
    float* const s_ni = reinterpret_cast<float*>(hist_l + envs_pw * 3 * HB) + eloc * 2 * NCS;
    float* const s_if = s_ni + NCS;

    // ---------------- env-wide collectives: inside the segment (W = 1), or over the W waves of the env through LDS
    // behind one barrier that every wave reaches. Successive exchanges alternate between two buffers: a wave writes a
    // buffer again only two exchanges later, after a barrier that the other waves reach once they have read it.
    int xbuf = 0;
    auto xchgw = [&](int v, int (&vals)[W]) {          // v: uniform in each wave; vals: every wave's, in wave order
        int* const b = s_xw + 2 * W * xbuf;
        xbuf ^= 1;
        if (wl == 0) b[lane >> 6] = v;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < W; ++w) vals[w] = b[w];
    };
    auto env_any = [&](bool p) -> bool {
        if constexpr (RBT == 32) {
            return lane_bit(seg32_any(__ballot(p)));
        } else if constexpr (W == 1) {
            return seg_any(p, rb, lane);
        } else {
            int a[W];
            xchgw(__ballot(p) != 0ull ? 1 : 0, a);
            int any = 0;
#pragma unroll
            for (int w = 0; w < W; ++w) any |= a[w];
            return any != 0;
        }
    };
    auto env_sum = [&](int v) -> int {
        if constexpr (W == 1) {
            return bsum(v, rb);
        } else {
            int a[W];
            xchgw(bsum(v, STEP_WAVE), a);
            int sum = 0;
#pragma unroll
            for (int w = 0; w < W; ++w) sum += a[w];
            return sum;
        }
    };

    // ---------------- load per-robot state (issued first: the loads are in flight while the tables are staged) ----
    int sent = 0, floor_ = 0, bsr = 0, sr_t = -1, last_tx = -1, enq = 0, qlen = 0;
    float olla = 0.f, avg = 100.f;
    float csi[S], hr[NCS], hi[NCS];
    uint32_t hmeta[P];
    int hlo[P], hhi[P], hrdy[P], htbs[P];
    float hcomb[P], hlexp[IR ? P : 1], hnrb[IR ? P : 1];
    const bool read_h = pm.fading && !(n_rows > 0 && (rows[0].flags & 4) && rows[0].rho == 0.0f);
    // (lanes without a robot read a clamped, valid address and discard the value: the loads are branch-free)
    sent = ldo(lk.sent, o_r); floor_ = ldo(lk.floor_, o_r);
    if constexpr (!DL) { bsr = ldo(st.bsr, o_r); sr_t = ldo(st.sr_t, o_r); }
    last_tx = ldo(lk.last_tx, o_r); enq = ldo(lk.enq, o_r); qlen = ldo(lk.qlen, o_r);
    olla = ldo(lk.olla, o_r); avg = ldo(lk.avg, o_r);
    qlen = qlen < 0 ? 0 : (qlen > F ? F : qlen);
    if (!act) { sent = 0; floor_ = 0; bsr = 0; sr_t = -1; last_tx = -1; enq = 0; qlen = 0; olla = 0.f; avg = 100.f; }
    const uint32_t o_hr0 = (uint32_t)(ee * NCS * R + rr0) * 4u;   // [E][NC S][R] at q = 0
#pragma unroll
    for (int s = 0; s < S; ++s) {
        csi[s] = ldo(lk.csi + s * R, o_sr);
        if (!act) csi[s] = 0.f;
    }
#pragma unroll
    for (int q = 0; q < NCS; ++q) {
        hr[q] = 0.f; hi[q] = 0.f;
        if (read_h && act) { hr[q] = ldo(st.h_re + q * R, o_hr0); hi[q] = ldo(st.h_im + q * R, o_hr0); }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int pr = p * R;
        hmeta[p] = ldo(lk.h_meta + pr, o_pr); hlo[p] = ldo(lk.h_lo + pr, o_pr); hhi[p] = ldo(lk.h_hi + pr, o_pr);
        hrdy[p] = ldo(lk.h_ready + pr, o_pr); htbs[p] = ldo(lk.h_tbs + pr, o_pr); hcomb[p] = ldo(lk.h_comb + pr, o_pr);
        if constexpr (IR) { hlexp[p] = ldo(lk.h_lexp + pr, o_pr); hnrb[p] = ldo(lk.h_nrb + pr, o_pr); }
        if (!act) {
            hmeta[p] = 0u; hlo[p] = 0; hhi[p] = 0; hrdy[p] = 0; htbs[p] = 0; hcomb[p] = 0.f;
            if constexpr (IR) { hlexp[p] = -INFINITY; hnrb[p] = 0.f; }
        }
    }
    // Rician state of every robot-cell link c ([E][NC][R]): specular phasor, K target kk, ramp start kf and slot kg
    float sp_re[NC], sp_im[NC], kk[NC], kf[NC];
    int kg[NC];
    auto o_rc = [&](int c) -> uint32_t { return (uint32_t)((ee * NC + c) * R + rr0) * 4u; };
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        sp_re[c] = 0.f; sp_im[c] = 0.f; kk[c] = 0.f; kf[c] = 0.f; kg[c] = 0;
        if (pm.rician && act) {
            sp_re[c] = ldo(st.spec_re, o_rc(c)); sp_im[c] = ldo(st.spec_im, o_rc(c)); kk[c] = ldo(st.k_lin, o_rc(c));
        }
    }
    // K from the LOS state (general build)
    const bool kl = FX == 0 && pm.k_from_los != 0;
#pragma unroll
    for (int c = 0; c < NC; ++c)
        if (kl && act) { kf[c] = ldo(st.k_from, o_rc(c)); kg[c] = ldo(st.k_g0, o_rc(c)); }
    int fci[NC];                                       // per-link delay spreads: each link's grid index in use
#pragma unroll
    for (int c = 0; c < NC; ++c) fci[c] = (fc2 && act) ? ldo(st.fc_idx, o_rc(c)) : 0;
    float lnp = 0.f;                                   // PRBs of the last PUSCH (ul_amc_alloc "previous")
    if (!DL && pm.amc_prev && act) lnp = ldo(st.last_nprb, o_r);
    // ---------------- stage the per-MCS and per-RBG tables in LDS ----------------
    if (lane < MAX_M) s_thr[lane] = lane <= tb.mcs_max ? tb.thr_ref[lane] : INFINITY;
    if (lane < MAX_M) s_se[lane] = lane < tb.M ? tb.se[lane] : 0.0f;
    if (lane < tb.M) {
        s_beta[lane] = tb.beta[lane];
        s_rbeta[lane] = 1.0f / tb.beta[lane];
        s_rate[lane] = tb.rate[lane];
    }
    // reciprocals of the BLER table's grid steps (div_const)
    const float rds = 1.0f / tb.ds, rdc = 1.0f / tb.dc;
    if (lane < S) { s_w[lane] = tb.w[lane]; s_logw[lane] = tb.logw[lane]; s_wdb[lane] = tb.wdb[lane]; }
    if constexpr (IR)
        for (int i = lane; i < tb.M * tb.EQW; i += CW) s_eq[i] = tb.mcs_eq[i];
    for (int i = lane; i < envs_pw * 3 * HB; i += CW) hist_l[i] = 0;
    // the step's rows, one per lane of each wavefront (n_rows <= 64), loaded together: the UL data rows' slots
    // in order (a ballot prefix), the last UL row, the last row whose fading state is kept, and whether every
    // evolving row is i.i.d. (rho = 0)
    unsigned long long m_ul, m_h, m_corr;
    {
        const bool have = wl < n_rows;                 // (each wavefront of the workgroup reads the rows)
        const int fl = have ? rows[wl].flags : 0;
        const int rel_l = have ? rows[wl].rel : 0;
        const float rho_l = have ? rows[wl].rho : 0.0f;
        m_ul = __ballot((fl & 2) != 0);
        m_h = __ballot((fl & 4) != 0 && (fl & 8) != 0);
        m_corr = __ballot((fl & 4) != 0 && rho_l != 0.0f);
        if (wbase == 0 && (fl & 2)) s_ulrel[__builtin_popcountll(m_ul & ((1ull << wl) - 1ull))] = rel_l;
    }
    __syncthreads();
    // "the highest m <= mcs_max with x >= thr[m]" is the highest m with x >= min(thr[m..mcs_max]): these suffix
    // minima are non-decreasing, so a binary search over them gives the linear scan's result for any table. Past
    // mcs_max the entries are NaN, which no comparison passes (not even x = +inf).
    // (a suffix-minimum scan over lanes 0..31, every lane taking part in the lane reads)
    {
        float v = (wl < MAX_M && wl <= tb.mcs_max) ? s_thr[wl] : INFINITY;
#pragma unroll
        for (int off = 1; off < MAX_M; off <<= 1) {
            const float o = __shfl_down(v, off, 64);
            v = wl + off < MAX_M ? fminf(v, o) : v;
        }
        if (lane < MAX_M) s_thrs[lane] = lane <= tb.mcs_max ? v : __builtin_nanf("");
    }
    // log of the held PRB count by count of held RBGs, when every RBG has the same width: the log-sum-exp over the
    // held RBGs then adds exp(0) = 1 once per RBG, so it depends only on that count (s_lnw[n])
    if (lane <= S) s_lnw[lane] = lse_logw<S>(s_logw, lane >= 32 ? ~0u : ((1u << lane) - 1u));
    if (fc && !fc2)
        for (int i = lane; i < S * S; i += blockDim.x) s_fcl[i] = pm.fc_L[i];
    bool lw_eq = true;
#pragma unroll
    for (int s = 1; s < S; ++s) lw_eq = lw_eq && s_logw[s] == s_logw[0];
    __syncthreads();

    // the step's arrivals (inet_nr_submit_step): FrameQueue.add / NRNet.add_frames of every message, class by class
    // (queues.py:87-103, nr_engine.py:466-487), at the tail of the FIFO, before the slots
    if constexpr (!DL) {
        if (arr.counts != nullptr && act) {
            int n_acc = 0;
            const size_t ci0 = ((size_t)ee * R + rr0) * (size_t)arr.n_cls;
            for (int c = 0; c < arr.n_cls; ++c) {
                const int nmsg = arr.counts[ci0 + c];
                float size = arr.sizes[c];
                if (arr.pkt_overhead) size = size + ceilf(size / (float)arr.pkt_payload) * (float)arr.pkt_overhead;
                const int nb = (int)rintf(size);
                for (int k = 0; k < nmsg; ++k) {
                    bool adm = true;
                    if (arr.discard_pdcp && qlen > 0 && (int)T - ldo(lk.q_cap, o_fr0) >= pm.timeout) adm = false;
                    if (adm && qlen < F && size > 0.0f) {
                        const int fr = qlen * R;
                        sto(lk.q_cap + fr, o_fr0, (int)T); sto(lk.q_start + fr, o_fr0, enq);
                        sto(lk.q_end + fr, o_fr0, enq + nb); sto(lk.q_fin + fr, o_fr0, (int)FIN_NONE);
                        sto(lk.q_meta + fr, o_fr0, (uint32_t)(c + 1) << 8); sto(st.q_hid + fr, o_fr0, 0);
                        enq += nb;
                        ++qlen;
                        ++n_acc;
                    }
                }
            }
            if (arr.accepted) sto(arr.accepted, o_r, n_acc);
        }
    }
    // several cells: association of this robot, the N+I estimates of its env (LDS), the env's interference statistic
    int serv = 0, a3_cand = -1, a3_cnt = 0, ho_end = 0, n_ho = 0;
    float ion = 0.f;
    // radio link failure (cl.rlf): the robot's RLF state machine (CellAssociation, radio.py:456-531) and its counts
    // of this step (rlf, reest, rlf_idle, t310_start, t310_stop)
    bool rlf_on = false;
    int oos_cnt = 0, is_cnt = 0, t310_end = -1, t311_end = -1, reest_end = -1, reest_cell = 0, n_rlf = 0;
    int c_rl[5] = {0, 0, 0, 0, 0};
    if constexpr (MC) {
        if (act) {
            serv = ldo(cl.serv, o_r); a3_cand = ldo(cl.a3_cand, o_r); a3_cnt = ldo(cl.a3_cnt, o_r);
            ho_end = ldo(cl.ho_end, o_r); n_ho = ldo(cl.n_ho, o_r);
            serv = serv < 0 ? 0 : (serv >= NC ? NC - 1 : serv);   // (indexes LDS rows: kept in range)
            if (cl.rlf) {
                rlf_on = ldo(cl.rlf_active, o_r) != 0; oos_cnt = ldo(cl.oos_cnt, o_r); is_cnt = ldo(cl.is_cnt, o_r);
                t310_end = ldo(cl.t310_end, o_r); t311_end = ldo(cl.t311_end, o_r); reest_end = ldo(cl.reest_end, o_r);
                reest_cell = ldo(cl.reest_cell, o_r); n_rlf = ldo(cl.n_rlf, o_r);
                reest_cell = reest_cell < 0 ? 0 : (reest_cell >= NC ? NC - 1 : reest_cell);
            }
        }
        if (e < E) {
            for (int q = r; q < NCS; q += rb) s_ni[q] = cl.ni_ul[(size_t)ee * NCS + q];
            if (r == 0) ion = cl.ion[ee];
        }
        __syncthreads();
    }

    // ---------------- inputs: SINR reference per subband and the reported SNR ----------------
    // the DL reference SINR per PRB (NRNet.step_rx / step, nr_engine.py:624-631, 651-653): with poses the gNB PSD
    // over the reciprocal path gain against the UE noise; with SNR input the input plus dl_snr_offset_db (or the DL
    // SNR as given)
    float ref[(VREF || MC) ? S : 1];
    float snr_out = 0.f;
    float pgc[NC];                                 // several cells: path gain to every cell (dB)
    // the stochastic LOS state of TR 38.901 (general build only)
    const StoLos sto_los{pm.los_cdf, pm.plos_scn, pm.sig_nlos, FX == 0 && pm.los_sto != 0};
    bool los_now = false, los_rep = false;         // this step's LOS state of the link (TR 38.901 with poses)
    bool los_c[NC];                                // several cells: that of every robot-cell link
#pragma unroll
    for (int c = 0; c < NC; ++c) los_c[c] = false;
    // per-robot Doppler (engine.py:862-864, radio.py:285-300): the robot's AR(1) correlation per ms, set anew by a pose
    // step from its speed (|vel|, else |pose - last pose| / control step, 0 right after a reset; floored); the DL step
    // derives the same value from the state the UL step then updates
    float rho_ms = 0.f;
    if (dop && act) rho_ms = ldo(st.rho_ms, o_r);
    auto observe_motion = [&](float px, float py) {
        if (!dop || !act) return;
        float v;
        if (pm.vel) {
            const float vx = ldo(pm.vel, o_r * 2u), vy = ldo(pm.vel + 1, o_r * 2u);
            v = sqrtf(fmaf(vy, vy, vx * vx));          // (torch's norm over the last two: x x, then fused y y +)
        } else {
            const float dx = px - ldo(st.prev_pos, o_r * 2u), dy = py - ldo(st.prev_pos + 1, o_r * 2u);
            v = sqrtf(fmaf(dy, dy, dx * dx)) / pm.dop_dt;
            if (ldo(st.has_prev, o_r) == 0) v = 0.f;
        }
        v = v < pm.dop_floor ? pm.dop_floor : v;    // (clamp(min): NaN stays NaN)
        rho_ms = inet::doppler_rho_ms(v, pm.dop_kf, pm.dop_kx);
        if constexpr (!DL) {
            sto(st.rho_ms, o_r, rho_ms);
            sto(st.prev_pos, o_r * 2u, px);
            sto(st.prev_pos + 1, o_r * 2u, py);
            sto(st.has_prev, o_r, 1);
        }
    };
    if constexpr (MC) {
        if (pm.input_kind == 3) {
            // the path gain of every robot-cell link as given, [E][R][NC] dB (step(pathgain_db=), engine.py:909-915):
            // no radio, so no LOS state and no motion
#pragma unroll
            for (int c = 0; c < NC; ++c) pgc[c] = act ? ldo(xin + c, o_r * (uint32_t)NC) : 0.f;
        } else {
            // RadioMC.pathgain_db of every robot-cell link (radio.py:238-277); the UL reference is set per UL slot
            float px = 0.f, py = 0.f;
            if (act) { px = ldo(xin, o_r * 2u); py = ldo(xin + 1, o_r * 2u); }
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float* fc = st.field + ((size_t)ee * NC + c) * pm.n_fields * pm.n_modes * 3;
                pgc[c] = radio_rx_dbm(pm, px, py, cl.gnb_xy[2 * c], cl.gnb_xy[2 * c + 1], fc, sto_los, &los_c[c]) -
                         pm.ue_tx;
            }
            observe_motion(px, py);
            los_rep = pm.radio_model == 1;
        }
#pragma unroll
        for (int s = 0; s < S; ++s) ref[s] = 0.f;
    } else if constexpr (VREF) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            ref[s] = act ? ldo(xin + s, o_r * S) : 0.f;
            if constexpr (DL) ref[s] = lk.snr_offset ? ref[s] + lk.snr_off : ref[s];
        }
        if constexpr (!DL) snr_out = aten_sum<S>(ref) / (float)S;
    } else if (pm.input_kind == 1) {
        ref[0] = act ? ldo(xin, o_r) : 0.f;
        if constexpr (DL) ref[0] = lk.snr_offset ? ref[0] + lk.snr_off : ref[0];
        snr_out = ref[0];
    } else {                                       // poses -> path gain (radio prologue)
        float px = 0.f, py = 0.f;
        if (act) { px = ldo(xin, o_r * 2u); py = ldo(xin + 1, o_r * 2u); }
        const float rx = radio_rx_dbm(pm, px, py, pm.gnb_x, pm.gnb_y,
                                      st.field + (size_t)ee * pm.n_fields * pm.n_modes * 3, sto_los, &los_now);
        observe_motion(px, py);
        los_rep = pm.radio_model == 1;
        const float pg = rx - pm.ue_tx;
        if constexpr (DL) ref[0] = (pg + lk.ref_off) - lk.noise_prb;
        else ref[0] = (pg + pm.ref_off) - pm.noise_prb;
        snr_out = (pg + pm.ue_tx) - pm.subband_noise;
    }
    auto REF = [&](int s) -> float { return (VREF || MC) ? ref[s] : ref[0]; };
    // PHR cap n_max (mac_ul.py:165-168): ref.mean(-1) -> snr_ref_prbs 10^((ref - phr_min) / 10) / w0 (several cells:
    // from the serving link's noise-only SNR at every UL slot)
    int n_max = S;
    if (!DL && !MC && pm.phr_cap && !pm.whole_band) {
        float rr[S];
#pragma unroll
        for (int s = 0; s < S; ++s) rr[s] = REF(s);
        float mref = aten_sum<S>(rr) / (float)S;
        float nmp = pm.snr_ref_prbs * from_db(mref - pm.phr_min);
        float f = floorf(nmp / pm.w0);
        f = clampf(f, 1.0f, (float)S);
        n_max = (int)f;
    }
    // UL power control at one cell (nr_engine.py:649-650, 671-675): the backoff from the full power over snr_ref_prbs
    // PRBs to the PSD P0 + alpha PL, the path loss from the mean UL reference SINR
    float pc1 = -INFINITY;
    if (!DL && !MC && pm.pc1_on) {
        float rr[S];
#pragma unroll
        for (int s = 0; s < S; ++s) rr[s] = REF(s);
        const float rx = aten_sum<S>(rr) / (float)S + pm.subband_noise;
        pc1 = pm.ue_tx - (pm.pc_p0 + pm.pc_alpha * (pm.ue_tx - rx));
    }
    const bool use_pc = MC || pm.pc1_on;           // (several cells: cl.pc_on, -inf backoff when off)

    // ---------------- counter RNG key of this env and step ----------------
    uint32_t base0 = 0;
    if (e < E) {
        uint32_t h = mix32((uint32_t)pm.seed_key ^ salt32((uint32_t)st.env_id[e]));
        h = mix32(h ^ salt32((uint32_t)st.episode[e]));
        h = mix32(h ^ salt32(CH_STEP));
        base0 = mix32(h ^ salt32((uint32_t)st.ctr_step[e]));
    }

    // per-robot counters of this step (summed over the segment at the end)
    int c_new = 0, c_retx = 0, c_ok = 0, c_fail = 0, c_exh = 0, c_new_pend = 0;
    int c_bytes_ok = 0, c_bytes_new = 0, c_prb = 0;
    int c_tbb = 0, c_tbe = 0, c_blk = 0;               // 5G-LENA grant accounting: TB bytes, empty TBs, TDMA blocks
    const bool lena = pm.pf_rbg || pm.pf_freeze || pm.retx_tdma || pm.amc_prev;   // (kept with a LENA switch on)

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

    int n_ul = 0;
    int nf = 0, lost_dl = 0;                      // DL: first frame not yet resolved, frames lost under RLC UM
    const int g0 = (int)(T * (int64_t)N);

    // ---------------- Rician K of the link (nr_engine.py:370-419, 602-611) ----------------
    // K of slot g on the ramp: the target once k_ramp slots have begun since kg, else k_from + (target - k_from) n / k_ramp
    auto k_at = [&](int c, int g) -> float {
        const int n = g - kg[c] + 1;
        return n >= pm.k_ramp ? kk[c] : kf[c] + (kk[c] - kf[c]) * ((float)n * pm.k_rinv);
    };
    // NRNet.set_los with this step's LOS state (target k_los where LOS, else 0; an env's first state since its reset
    // applies at once), then _rician_update at g0 (a changed target starts a ramp from the K of slot g0 - 1)
    // NRNet.set_los for the delay spread (nr_engine.py:377-381): the link's LOS or NLOS grid index
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const bool lc = MC ? los_c[c] : los_now;
        if (fc2 && los_rep && act) fci[c] = lc ? ldo(st.fc_idl, o_rc(c)) : ldo(st.fc_idn, o_rc(c));
        fci[c] = fci[c] < 0 ? 0 : (fci[c] < pm.fc_G ? fci[c] : pm.fc_G - 1);
    }
    if (kl && los_rep) {
        const bool fresh = act && st.k_fresh[ee] != 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const bool lc = MC ? los_c[c] : los_now;
            const float kt = (act && lc) ? ldo(st.k_los, o_rc(c)) : 0.f;
            if (fresh) { kk[c] = kt; kf[c] = kt; }
            else if (pm.k_ramp == 0) kk[c] = kt;
            else if (kt != kk[c]) { kf[c] = k_at(c, g0 - 1); kg[c] = g0; kk[c] = kt; }
        }
    }
    // gain coefficients inv = 1 / (K + 1), sqrt(K inv), sqrt(inv); while a ramp runs, set again in every slot
    float ka[NC], kb[NC];
    auto set_k = [&](int c, float k) {
        const float kinv = 1.0f / (k + 1.0f);
        ka[c] = sqrtf(k * kinv);
        kb[c] = sqrtf(kinv);
    };
#pragma unroll
    for (int c = 0; c < NC; ++c) set_k(c, kk[c]);
    const bool k_ramps = kl && pm.k_ramp > 0;

    // ---------------- several cells: association and the A3 plan of this step (CellAssociation, radio.py:410-437) ----
    // rx = path gain + ue_tx (RSRP up to a constant); a pending env attaches every robot to its max-rx cell; the A3
    // condition (best other cell > (serving + offset) + hysteresis, and above the admission floor) held toward the same
    // target for ttt slots fires at slot k_ho = ttt - cnt - 1 of this step when that is inside the step
    int k_ho = -1, tgt = 0;
    bool fired = false;
    // frames that handovers and radio link failures drop in this step: a mask over the robot's FIFO and the UL slot
    // (0 .. n_ul) before which it applies, replayed in order by the epilogue so that frames completed earlier keep
    // their completion (at most three per step: a handover; or T311's idling or an RLF, then a re-establishment)
    constexpr int ND = MC ? 3 : 1;
    unsigned long long drop_m[ND];
    int drop_j[ND];
    int n_drop = 0;
#pragma unroll
    for (int i = 0; i < ND; ++i) { drop_m[i] = 0ull; drop_j[i] = 0; }
    // The MAC side of a handover (UlMac.handover, mac_ul.py:238-247, mac.py:557-581; also of an RLF, a
    // re-establishment and idling, NRNet._rlf_links, nr_engine.py:684-689): under RLC UM or with flush the frames
    // overlapping the undecoded HARQ bytes (flush: every queued frame) are lost, marked when the epilogue replays the
    // UL slots, and those processes are freed; otherwise they restart their combining at the target. OLLA, the PF
    // average and the CSI start afresh; the BSR reaches the target, a pending SR is dropped.
    auto link_handover = [&](bool flush) {
        if (pm.harq_drop || flush) {
            unsigned long long mk = 0ull;
            if (flush) {
                mk = qlen >= 64 ? ~0ull : ((1ull << qlen) - 1ull);
            } else {
                for (int f = 0; f < qlen; ++f) {
                    const int qs = ldo(lk.q_start + f * R, o_fr0), qe = ldo(lk.q_end + f * R, o_fr0);
                    bool ov = false;
#pragma unroll
                    for (int p = 0; p < P; ++p) ov |= hm_state(hmeta[p]) == 1 && qs < hhi[p] && qe > hlo[p];
                    if (ov) mk |= 1ull << f;
                }
            }
#pragma unroll
            for (int i = 0; i < ND; ++i)
                if (i == n_drop || (i == ND - 1 && n_drop >= ND)) {
                    drop_m[i] |= mk;                   // (a fourth event would join the third: never reached)
                    if (i == n_drop) drop_j[i] = n_ul;
                }
            n_drop = n_drop < ND ? n_drop + 1 : ND;
            if (flush) sent = enq;
#pragma unroll
            for (int p = 0; p < P; ++p)
                if (hm_state(hmeta[p]) == 1) hmeta[p] = hm_pack(0, hm_ntx(hmeta[p]), hm_mcs(hmeta[p]), hm_nsb(hmeta[p]));
        } else {
#pragma unroll
            for (int p = 0; p < P; ++p) {
                if (hm_state(hmeta[p]) == 1) {
                    hmeta[p] = hm_pack(1, 0, hm_mcs(hmeta[p]), hm_nsb(hmeta[p]));
                    hcomb[p] = 0.f;
                    if constexpr (IR) { hlexp[p] = -INFINITY; hnrb[p] = 0.f; }
                }
            }
        }
        olla = 0.f;
        avg = 100.f;
#pragma unroll
        for (int s = 0; s < S; ++s) csi[s] = 0.f;
        if constexpr (!DL) { sr_t = -1; bsr = enq - sent; }
    };
    // NRNet._handover at slot g_sw (nr_engine.py:677-682): the switch (radio.py:439-448; with RLF it stops T310 and
    // the indication counts), then the MAC side with ho_rlc's flush
    auto handover = [&](int g_sw) {
        serv = tgt;
        ho_end = g_sw + cl.ho_int;
        ++n_ho;
        fired = true;
        if (cl.rlf) {
            c_rl[4] += t310_end >= 0 ? 1 : 0;
            t310_end = -1;
            oos_cnt = 0;
            is_cnt = 0;
        }
        link_handover(cl.ho_flush != 0);
    };
    // radio link failure: the SINR estimate toward every cell at the step start (nr_engine.py:704-707), the cell search
    // (radio.py:503-519: the max-RSRP cell whose estimate reaches qin and whose RSRP the floor, re-establishment reest
    // slots after slot g), and the events due by slot g (NRNet._rlf_events, nr_engine.py:691-702: T310 expiries not
    // preceded by a handover declare RLF, then the re-establishments due complete); returns the handover due by g
    float sinr_c[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) sinr_c[c] = 0.f;
    auto rlf_search = [&](int g, bool mask) {
        bool any = false;
        int bc = 0;
        float bv = -INFINITY;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float rxv = pgc[c] + pm.ue_tx;
            const bool ok = sinr_c[c] >= cl.qin && (!cl.has_floor || rxv >= cl.floor_rx);
            any |= ok;
            const float v = ok ? rxv : -INFINITY;
            if (c == 0 || v > bv) { bv = v; bc = c; }
        }
        if (mask && rlf_on && reest_end < 0 && any) { reest_end = g + cl.reest; reest_cell = bc; }
    };
    auto rlf_events = [&](int g) -> bool {
        if (!act) return false;
        const int g_ho = g0 + k_ho;
        const bool ho = !fired && k_ho >= 0 && g_ho <= g;
        const bool ex = t310_end >= 0 && t310_end <= g && !rlf_on && !(ho && g_ho <= t310_end);
        if (ex) {                                      // CellAssociation.declare (radio.py:486-501)
            const int g_rlf = t310_end;
            rlf_on = true;
            t311_end = g_rlf + cl.t311;
            t310_end = -1;
            reest_end = -1;
            oos_cnt = 0;
            is_cnt = 0;
            a3_cnt = 0;
            a3_cand = -1;
            ++n_rlf;
            ++c_rl[0];
            rlf_search(g_rlf, true);
            link_handover(cl.rlf_flush != 0);
            fired = true;
        }
        if (rlf_on && reest_end >= 0 && reest_end <= g) {   // CellAssociation.complete (radio.py:521-531)
            serv = reest_cell;
            rlf_on = false;
            t311_end = -1;
            reest_end = -1;
            ++c_rl[1];
            link_handover(false);
        }
        return ho && !rlf_on && !ex;
    };
    if constexpr (MC) {
        float rxc[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) rxc[c] = pgc[c] + pm.ue_tx;
        if (act && cl.pending[ee] != 0) {
            int b = 0;
            float bv = rxc[0];
#pragma unroll
            for (int c = 1; c < NC; ++c) if (rxc[c] > bv) { bv = rxc[c]; b = c; }
            serv = b;
        }
        if (cl.rlf && act) {
            // radio link monitoring at the step's first slot (nr_engine.py:733-736, radio.py:456-480): the SINR
            // estimate toward every cell against its gNB's latest wideband N+I estimate (the serving one is the
            // serving link's), ((pg + ue_tx) - ref_db) - 10 log10(mean_s ni)
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                float nrow[S];
#pragma unroll
                for (int s2 = 0; s2 < S; ++s2) nrow[s2] = s_ni[c * S + s2];
                sinr_c[c] = ((pgc[c] + pm.ue_tx) - cl.ref_db) - 10.0f * log10f(aten_sum<S>(nrow) / (float)S);
            }
            const float sinr_s = sel_of(sinr_c, serv);
            const bool idle = rlf_on && reest_end < 0 && t311_end >= 0 && t311_end <= g0;
            if (idle) { t311_end = -1; ++c_rl[2]; }
            rlf_search(g0, rlf_on);
            const bool conn = !rlf_on;
            const bool oos = conn && cl.qout > sinr_s, ins = conn && sinr_s > cl.qin;
            const bool run = t310_end >= 0;
            const int oc = ins ? 0 : oos_cnt + (oos ? 1 : 0);
            const bool start = conn && !run && oc >= cl.n310;
            const int ic = oos ? 0 : is_cnt + (ins ? 1 : 0);
            const bool stop = run && ic >= cl.n311;
            oos_cnt = (run || start || !conn) ? 0 : oc;
            is_cnt = (run && !stop) ? ic : 0;
            t310_end = start ? g0 + cl.t310 : (stop ? -1 : t310_end);
            c_rl[3] += start ? 1 : 0;
            c_rl[4] += stop ? 1 : 0;
            if (idle) link_handover(true);             // the idle robot's queue is dropped (nr_engine.py:736)
        }
        if (act) {
            const float rs = sel_of(rxc, serv);
            float best = 0.f;
            int bc = 0;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float v = c == serv ? -INFINITY : rxc[c];
                if (c == 0 || v > best) { best = v; bc = c; }
            }
            bool cond = best > ((rs + cl.a3_off) + cl.a3_hyst);
            if (cl.has_floor) cond = cond && best >= cl.floor_rx;
            if (cl.rlf) cond = cond && !rlf_on;       // no measurement reporting while in RLF
            const int cnt = (cond && bc == a3_cand) ? a3_cnt : 0;
            int kf = cl.ttt - cnt - 1;
            kf = kf > 0 ? kf : 0;
            const bool fire = cond && kf < N;
            a3_cnt = (cond && !fire) ? cnt + N : 0;
            a3_cand = (cond && !fire) ? bc : -1;
            k_ho = fire ? kf : -1;
            tgt = bc;
        }
    }
    // i.i.d. fading (rho = 0 at every evolving row): a robot's fading state and CSI are then pure functions of the
    // latest draw, so a robot with nothing to send and no HARQ process pending (it takes part in no decision for the
    // rest of the step) skips the draws until the last row that fixes the stored state (the last UL slot for the CSI,
    // the last row needing the state for h)
    const int last_ul_row = m_ul ? 63 - __builtin_clzll(m_ul) : -1;
    const int last_h_row = m_h ? 63 - __builtin_clzll(m_h) : -1;
    const bool iid = m_corr == 0ull;
    INET_PH(0);                                    // prologue: tables, state loads, arrivals, radio
    // ================================================================ slot loop
    for (int k = 0; k < n_rows; ++k) {
        const InetNrRow row = rows[k];
        const int g = g0 + row.rel;
        if (k_ramps) {
#pragma unroll
            for (int c = 0; c < NC; ++c) set_k(c, k_at(c, g));
        }
        if constexpr (MC) {                        // A3 handovers due by this slot (nr_engine.py:740-754)
            const bool ho_now = cl.rlf ? rlf_events(g) : (act && !fired && k_ho >= 0 && k_ho <= row.rel);
            if (ho_now) handover(g0 + k_ho);
        }
        if ((row.flags & 4) && (row.flags & 8)) {  // AR(1) fading innovation of this slot (nr_engine.py:575-589)
            // The 2 NC S normals of every robot that needs them are drawn cooperatively by the whole wavefront: the
            // (robot, link) pairs are dealt round-robin over the 64 lanes, each pair's two normals land in the
            // robot's LDS column (s_x), and the robot then updates its own state. Normal j = 2 NC S r + 2 q + {0, 1}
            // (link q = c S + s of cell c and subband s; real, imaginary part) uses hash elements 2j, 2j + 1.
            bool busy = false;
#pragma unroll
            for (int p = 0; p < P; ++p) busy |= hm_state(hmeta[p]) == 1;
            busy |= (enq - sent) > 0;
            // (the DL draws every robot's gain at its CQI rows, which set the CSI of every robot)
            const bool full = !iid || (DL ? (row.flags & 1) != 0 : (k == last_ul_row || k == last_h_row));
            const bool draw = act && (full || busy);
            const unsigned long long need = __ballot(draw);              // (per wave: each draws its own robots)
            float* const s_z = s_x;
            // the env's key of this slot, and the hash input of the robot's first element (robot r's normals start at
            // element 2 NC S r, hash element 2 (2 NC S r) = 4 NC S r)
            const uint32_t bf = mix32(base0 ^ row.salt_fade);
            if (draw)
                s_dlist[wbase + __builtin_popcountll(need & ((1ull << wl) - 1ull))] =
                    make_uint4((uint32_t)lane, bf + (uint32_t)(4 * r * NCS) * GOLD, bf, 0u);
            __syncthreads();
            // pairs in subband-major order: the lanes of one pass write different robots' columns (no LDS bank
            // conflicts between the pairs of one robot)
            const int n_need = __builtin_popcountll(need);
            const int items = n_need * NCS;
            // item it = q n_need + ri (subband q of the ri-th drawing robot); a lane's items are 64 apart, so (q, ri)
            // advance by (dq, dr) with one carry, the subband's hash term 4 q GOLD with them, and the next item's
            // robot is read from the list ahead of its use
            int q = 0, ri = 0, dq = 0, dr = 0;
            uint32_t qterm = 0u, dqterm = 0u;
            uint4 ent = make_uint4(0u, 0u, 0u, 0u);
            if (n_need > 0) {
                dq = STEP_WAVE / n_need;
                dr = STEP_WAVE - dq * n_need;
                q = wl / n_need;
                ri = wl - q * n_need;
                qterm = (uint32_t)(4 * q) * GOLD;
                dqterm = (uint32_t)(4 * dq) * GOLD;
                ent = s_dlist[wbase + ri];
            }
#pragma unroll 1
            for (int it = wl; it < items; it += STEP_WAVE) {
                const int Lc = (int)ent.x, qc = q;
                const uint32_t hin = ent.y + qterm, bfc = ent.z;
                q += dq;
                ri += dr;
                qterm += dqterm;
                if (ri >= n_need) { ri -= n_need; ++q; qterm += 4u * GOLD; }
                ent = s_dlist[wbase + ri];                    // (ri < n_need: a valid entry, read for the next item)
                const float zr = normal_of(mix32(mix32(hin) ^ bfc), mix32(mix32(hin + GOLD) ^ bfc));
                const float zi = normal_of(mix32(mix32(hin + 2u * GOLD) ^ bfc), mix32(mix32(hin + 3u * GOLD) ^ bfc));
                // the innovation term sqrt(1 - rho^2) z / sqrt(2) of the AR(1) step, ready for the robot's update
                // (frequency-correlated fading: z itself, correlated by the robot first; per-robot Doppler: z, scaled
                // by the robot's own coefficient)
                s_z[(2 * qc) * CW + Lc] = (fc || dop) ? zr : div_const(row.c1 * zr, SQRT2_F, INV_SQRT2_F);
                s_z[(2 * qc + 1) * CW + Lc] = (fc || dop) ? zi : div_const(row.c1 * zi, SQRT2_F, INV_SQRT2_F);
            }
            INET_PH(1);                            // fading innovations (the robots' own updates follow)
            // the AR(1) coefficients: the row's, or with per-robot Doppler rho = rho_ms^(dt slot_ms) and
            // sqrt(1 - rho^2) of the robot (nr_engine.py:586-589)
            float rho_k = row.rho, c1_k = row.c1;
            if (dop) {
                rho_k = inet::pow_scalar_f32(rho_ms, row.rho);
                c1_k = sqrtf(1.0f - rho_k * rho_k);
            }
            __syncthreads();
            if (draw && fc2) {
                // per-link delay spreads: L = fc_tab[the link's grid index] (nr_engine.py:365-368), read from global
                // memory (the table is a few KB, cached); the reference's batched product accumulates separately
                // rounded products while S S 2 < 400 and fused ones above
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    uint32_t lo0 = (uint32_t)fci[c] * (uint32_t)(S * S * 4);   // byte offset of the link's L
                    asm volatile("" : "+v"(lo0));      // (recomputed here: no per-row offsets kept across the slots)
#pragma unroll
                    for (int i = 0; i < S; ++i) {
                        float ar = 0.f, ai = 0.f;
#pragma unroll 1
                        for (int j = 0; j <= i; ++j) {
                            const float l = ldo(pm.fc_tab, lo0 + (uint32_t)((i * S + j) * 4));
                            const float zr = s_z[(2 * (c * S + j)) * CW + lane];
                            const float zi = s_z[(2 * (c * S + j) + 1) * CW + lane];
                            if constexpr (FC_SEQ) { ar = ar + l * zr; ai = ai + l * zi; }
                            else { ar = fmaf(l, zr, ar); ai = fmaf(l, zi, ai); }
                        }
                        const int q = c * S + i;
                        hr[q] = rho_k * hr[q] + div_const(c1_k * ar, SQRT2_F, INV_SQRT2_F);
                        hi[q] = rho_k * hi[q] + div_const(c1_k * ai, SQRT2_F, INV_SQRT2_F);
                    }
                }
            } else if (draw && fc) {
                // z <- L z over the subbands of every link (L lower-triangular; the products accumulated with fused
                // multiply-adds in subband order, as a float32 matrix product), then the AR(1) step
                // (the draws are read from LDS term by term: no register copy of the S draws of a link)
#pragma unroll
                for (int c = 0; c < NC; ++c) {
#pragma unroll
                    for (int i = 0; i < S; ++i) {
                        float ar = 0.f, ai = 0.f;
#pragma unroll 1
                        for (int j = 0; j <= i; ++j) {
                            const float l = s_fcl[i * S + j];
                            ar = fmaf(l, s_z[(2 * (c * S + j)) * CW + lane], ar);
                            ai = fmaf(l, s_z[(2 * (c * S + j) + 1) * CW + lane], ai);
                        }
                        const int q = c * S + i;
                        hr[q] = rho_k * hr[q] + div_const(c1_k * ar, SQRT2_F, INV_SQRT2_F);
                        hi[q] = rho_k * hi[q] + div_const(c1_k * ai, SQRT2_F, INV_SQRT2_F);
                    }
                }
            } else if (draw && dop) {
#pragma unroll
                for (int q = 0; q < NCS; ++q) {
                    hr[q] = rho_k * hr[q] + div_const(c1_k * s_z[(2 * q) * CW + lane], SQRT2_F, INV_SQRT2_F);
                    hi[q] = rho_k * hi[q] + div_const(c1_k * s_z[(2 * q + 1) * CW + lane], SQRT2_F, INV_SQRT2_F);
                }
            } else if (draw) {
#pragma unroll
                for (int q = 0; q < NCS; ++q) {
                    hr[q] = row.rho * hr[q] + s_z[(2 * q) * CW + lane];
                    hi[q] = row.rho * hi[q] + s_z[(2 * q + 1) * CW + lane];
                }
            }
        }
        // fading gain (dB) of subband s of the serving link in this slot (nr_engine.py:602-611; several cells: the
        // serving cell's, pick(gain_c, serv)), and of link (c, s) (gain_cs)
        // (the powers are finite and clamped to at least 1e-6, where log10_pos is log10f)
        // power of link q = c S + s: |sqrt(K inv) e^{j phi} + sqrt(inv) h|^2 with Rician fading, else |h|^2
        auto power_cs = [&](int q, bool rician) -> float {
            const int c = q / S;
            if (rician) {
                const float xr = ka[c] * sp_re[c] + kb[c] * hr[q];
                const float xi = ka[c] * sp_im[c] + kb[c] * hi[q];
                return xr * xr + xi * xi;
            }
            return hr[q] * hr[q] + hi[q] * hi[q];
        };
        auto power_of = [&](int s, bool rician) -> float {
            if constexpr (MC) {
                float p = power_cs(s, rician);
#pragma unroll
                for (int c = 1; c < NC; ++c) {
                    const float pc_ = power_cs(c * S + s, rician);
                    p = serv == c ? pc_ : p;
                }
                return p;
            } else if (rician) {
                return power_cs(s, true);
            } else {
                return hr[s] * hr[s] + hi[s] * hi[s];
            }
        };
        auto gain_of = [&](int s) -> float {
            return pm.fading ? 10.0f * log10_pos(clamp_min(power_of(s, pm.rician), 1e-6f)) : 0.0f;
        };
        // every subband's gain into g[S], the mode tests hoisted out of the subband loop
        auto gains_of = [&](float (&gv)[S]) {
            if (!pm.fading) {
#pragma unroll
                for (int s = 0; s < S; ++s) gv[s] = 0.0f;
            } else if (pm.rician) {
#pragma unroll
                for (int s = 0; s < S; ++s) gv[s] = 10.0f * log10_pos(clamp_min(power_of(s, true), 1e-6f));
            } else {
#pragma unroll
                for (int s = 0; s < S; ++s) gv[s] = 10.0f * log10_pos(clamp_min(power_of(s, false), 1e-6f));
            }
        };
        auto gain_cs = [&](int q) -> float {
            return pm.fading ? 10.0f * log10_pos(clamp_min(power_cs(q, pm.rician), 1e-6f)) : 0.0f;
        };
        if constexpr (DL) {
            if (row.flags & 1) {                   // CQI report (DlMac.cqi_report, mac_dl.py:30-40)
                // per subband the best MCS at ref + gain (mcs_at: the highest m <= mcs_max with x >= thr_ref[m], else
                // 0), or the 38.214 CQI mapped back to an MCS; the gNB keeps that MCS's threshold as its estimate
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const float x = REF(s) + gain_of(s);
                    int m = 0;
                    if (lk.cqi_thr) {
                        int q = 0;
                        for (int j = 0; j < 15; ++j) q += x >= lk.cqi_thr[j] ? 1 : 0;
                        m = lk.cqi_mcs[q];
                    } else {
                        for (int j = 0; j <= tb.mcs_max; ++j) m = x >= s_thr[j] ? j : m;
                    }
                    csi[s] = s_thr[m] - REF(s);
                }
            }
        } else {
            if (row.flags & 1) {                   // SR opportunity (UlMac.sr_step, lumped)
                if ((enq - sent) > 0 && bsr <= 0 && sr_t < 0) sr_t = g;
            }
        }
        if (!(row.flags & 2)) { INET_PH(2); continue; }
        // ============================ data slot (MacLink.slot) ============================
        // several cells (nr_engine.py:757-766): the UL reference of the serving link per subband against the serving
        // gNB's N+I estimate, the PHR cap from its noise-only SNR, the power-control backoff, this row's cells
        float pc = pc1;
        float ni_la[MC ? S : 1];
        unsigned long long mycell = 0ull;
        if constexpr (MC) {
            const float pg_s = sel_of(pgc, serv);
#pragma unroll
            for (int s = 0; s < S; ++s) {
                ni_la[s] = 10.0f * log10f(s_ni[serv * S + s]);
                ref[s] = (pm.ref_off + pg_s) - ni_la[s];
            }
            const float rx_s = pg_s + pm.ue_tx;
            if (cl.pc_on) pc = pm.ue_tx - (cl.pc_p0 + cl.pc_alpha * (pm.ue_tx - rx_s));
            n_max = S;
            if (pm.phr_cap && !pm.whole_band) {
                const float phr = rx_s - pm.subband_noise;
                float f = floorf((pm.snr_ref_prbs * from_db(phr - pm.phr_min)) / pm.w0);
                n_max = (int)clampf(f, 1.0f, (float)S);
            }
            unsigned long long cm[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) cm[c] = __ballot(act && serv == c);
            mycell = sel_of(cm, serv) & seg_bits(rb, lane);
        }
        // any lane of this lane's scheduler (its env's segment; several cells: the env's robots of its cell)
        auto cell_any = [&](bool p) -> bool {
            if constexpr (MC) return (__ballot(p) & mycell) != 0ull;
            else return env_any(p);
        };
        // true in the lane that wins the RBG with bid m (-1: no bid) in its scheduler: the highest bid, the first
        // robot on ties (torch max)
        auto winner = [&](int m) -> bool {
            if constexpr (MC) {
                int v[NC];
#pragma unroll
                for (int c = 0; c < NC; ++c) v[c] = serv == c ? m : -1;
                bmax_n<NC>(v, rb);
                const int mx = sel_of(v, serv);
                const unsigned long long b = (__ballot(m == mx) & mycell) >> (lane & ~(rb - 1));
                return m >= 0 && b != 0ull && (int)__builtin_ctzll(b) == r;
            } else if constexpr (W > 1) {
                // each wave's max and its first lane holding it; the env's winner is the first wave's on ties
                const int mxw = bmax_i(m, STEP_WAVE);
                const int fw = (int)__builtin_ctzll(__ballot(m == mxw));
                int* const b = s_xw + 2 * W * xbuf;       // (alternating buffers, as xchgw)
                xbuf ^= 1;
                if (wl == 0) { b[2 * (lane >> 6)] = mxw; b[2 * (lane >> 6) + 1] = fw; }
                __syncthreads();
                int best = b[0], at = b[1];
#pragma unroll
                for (int w = 1; w < W; ++w)
                    if (b[2 * w] > best) { best = b[2 * w]; at = STEP_WAVE * w + b[2 * w + 1]; }
                return m >= 0 && lane == at;
            } else if constexpr (RBT == 32) {
                // the first lane of each 32-lane segment holding the maximum, found on the scalar unit
                const int mx = bmax_i(m, 32);
                return m >= 0 && lane_bit(seg32_lowest(__ballot(m == mx)));
            } else {
                const int mx = bmax_i(m, rb);
                const int f = seg_first(m == mx, rb, lane);             // (every lane takes part in the ballot)
                return m >= 0 && f == r;
            }
        };
        const int unsent = enq - sent;
        if constexpr (DL) {
            // DL processes whose HARQ-ACK has reached the gNB become free (mac.py:243)
#pragma unroll
            for (int p = 0; p < P; ++p)
                if (hm_state(hmeta[p]) == 2 && hrdy[p] <= g)
                    hmeta[p] = hm_pack(0, hm_ntx(hmeta[p]), hm_mcs(hmeta[p]), hm_nsb(hmeta[p]));
        } else {
            // grants (UlMac._pre_slot_lumped)
            if (row.flags & 16) bsr = bsr > 1 ? bsr : 1;
            if (sr_t >= 0 && g - sr_t >= pm.sr_delay) { bsr = bsr > 1 ? bsr : 1; sr_t = -1; }
        }
        // candidates: the retransmission ready first (lowest ready slot, then lowest process), the lowest free process
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
        const int need = DL ? unsent : (bsr < unsent ? bsr : unsent);
        bool new_el = any_free && need > 0 && !has_rx && act;
        has_rx = has_rx && act;
        if constexpr (MC) {                        // handover interruption (mac.py:249-251, radio.py:450-453)
            const bool ok_ = g >= ho_end && !rlf_on;
            has_rx = has_rx && ok_;
            new_el = new_el && ok_;
        }
        int rx_nsb = 0;
#pragma unroll
        for (int p = 0; p < P; ++p) rx_nsb = p == rx_p ? hm_nsb(hmeta[p]) : rx_nsb;
        // Scheduler estimate with OLLA -> MCS -> rate -> metric per RBG (mac_ul.py:154-171, mac.py:256-275), for the
        // robots that can bid in this slot (a retransmission ready or new data with a free process; the others'
        // rates and metrics are never read). Each such robot writes its estimate row to LDS; the (robot, RBG) pairs
        // are then dealt round-robin over the wavefront (subband-major, as the fading draws), and each pair's MCS,
        // rate and metric land in the robot's LDS columns: the metric in rows 0..S-1 of s_x, the rate in s_lin (free
        // until link adaptation). s_la_slot and s_la_f (the link adaptation work list) hold the list and the PF
        // average or RR age until then.
        float* const s_met = s_x;
        float* const s_eo = s_x + S * CW;
        float* const s_rt = s_lin;
        {
            const bool bid0 = has_rx || new_el;
            if (bid0) {
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    // UL: the PSD over one RBG, at most the power-control PSD (mac_ul.py:154-171); DL: sinr_ref + csi
                    // (mac_dl.py:42-43)
                    // (ul_power "whole_band": the fixed PSD over the carrier, mac_ul.py:157-160)
                    const float wdb = pm.whole_band ? pm.wb_db : s_wdb[s];
                    const float wd = use_pc ? (wdb > pc ? wdb : pc) : wdb;
                    const float est = DL ? REF(s) + csi[s] : (REF(s) - wd) + csi[s];
                    s_eo[s * CW + lane] = pm.olla ? est + olla : est;
                }
                s_la_f[lane] = pm.sched == 0 ? clamp_min(avg, 1e-9f) : (float)(g - last_tx);
            }
            const unsigned long long bm = __ballot(bid0);
            const int n_b = __popcll(bm);
            if (bid0) s_la_slot[wbase + __popcll(bm & ((1ull << wl) - 1ull))] = lane;
            // highest m <= mcs_max with eo >= thr[m] (0 when none, or NaN): a binary search over the suffix minima,
            // whose first three levels compare with seven values held by every lane, then a count of the values
            // passed in the last block of four
            const float t16 = s_thrs[16], t8 = s_thrs[8], t24 = s_thrs[24];
            const float t4 = s_thrs[4], t12 = s_thrs[12], t20 = s_thrs[20], t28 = s_thrs[28];
            auto mcs_search = [&](float e) -> int {
                int m = e >= t16 ? 16 : 0;
                m += e >= (m ? t24 : t8) ? 8 : 0;
                m += e >= (m < 16 ? (m < 8 ? t4 : t12) : (m < 24 ? t20 : t28)) ? 4 : 0;
                return m + (e >= s_thrs[m + 1] ? 1 : 0) + (e >= s_thrs[m + 2] ? 1 : 0) + (e >= s_thrs[m + 3] ? 1 : 0);
            };
            // the wideband rate (mac.py:259-264): the MCS of every bidding robot from its effective SINR over every
            // RBG (general build only), into s_la_top (free until link adaptation)
            const bool wbr = FX == 0 && pm.pf_wb != 0;
            if (wbr) {
                const uint32_t all = (1u << S) - 1u;
                const float lnw_all = lw_eq ? s_lnw[S] : lse_logw<S>(s_logw, all);
                if (!pm.eesm) {
                    // mean_db: the PRB-weighted mean of the estimate over every RBG, then the highest MCS it reaches
                    if (bid0) s_la_top[lane] = mcs_search(mean_db_held<S, CW>(s_eo, lane, s_logw, all, lnw_all));
                } else {
                    // EESM: for every MCS m <= mcs_max, -beta_m (lse_s((-lin_s) / beta_m + log w_s) - lnw) in dB
                    // against thr_ref[m]; the (robot, MCS) items are dealt over the wavefront and each passing item
                    // sets its bit in the robot's mask (an LDS atomic OR); the robot takes the highest bit (0: none)
                    bool nanr = false;
                    if (bid0) {
#pragma unroll
                        for (int s2 = 0; s2 < S; ++s2) {
                            const float x = s_eo[s2 * CW + lane];
                            nanr |= x != x;
                            s_lin[s2 * CW + lane] = from_db_mid(clampf(x, -30.0f, 60.0f));
                        }
                    }
                    s_la_top[lane] = 0;
                    s_la_i[lane] = nanr ? 1 : 0;
                    __syncthreads();
                    const int nm = tb.mcs_max + 1;
#pragma unroll 1
                    for (int it = wl; it < n_b * nm; it += STEP_WAVE) {
                        const int mi = it / n_b, L = s_la_slot[wbase + (it - mi * n_b)];
                        const float beta = s_beta[mi];
                        const float eff = db_of((-beta) * (lse_eesm<S>([&](int s2) { return s_lin[s2 * CW + L]; },
                                                                         s_logw, all, beta, s_rbeta[mi],
                                                                         s_la_i[L] != 0) - lnw_all));
                        if (eff >= s_thr[mi]) atomicOr(&s_la_top[L], 1 << mi);
                    }
                    __syncthreads();
                    const int mk = s_la_top[lane];
                    if (bid0) s_la_top[lane] = mk ? 31 - __builtin_clz((uint32_t)mk) : 0;
                }
            }
            __syncthreads();
            const int items = n_b * S;
            int q = 0, ri = 0, dq = 0, dr = 0;
            if (n_b > 0) {
                dq = STEP_WAVE / n_b;
                dr = STEP_WAVE - dq * n_b;
                q = wl / n_b;
                ri = wl - q * n_b;
            }
#pragma unroll 1
            for (int it = wl; it < items; it += STEP_WAVE) {
                const int L = s_la_slot[wbase + ri], qc = q;
                q += dq;
                ri += dr;
                if (ri >= n_b) { ri -= n_b; ++q; }
                const float e = s_eo[qc * CW + L];
                if (wbr) {
                    // the wideband rate: (se[m] re_prb / 8) w_s, in the reference's order
                    const float rt = ((s_se[s_la_top[L]] * row.re_prb) / 8.0f) * s_w[qc];
                    const float a = s_la_f[L];
                    s_met[qc * CW + L] = pm.sched == 0 ? DivBy(a)(rt) : (pm.sched == 1 ? rt : a);
                    s_rt[qc * CW + L] = rt;
                    continue;
                }
                int m = e >= t16 ? 16 : 0;
                m += e >= (m ? t24 : t8) ? 8 : 0;
                m += e >= (m < 16 ? (m < 8 ? t4 : t12) : (m < 24 ? t20 : t28)) ? 4 : 0;
                // the block's search values and spectral efficiencies, read together (the empty asm keeps the
                // values in registers, so that the selection below stays branch-free)
                float4 tq = *reinterpret_cast<const float4*>(&s_thrs[m]);
                float4 gq = *reinterpret_cast<const float4*>(&s_se[m]);
                asm("" : "+v"(tq.y), "+v"(tq.z), "+v"(tq.w), "+v"(gq.x), "+v"(gq.y), "+v"(gq.z), "+v"(gq.w));
                const int k = (e >= tq.y ? 1 : 0) + (e >= tq.z ? 1 : 0) + (e >= tq.w ? 1 : 0);
                float se = gq.x;
                se = k >= 1 ? gq.y : se;
                se = k >= 2 ? gq.z : se;
                se = k >= 3 ? gq.w : se;
                const float rt = ((se * row.re_prb) * s_w[qc]) / 8.0f;
                // the metric (mac.py:267-275): PF rate / max(avg, 1e-9) (rates in [0, 2^20], the average in
                // [1e-9, 2^40]: DivBy gives the IEEE quotient), max C/I the rate, RR the age
                const float a = s_la_f[L];
                const float mt = pm.sched == 0 ? DivBy(a)(rt) : (pm.sched == 1 ? rt : a);
                s_met[qc * CW + L] = mt;
                s_rt[qc * CW + L] = rt;
            }
            __syncthreads();
        }
        auto metric_of = [&](int s) -> float { return s_met[s * CW + lane]; };
        INET_PH(2);                                // SR / CQI, grants, candidates, estimate, MCS, rate, metric
        // retransmission admission (mac.py:300-313): rank by the metric sum inside each scheduler, admit while the RBG
        // counts fit (the segment's total fitting implies every cell's)
        if (!DL && pm.retx_tdma) {
            // ul_retx_sched "tdma" (mac.py:279-299): one retransmission per scheduler, the oldest NACK (the lowest
            // ready slot of the robot's ready process, the first robot on ties), alone in its slot: the scheduler
            // takes no new data. (Ready slots are non-negative, so the bid is too.)
            const bool adm = winner(has_rx ? 0x7fffffff - best_rdy : -1);
            const bool blk = cell_any(adm);
            c_blk += (adm && rx_nsb < S) ? 1 : 0;
            new_el = new_el && !blk;
            has_rx = adm;
        } else {
            // Ranked by the metric sum, descending (rkey = -1 for the robots that are not candidates of the
            // scheduler), the candidates taken while their RBG counts fit. The order is torch's argsort: ATen's
            // comparator (a NaN key first, then the larger), and for keys it holds equal the order std::sort leaves
            // them in. Up to 16 robots that is the index order (insertion sort); above, a scheduler whose candidates
            // hold equal keys takes the sort's own steps (aten_sort.h, rank_exact below).
            const bool cand = has_rx;
            bool tie = false, ranked = false;
            float rkey = -1.0f;
            if (env_any(has_rx)) {
                int val = has_rx ? rx_nsb : 0;
                int tot = env_sum(val);
                if (tot > S) {
                    ranked = true;
                    float mt[S];
#pragma unroll
                    for (int s = 0; s < S; ++s) mt[s] = metric_of(s);
                    rkey = has_rx ? aten_sum<S>(mt) : -1.0f;
                    int cum = 0;
                    const int sb = lane & ~(rb - 1);
                    if constexpr (W > 1) {             // the env's keys and counts through LDS
                        s_rkey[lane] = rkey;
                        s_rval[lane] = val;
                        __syncthreads();
                    }
#pragma unroll 1
                    for (int j = 0; j < rb; ++j) {
                        float kj;
                        int vj;
                        if constexpr (W > 1) { kj = s_rkey[j]; vj = s_rval[j]; }
                        else { kj = __shfl(rkey, sb + j, 64); vj = __shfl(val, sb + j, 64); }
                        bool same = true;
                        if constexpr (MC) same = __shfl(serv, sb + j, 64) == serv;
                        const bool fwd = AtenSortDesc::comp(kj, rkey), bwd = AtenSortDesc::comp(rkey, kj);
                        cum += (same && (fwd || (!bwd && j <= r))) ? vj : 0;
                        tie |= same && has_rx && vj > 0 && j != r && !fwd && !bwd;
                    }
                    has_rx = has_rx && cum <= S;
                }
            }
            // rank_exact: one lane per (env, scheduler) sorts the env's keys with std::sort's steps (the reference's
            // tensor: the keys of the scheduler's candidates, -1 elsewhere, robots 0..R-1) in LDS (rows S.. of s_x,
            // free between the estimate and the allocation), walks the sorted order and marks the candidates whose
            // running RBG count fits. (Wave-uniform: every env of the wavefront takes part when any env needs it.)
            bool exact = false;
            if constexpr (W == 1) exact = rb > 16 && __ballot(tie) != 0ull;
            else if (ranked) exact = env_any(tie);          // (W > 1: one env per workgroup, `ranked` is uniform)
            if (exact) {
                const int XS = NC * 3 * rb + rb + NC * 64;   // ints per env: NC (keys, indices, counts), marks, stacks
                int* const xs = reinterpret_cast<int*>(s_x + S * CW) + eloc * XS;
                int* const mark = xs + NC * 3 * rb;
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const bool in_c = cand && (!MC || serv == c);
                    reinterpret_cast<float*>(xs)[c * 3 * rb + r] = in_c ? rkey : -1.0f;
                    xs[c * 3 * rb + rb + r] = r;
                    xs[c * 3 * rb + 2 * rb + r] = in_c ? rx_nsb : 0;
                }
                mark[r] = 0;
                __syncthreads();
                if (r < NC && e < E && ranked) {
                    int* const kc = xs + r * 3 * rb;
                    AtenSortDesc srt{reinterpret_cast<float*>(kc), kc + rb};
                    srt.sort(R, mark + rb + r * 64);
                    int run = 0;
                    for (int i = 0; i < R; ++i) {
                        const int j = kc[rb + i];
                        const int v = kc[2 * rb + j];
                        run += v;
                        if (v > 0) mark[j] = run <= S ? 1 : 0;
                    }
                }
                __syncthreads();
                if (ranked) has_rx = cand && mark[r] != 0;
            }
        }
        INET_PH(3);                                // retransmission admission
        const int want_cnt = has_rx ? rx_nsb : (new_el ? n_max : 0);
        // RBG-by-RBG allocation (mac.py:322-352); the metric row is read into registers first, so that no bid waits
        // for its LDS read
        const float prio = pm.retx_prio ? (has_rx ? 1e9f : 0.0f) : 0.0f;
        float mrow[S], rate[S];                         // the bids' values (metric + retransmission priority), rates
#pragma unroll
        for (int s = 0; s < S; ++s) {
            mrow[s] = metric_of(s) + prio;
            rate[s] = s_rt[s * CW + lane];
            asm volatile("" : "+v"(mrow[s]), "+v"(rate[s]));
        }
        int cnt = 0;
        float left = (float)need;
        uint32_t won = 0;
        // pf_update "rbg" (mac.py:325-329, 526-532): the metric of RBG s is rate_s / max(base + wwin got, 1e-9) with
        // base = (1 - wwin) avg and got the rate of the RBGs this robot won so far in the slot
        const float pf_base = pm.pf_a * avg;
        float got = 0.f;
        auto rbg_metric = [&](int s) { return DivBy(clamp_min(pf_base + pm.pf_b * got, 1e-9f))(rate[s]); };
        // (one copy of the loop per retx-priority setting, so that the test is not repeated per RBG)
        auto allocate = [&](auto retx_prio) {
            constexpr bool RP = decltype(retx_prio)::value;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const bool want = (cnt < want_cnt) && (has_rx || left > 0.0f);
                // bid key: the bit pattern of the non-negative metric (ordered like the float), -1 for no bid
                int m = want ? __float_as_int(pm.pf_rbg ? rbg_metric(s) + prio : mrow[s]) : -1;
                if constexpr (RP) {
                    const bool wr = want && has_rx;
                    if (cell_any(wr) && !wr) m = -1;
                }
                // argmax over the robots of the scheduler, first robot on ties (torch argmax); -1: no bid
                const bool sel = winner(m);
                if (sel) { won |= 1u << s; ++cnt; }
                if (pm.pf_rbg && sel) got = got + rate[s];
                left = left - ((sel && !has_rx) ? rate[s] : 0.0f);
            }
        };
        // (the lexicographic mask only acts where some robot of the scheduler has an admitted retransmission)
        if (pm.retx_prio && (W > 1 || __ballot(has_rx) != 0ull)) allocate(std::true_type{});
        else allocate(std::false_type{});
        if (!pm.retx_prio) {                          // release short retransmissions (mac.py:353-379)
            bool short_ = has_rx && (__popc(won) != rx_nsb);
            uint32_t rel_rs = short_ ? won : 0u;
            if (short_) won = 0u;
            cnt = __popc(won);
#pragma unroll
            for (int s = 0; s < S; ++s) {
                bool avs = cell_any((rel_rs >> s) & 1u);
                bool want = (cnt < want_cnt) && new_el && (left > 0.0f);
                const float ms = pm.pf_rbg ? rbg_metric(s) : metric_of(s);
                const int m = want ? __float_as_int(ms) : -1;
                const bool sel = winner(m) && avs;
                if (sel) { won |= 1u << s; ++cnt; }
                if (pm.pf_rbg && sel) got = got + rate[s];
                left = left - (sel ? rate[s] : 0.0f);
            }
        }
        INET_PH(4);                                // RBG-by-RBG allocation
        const int n_sb = __popc(won);
        float n_prb = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) n_prb += ((won >> s) & 1u) ? s_w[s] : 0.0f;
        const bool tx_rx = has_rx && n_sb == rx_nsb && n_sb > 0;
        const bool tx_new = new_el && n_sb > 0;
        const bool tx = tx_rx || tx_new;
        // power split (mac_ul.py:173-180): PUSCH power spread over n_prb PRBs, at least the power-control backoff
        const float sp0 = pm.whole_band ? pm.wb_db : 10.0f * log10_clamped(clamp_min(n_prb / pm.snr_ref_prbs, 1e-3f));
        const float sp = use_pc ? (sp0 > pc ? sp0 : pc) : sp0;
        // log of the held PRB count as torch computes it: logsumexp of log w over the held RBGs
        const float lnw = lw_eq ? s_lnw[__popc(won)] : lse_logw<S>(s_logw, won);
        // The (robot lane, RBG) pairs of the robots with `who` over the RBGs they hold, in lane order, into this wave's
        // part of pl ([64 S] entries per wave: lane | RBG << 8); returns this wave's count. Per-RBG work on the held
        // RBGs (at most S per scheduler, against S per robot) is then dealt over the wavefront.
        auto build_pairs = [&](bool who, uint32_t msk, int* pl) -> int {
            int n;
            int off = wave_prefix64(who ? __popc(msk) : 0, wl, n);
            int* const wpl = pl + wbase * S;
#pragma unroll
            for (int s = 0; s < S; ++s)
                if (who && ((msk >> s) & 1u)) wpl[off++] = lane | (s << 8);
            return n;
        };
        // lse_eesm (the EESM log-sum over the held RBGs) of every robot with `who`, for its dB row xv and MCS mc: the
        // pairs' terms (-lin_s) / beta + log w_s and then exp(term - max) are computed on the pair list; each robot
        // takes the max and the ATen-order sum over its own RBGs (the RBGs it does not hold add exact zeros), which are
        // lse_held's steps. Called by every lane (barriers); the result is read in the lanes with `who`. LDS: the dB
        // rows in s_x rows S..2S-1, the pair list in rows 0..S-1, terms in s_lin, the MCS and max in s_la_i / s_la_f.
        auto held_lse = [&](bool who, const float (&xv)[S], int mc, bool nanv) -> float {
            float* const s_dx = s_x + S * CW;
            int* const s_pl = reinterpret_cast<int*>(s_x);
            if (who) {
#pragma unroll
                for (int s = 0; s < S; ++s) s_dx[s * CW + lane] = xv[s];
                s_la_i[lane] = mc;
            }
            const int n_pairs = build_pairs(who, won, s_pl);
            __syncthreads();
#pragma unroll 1
            for (int it = wl; it < n_pairs; it += STEP_WAVE) {
                const int en = s_pl[wbase * S + it], L = en & 0xff, sq = en >> 8;
                const int m = s_la_i[L];
                const float lin = from_db_mid(clampf(s_dx[sq * CW + L], -30.0f, 60.0f));
                s_lin[sq * CW + L] = div_const(-lin, s_beta[m], s_rbeta[m]) + s_logw[sq];
            }
            __syncthreads();
            float mx = -INFINITY;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const float v = ((won >> s) & 1u) ? s_lin[s * CW + lane] : -INFINITY;
                mx = v > mx ? v : mx;
            }
            if (mx == INFINITY || mx == -INFINITY) mx = 0.f;
            s_la_f[lane] = mx;
            __syncthreads();
#pragma unroll 1
            for (int it = wl; it < n_pairs; it += STEP_WAVE) {
                const int en = s_pl[wbase * S + it], L = en & 0xff, sq = en >> 8;
                s_lin[sq * CW + L] = exp_nonpos(s_lin[sq * CW + L] - s_la_f[L]);
            }
            __syncthreads();
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < S; ++i) {
                const int sq = aten_unrot<S>(i);
                sum += ((won >> sq) & 1u) ? s_lin[sq * CW + lane] : 0.0f;
            }
            const float res = (sum == 0.0f ? -INFINITY : ln_unit(sum)) + mx;
            return nanv ? NAN : res;
        };
        // ---- link adaptation for new TBs (phy.select_mcs): the highest MCS meeting the BLER target ----
        int mcs_new = 0, tbs_new = 0;
        bool any_new;                                  // (W = 2: both waves enter, the search has barriers)
        if constexpr (W == 1) any_new = __ballot(tx_new) != 0ull;
        else any_new = env_any(tx_new);
        if (any_new) {
            // the RBGs the MCS is searched over: the held ones; ul_amc_alloc "previous" with whole-band power, every
            // RBG (mac.py:396)
            const bool la_all = !DL && pm.amc_prev && pm.whole_band;
            const uint32_t la_m = la_all ? (1u << S) - 1u : won;
            const float la_lnw = la_all ? (lw_eq ? s_lnw[S] : lse_logw<S>(s_logw, la_m)) : lnw;
            // estimated SINR per RBG: x_s = (ref_s - sp) + csi_s in dB, and its linear value on those RBGs
            bool nan = false;
            if (pm.eesm) {
                // the linear values on the pair list of the new TBs' held RBGs (the dB rows in s_x rows S..2S-1, the
                // list in rows 0..S-1; the search's first round passes a barrier before it reads s_lin)
                float* const s_ex = s_x + S * CW;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const float x = DL ? REF(s) + csi[s] : (REF(s) - sp) + csi[s];   // DL: the scheduler's estimate
                    nan |= x != x;
                    if (tx_new) s_ex[s * CW + lane] = x;
                }
                int* const s_pl = reinterpret_cast<int*>(s_x);
                const int n_pairs = build_pairs(tx_new, la_m, s_pl);
                __syncthreads();
#pragma unroll 1
                for (int it = wl; it < n_pairs; it += STEP_WAVE) {
                    const int en = s_pl[wbase * S + it], L = en & 0xff, sq = en >> 8;
                    s_lin[sq * CW + L] = from_db_mid(clampf(s_ex[sq * CW + L], -30.0f, 60.0f));
                }
            } else {
                const uint32_t held = tx_new ? la_m : 0u;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const float x = DL ? REF(s) + csi[s] : (REF(s) - sp) + csi[s];
                    nan |= x != x;
                    s_x[s * CW + lane] = x;                                  // (the mean-dB row)
                    if ((held >> s) & 1u) s_lin[s * CW + lane] = from_db_mid(clampf(x, -30.0f, 60.0f));
                }
            }
            const float eff_md = (!pm.eesm && tx_new) ? mean_db_held<S, CW>(s_x, lane, s_logw, la_m, la_lnw) : 0.f;
            const int np = (int)n_prb;
            const int toff = (row.nsym_idx * (tb.NPRB + 1) + np) * tb.M;
            // ul_amc_alloc "previous" (mac.py:393-401): the MCS is searched on the table row of the last PUSCH's PRB
            // count (this allocation's while there was none); the TB of the chosen MCS is this allocation's
            const int np_sel = (!DL && pm.amc_prev && lnp > 0.0f) ? (int)lnp : np;
            const int toff_sel = (row.nsym_idx * (tb.NPRB + 1) + np_sel) * tb.M;
            // The search for the highest MCS that meets the target is shared by the whole wavefront: every round,
            // each robot still searching gets 64 / n_searching lanes, which evaluate its next MCS candidates in
            // parallel (top, top - 1, ...); the robot takes the highest candidate that passes or moves its top down.
            // The result is the top-down scan's (phy.select_mcs takes the highest passing MCS), without its
            // divergent tail. A robot's inputs (table row, held RBGs, lnw, OLLA offset, mean_db value) and its
            // linear SINR row are read from LDS by its helpers.
            // (W = 2: each wave searches for its own robots; the rounds go on while either wave has robots left)
            s_la_i[lane] = toff_sel;
            s_la_i[CW + lane] = (int)(la_m | (nan ? 0x80000000u : 0u));
            s_la_f[lane] = la_lnw;
            s_la_f[CW + lane] = pm.olla ? olla : 0.0f;
            s_la_f[2 * CW + lane] = eff_md;
            int top = tb.mcs_max, found_m = -1, tbs_found = 0;
            bool mine = tx_new;
            unsigned long long searching = __ballot(mine);
            auto more = [&]() -> bool {
                if constexpr (W == 1) return searching != 0ull;
                else return env_any(searching != 0ull);
            };
            while (more()) {
                const int n_s = __popcll(searching);
                const int chunk = n_s ? STEP_WAVE / n_s : STEP_WAVE;
                const int rank = __popcll(searching & ((1ull << wl) - 1ull));
                if (mine) { s_la_slot[wbase + rank] = lane; s_la_top[lane] = top; }
                __syncthreads();
                const int slot = wl / chunk, j = wl - slot * chunk;
                bool pass = false;
                int tbs_c = 0;                             // this candidate's TBS (the winner's is the TB's)
                const int rl = slot < n_s ? s_la_slot[wbase + slot] : 0;
                const int m = slot < n_s ? s_la_top[rl] - j : -1;
                if (m >= 0) {
                    // the four table words are loaded first; the EESM (LDS and ALU only) runs while they arrive
                    const int ti = s_la_i[rl] + m;
                    const int tbs_m = tb.la_tbs[ti], ci0 = tb.la_ci0[ti];
                    const float cwi = tb.la_cwi[ti], ncb = tb.la_ncb[ti];
                    tbs_c = tbs_m;
                    float eff;
                    if (pm.eesm) {
                        const uint32_t wr = (uint32_t)s_la_i[CW + rl];
                        const float beta = s_beta[m];
                        eff = db_of((-beta) * (lse_eesm<S>([&](int s) { return s_lin[s * CW + rl]; }, s_logw,
                                                           wr & 0x7fffffffu, beta, s_rbeta[m], (wr >> 31) != 0u) -
                                               s_la_f[rl]));
                    } else {
                        eff = s_la_f[2 * CW + rl];
                    }
                    eff = eff + s_la_f[CW + rl];
                    if (tbs_m > 0) {
                        float b = bler_at(tb.bler, (m * tb.C + ci0) * tb.G, tb.G, tb.s0, tb.ds, rds, eff, cwi);
                        float tbler = 1.0f - pow_count(1.0f - b, ncb);
                        pass = tbler <= pm.target;
                    }
                }
                const unsigned long long pb = __ballot(pass);
                const unsigned long long cm =
                    mine ? (pb >> (rank * chunk)) & (chunk >= STEP_WAVE ? ~0ull : ((1ull << chunk) - 1ull)) : 0ull;
                // the passing candidate's TBS from the lane that evaluated it (every lane takes part in the read)
                const int tw = __shfl(tbs_c, wbase + rank * chunk + (cm ? (int)__builtin_ctzll(cm) : 0), 64);
                if (mine) {
                    if (cm) { found_m = top - (int)__builtin_ctzll(cm); tbs_found = tw; mine = false; }
                    else { top -= chunk; mine = top >= 0; }
                }
                searching = __ballot(mine);
                __syncthreads();
            }
            if (tx_new) {
                mcs_new = found_m >= 0 ? found_m : 0;
                // (searched on this allocation's table row: the TBS the search read; else the row's entry)
                tbs_new = (found_m >= 0 && toff_sel == toff) ? tbs_found : tb.la_tbs[toff + mcs_new];
            }
        }
        INET_PH(5);                                // link adaptation (power split, lse of log w, MCS search)
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
                    hcomb[p] = 0.f;
                    if constexpr (IR) { hlexp[p] = -INFINITY; hnrb[p] = 0.f; }
                }
                mcs = hm_mcs(hmeta[p]); tbs = htbs[p]; ntx = hm_ntx(hmeta[p]) + 1;
                comb_p = hcomb[p]; lo_tx = hlo[p]; hi_tx = hhi[p];
                if constexpr (IR) { lexp_p = hlexp[p]; nrb_p = hnrb[p]; }
            }
        }
        mcs = mcs < tb.M ? mcs : tb.M - 1;
        if (tx_new) sent = sent + byt_new;
        // ---- actual channel of this slot: fading gain per subband; in the UL it becomes the CSI (mac_ul.py:229-236)
        float gn[DL ? S : 1];
        if constexpr (DL) gains_of(gn);
        else gains_of(csi);
        // ---- several cells: same-slot UL interference (NRNet._ul_ici, nr_engine.py:799-816) ----
        // Every robot that transmits adds, at each other cell c and RBG s it holds, its received power
        // 10^((((pg_c + ue_tx) - ref_db) - split + gain_cs) / 10) (mW per PRB). Each lane writes its NC S terms (zeros
        // elsewhere) to its LDS column; one lane per (cell, RBG) of the env sums its column over the robots in torch's
        // order, and updates that gNB's N+I estimate (EWMA li_a now + li_b estimate) and the I/N statistic.
        if constexpr (MC) {
            if (cl.use_int) {
                const bool txing = tx && act;
                float* const s_t = s_x + S * STEP_WAVE;
                if (rb == STEP_WAVE) {
                    // one env per wavefront (at most NC S held (cell, RBG) pairs): the terms are computed
                    // cooperatively. The columns are cleared, every transmitting robot lists its held RBGs with its
                    // fading state on every cell, and the (RBG, other cell) terms of the list are dealt over the
                    // wavefront.
                    {
                        const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
                        for (int i = lane; i < NCS * STEP_WAVE / 4; i += STEP_WAVE)
                            reinterpret_cast<float4*>(s_t)[i] = z4;
                    }
                    int n_pairs;
                    int off = wave_prefix64(txing ? __popc(won) : 0, wl, n_pairs);
                    // the robot's PSD at every cell: ((pg_c + ue_tx) - ref_db) - split
                    float* const s_psd = s_ipsd;
#pragma unroll
                    for (int c = 0; c < NC; ++c) s_psd[c * STEP_WAVE + lane] = ((pgc[c] + pm.ue_tx) - cl.ref_db) - sp;
#pragma unroll
                    for (int s = 0; s < S; ++s) {
                        if (txing && ((won >> s) & 1u)) {
                            float* const ent = s_ipair + off * (1 + 2 * NC);
                            ent[0] = __int_as_float(lane | (s << 8) | (serv << 16));
                            // the link's complex gain whose power power_cs takes: with Rician fading the specular
                            // phasor and the scattered part at this slot's K (ka, kb), else the fading state
#pragma unroll
                            for (int c = 0; c < NC; ++c) {
                                const int q = c * S + s;
                                ent[1 + 2 * c] = pm.rician ? ka[c] * sp_re[c] + kb[c] * hr[q] : hr[q];
                                ent[2 + 2 * c] = pm.rician ? ka[c] * sp_im[c] + kb[c] * hi[q] : hi[q];
                            }
                            ++off;
                        }
                    }
                    __syncthreads();
#pragma unroll 1
                    for (int it = wl; it < n_pairs * (NC - 1); it += STEP_WAVE) {
                        const int pi = it / (NC - 1), k = it - pi * (NC - 1);
                        const float* const ent = s_ipair + pi * (1 + 2 * NC);
                        const uint32_t w = __float_as_uint(ent[0]);
                        const int L = (int)(w & 0xffu), sq = (int)((w >> 8) & 0xffu), sv = (int)(w >> 16);
                        const int c = k < sv ? k : k + 1;            // the k-th cell other than the serving one
                        const float xr = ent[1 + 2 * c], xi = ent[2 + 2 * c];
                        const float gc =
                            pm.fading ? 10.0f * log10_pos(clamp_min(xr * xr + xi * xi, 1e-6f)) : 0.0f;
                        s_t[(c * S + sq) * STEP_WAVE + L] = from_db(s_psd[c * STEP_WAVE + L] + gc);
                    }
                } else {                                // several envs per wavefront: each lane its own terms
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        const float psd = ((pgc[c] + pm.ue_tx) - cl.ref_db) - sp;
#pragma unroll
                        for (int s = 0; s < S; ++s) {
                            float v = 0.f;
                            if (txing && c != serv && ((won >> s) & 1u)) v = from_db(psd + gain_cs(c * S + s));
                            s_t[(c * S + s) * STEP_WAVE + lane] = v;
                        }
                    }
                }
                __syncthreads();
                if (e < E) {
                    const int sb = lane & ~(rb - 1);
                    for (int q = r; q < NCS; q += rb) {
                        const float* col = s_t + q * STEP_WAVE + sb;
                        const float itf = aten_outer_sum(R, q < 32 * (NCS / 32), [&](int i) { return col[i]; });
                        s_if[q] = itf;
                        const float now = cl.noise_mw + itf;
                        s_ni[q] = cl.li_b == 0.0f ? now : cl.li_a * now + cl.li_b * s_ni[q];
                    }
                }
                __syncthreads();
                if (r == 0 && e < E) ion = ion + aten_row_sum(NCS, [&](int i) { return s_if[i] / cl.noise_mw; });
            }
        }
        INET_PH(6);                                // binding, actual gains (CSI), interference
        // ---- decoding on the actual channel (mac.py:428-454, mac_ul.py:185-192) ----
        bool ok = false, fail = false, exh = false;
        float comb = comb_p, lexp = lexp_p, nrb = nrb_p;
        bool any_tx;                                   // (W = 2: both waves enter, the EESM has barriers)
        if constexpr (W == 1) any_tx = __ballot(tx) != 0ull;
        else any_tx = env_any(tx);
        if (any_tx) {
            const float beta = s_beta[mcs], rbeta = s_rbeta[mcs];
            bool nan = false;
            float xs[S];
#pragma unroll
            for (int s = 0; s < S; ++s) {
                float x;                          // UL: ref - split + gain (mac_ul.py:185-192); DL: ref + gain
                if constexpr (DL) x = REF(s) + gn[s];
                else x = (REF(s) - sp) + csi[s];
                if constexpr (MC)                 // minus the measured N+I over the estimate (nr_engine.py:815)
                    if (cl.use_int) x = x - ((10.0f * log10f(cl.noise_mw + s_if[serv * S + s])) - ni_la[s]);
                nan |= x != x;
                xs[s] = x;
                if (!pm.eesm) s_x[s * CW + lane] = x;                    // (the mean-dB row)
            }
            // the EESM log-sum of the held RBGs (lse_eesm of the linear SINR per RBG)
            const float lse_tx = (IR || pm.eesm) ? held_lse(tx, xs, mcs, nan) : 0.0f;
            float eff_used;
            int m_look = mcs;
            if constexpr (IR) {
                float lse = lse_tx;
                // torch.logaddexp: equal infinities stay, else max + log1p(exp(-|a - b|))
                if (isinf(lexp_p) && lexp_p == lse) lexp = lexp_p;
                else { float mx = lexp_p > lse ? lexp_p : lse; lexp = mx + log1pf(expf(-fabsf(lexp_p - lse))); }
                nrb = nrb_p + n_prb;
                float v = (-beta) * (lexp - logf(clamp_min(nrb, 1.0f)));
                eff_used = nan_to_num(10.0f * log10_clamped(clamp_min(v, 1e-6f)), -30.0f, 60.0f, -30.0f);
                int nt = ntx < tb.EQW - 1 ? ntx : tb.EQW - 1;
                m_look = s_eq[mcs * tb.EQW + nt];
                comb = comb_p;
            } else {
                float eff;
                if (pm.eesm) {
                    eff = db_of((-beta) * (lse_tx - lnw));
                } else {
                    eff = mean_db_held<S, CW>(s_x, lane, s_logw, won, lnw);
                }
                float lin_e = from_db(eff);
                comb = pm.comb == 1 ? comb_p + lin_e : lin_e;
                eff_used = 10.0f * log10_clamped(clamp_min(comb, 1e-9f));
            }
            float cbs, ncb;
            segment_f(tbs, s_rate[mcs], cbs, ncb);
            float xc = clampf(div_const(cbs - tb.c0, tb.dc, rdc), 0.0f, (float)(tb.C - 1));
            float i0f = clamp_max(floorf(xc), (float)(tb.C - 2));
            float wi = xc - i0f;
            float b = bler_at(tb.bler, (m_look * tb.C + (int)i0f) * tb.G, tb.G, tb.s0, tb.ds, rds, eff_used, wi);
            float p_err = 1.0f - pow_count(1.0f - b, ncb);
            float u = uniform_bits(elem_hash(mix32(base0 ^ row.salt_bler), (uint32_t)r));
            ok = tx && u >= p_err;
            fail = tx && !ok;
            exh = fail && ntx >= pm.max_tx;
        }
        INET_PH(7);                                // decoding
        // ---- HARQ state update (mac.py:456-477; UL timing mac_ul.py:218-219, DL mac_dl.py:47-49: decoded TBs wait
        // for their HARQ-ACK at the row's ACK slot, and both outcomes are known gnb_proc slots after it) ----
        int rdy_ok = g, rdy_fail = g + pm.ul_rtt, st_ok = 0;
        if constexpr (DL) {
            rdy_ok = g0 + ((row.flags >> 8) & 0xffff) + lk.gnb_proc;
            rdy_fail = rdy_ok;
            st_ok = 2;
        }
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (p == p_tx && tx) {
                int stp = hm_state(hmeta[p]);
                int ntxp = ntx;
                if (ok) { stp = st_ok; hrdy[p] = rdy_ok; }
                hcomb[p] = comb;
                if constexpr (IR) { hlexp[p] = lexp; hnrb[p] = nrb; }
                if (fail) hrdy[p] = rdy_fail;
                if (exh) {
                    if (pm.harq_drop) stp = 0;
                    else {
                        ntxp = 0; hcomb[p] = 0.f;
                        if constexpr (IR) { hlexp[p] = -INFINITY; hnrb[p] = 0.f; }
                        hrdy[p] = g + pm.rlc_retx;
                    }
                }
                hmeta[p] = hm_pack(stp, ntxp, hm_mcs(hmeta[p]), hm_nsb(hmeta[p]));
            }
        }
        // ---- OLLA, BSR, PF average, RR (mac.py:479-485, mac_ul.py:229-236, mac.py:534-554) ----
        if (pm.olla) olla = clampf((olla + pm.olla_up * (ok ? 1.0f : 0.0f)) - pm.olla_dn * (fail ? 1.0f : 0.0f),
                                   -10.0f, 10.0f);
        const int served = ok ? hi_tx - lo_tx : 0;
        if (!DL && tx) bsr = enq - sent;
        if (!DL && pm.amc_prev && tx) lnp = n_prb;        // UlMac.last_nprb (mac.py:484)
        {
            // PF average (mac.py:534-554): EWMA of the served bytes; pf_update "rbg": of the granted bytes of a new TB;
            // pf_avg_idle "freeze": only robots with new data to schedule in this slot move it
            const float upd = pm.pf_rbg ? (float)(tx_new ? tbs_new / 8 : 0) : (float)served;
            const float na = clamp_min(pm.pf_a * avg + pm.pf_b * upd, 1e-9f);
            avg = (pm.pf_freeze && !(need > 0 && !has_rx)) ? avg : na;
        }
        if (pm.sched == 2 && tx) last_tx = g;
        // ---- counters ----
        c_new += tx_new; c_retx += tx_rx; c_ok += ok; c_fail += fail; c_exh += exh;
        c_bytes_ok += served; c_bytes_new += tx_new ? byt_new : 0; c_new_pend += (tx_new && pending);
        c_prb += tx ? (int)n_prb : 0;
        if (lena) { c_tbb += tx_new ? tbs_new / 8 : 0; c_tbe += (tx_new && byt_new == 0) ? 1 : 0; }
        if (tx) {
            int kh = ntx < pm.max_tx ? ntx : pm.max_tx;
            atomicAdd(&my_hist[HB + kh], 1);
            atomicAdd(&my_hist[(ok ? 0 : 2 * HB) + kh], 1);
        }
        // ---- RLC in-order pointer of this slot ----
        if constexpr (DL) {
            // the DL link resolves its frames as the pointer moves (no per-slot history in LDS): under RLC UM the
            // frames an exhausted TB overlaps are lost (mac.py:474-477), then the frames the in-order pointer has
            // passed complete at this slot (mac.py:500-503). Frames before nf are lost or completed, and no
            // completed frame overlaps an undecoded TB, so both scans start at nf.
            if (act) {
                if (pm.harq_drop && exh) {
                    for (int f = nf; f < qlen; ++f) {
                        const int fr = f * R;
                        if (ldo(lk.q_start + fr, o_fr0) >= hi_tx) break;
                        if (ldo(lk.q_end + fr, o_fr0) > lo_tx) {
                            const uint32_t m = ldo(lk.q_meta + fr, o_fr0);
                            if (!(m & 1u)) { sto(lk.q_meta + fr, o_fr0, m | 1u); ++lost_dl; }
                        }
                    }
                }
                const int a = ack_ptr();
                for (; nf < qlen; ++nf) {
                    const int fr = nf * R;
                    const uint32_t m = ldo(lk.q_meta + fr, o_fr0);
                    if ((m & 1u) || ldo(lk.q_fin + fr, o_fr0) != FIN_NONE) continue;   // lost, or completed before
                    if (ldo(lk.q_end + fr, o_fr0) > a) break;
                    sto(lk.q_fin + fr, o_fr0, g);
                }
            }
        } else if (n_ul < n_ul_max) {            // (UL: recorded, completion replayed in the epilogue)
            ack_l[n_ul * CW + lane] = ack_ptr();
            if (pm.harq_drop) {
                exlo_l[n_ul * CW + lane] = exh ? lo_tx : 0;
                exhi_l[n_ul * CW + lane] = exh ? hi_tx : 0;
            }
        }
        ++n_ul;
        INET_PH(8);                                // HARQ / OLLA / PF update, counters, in-order pointer
    }
    const int n_hist = DL ? 0 : (n_ul < n_ul_max ? n_ul : n_ul_max);

    // ================================================================ end of step (NRNet._finish)
    if constexpr (MC) {                            // A3 triggers after the step's last active slot (nr_engine.py:780)
        const bool late = cl.rlf ? rlf_events(g0 + N - 1) : (act && !fired && k_ho >= 0);
        if (late) handover(g0 + k_ho);
        // the reported SINR (serving_sinr_db, nr_engine.py:709-713): full power over snr_ref_prbs PRBs against the
        // serving gNB's wideband N+I estimate, ((pg + ue_tx) - ref_db) - 10 log10(mean_s ni)
        float nrow[S];
#pragma unroll
        for (int s = 0; s < S; ++s) nrow[s] = s_ni[serv * S + s];
        snr_out = ((sel_of(pgc, serv) + pm.ue_tx) - cl.ref_db) - 10.0f * log10f(aten_sum<S>(nrow) / (float)S);
    }
    const int t = (int)T;
    const int ack_end = ack_ptr();
    const int ep0 = act ? st.epoch[ee] : 0;
    int newest = -1, kept = 0, lost_new = 0;
    bool det_hit = false;
    int new_floor = enq;
    const int64_t hid_cur = (act && cur_hid) ? cur_hid[ee] : 0;
    const double po = (double)pm.proc_off_hi + (double)pm.proc_off_lo;
    const uint32_t ob = (uint32_t)(ee * R + rr0) * (uint32_t)F;   // output row of this robot [E][R][F], elements
    uint32_t o_fr = o_fr0;
    asm volatile("" : "+v"(o_fr));
    const int qv = act ? qlen : 0;                     // queued frames of this robot (a prefix of the FIFO)
    for (int f = 0; f < qv; ++f) {
        const int fr = f * R;
        const int cap = ldo(lk.q_cap + fr, o_fr), qs = ldo(lk.q_start + fr, o_fr), qe = ldo(lk.q_end + fr, o_fr);
        int fin = ldo(lk.q_fin + fr, o_fr);
        const uint32_t meta = ldo(lk.q_meta + fr, o_fr);
        bool lost = meta & 1u;
        // the losses of handovers and radio link failures, each at its place among the slots: frames not completed and
        // not lost by then
        auto drop_at = [&](int j, bool after) {
            if constexpr (MC) {
#pragma unroll
                for (int i = 0; i < ND; ++i) {
                    const bool at = after ? drop_j[i] >= n_hist : drop_j[i] == j;
                    if (i < n_drop && at && ((drop_m[i] >> (f & 63)) & 1ull) != 0ull && fin == FIN_NONE) {
                        if (!lost) ++lost_new;
                        lost = true;
                    }
                }
            }
        };
        // replay the slots: lost marking (handover, RLC UM) first, then in-order completion (mac.py:474-477, 500-503)
        for (int j = 0; j < n_hist; ++j) {
            drop_at(j, false);
            if (pm.harq_drop) {
                int xl = exlo_l[j * CW + lane], xh = exhi_l[j * CW + lane];
                if (xh > xl && qs < xh && qe > xl) {
                    if (!lost) ++lost_new;
                    lost = true;
                }
            }
            if (fin == FIN_NONE && !lost && qe <= ack_l[j * CW + lane]) fin = g0 + s_ulrel[j];
        }
        drop_at(0, true);
        double fin_d = INFINITY;
        if (fin != FIN_NONE) {
            int tf = fin / N, rel = fin - tf * N;
            fin_d = ((double)tf + (double)(rel + 1) / (double)N) + po;
        }
        const bool delivered = fin_d <= ((double)t + 1.0) + 1e-9;
        const bool timed = pm.purge && fin == FIN_NONE && (t + 1 - cap) >= pm.timeout;
        const bool dropped = lost && qe <= ack_end && !timed;
        float delay = NAN;
        if (delivered) {
            delay = (float)(fin_d - (double)cap);
            newest = cap > newest ? cap : newest;
            if constexpr (!DL)
                if ((meta & 2u) && ldo(st.q_hid + fr, o_fr) == (int32_t)hid_cur) det_hit = true;
        }
        const int cap_rel = cap >= 0 ? cap - ep0 : -1;
        const int cls = (int)((meta >> 8) & 0xffu);
        if constexpr (DL) {
            // the DL's step outputs hold no per-frame keys (nr_engine.py:866-881); its delays go out only when the
            // caller keeps statistics
            if (lk.out_delay) sto(lk.out_delay + f, ob * 4u, delay);
        } else if (pm.out_ref) {
            sto(out.delivered + f, ob, (uint8_t)delivered);
            sto(out.timed_out + f, ob, (uint8_t)timed);
            sto(out.dropped + f, ob, (uint8_t)dropped);
            sto(out.cap + f, ob * 8u, (int64_t)cap_rel);
            sto(out.cls + f, ob * 8u, (int64_t)cls);
        } else {
            sto(out.delivered + f, ob, (uint8_t)(delivered | (timed << 1) | (dropped << 2)));
            sto(out.cap32 + f, ob * 4u, (int32_t)cap_rel);
            sto(out.cls8 + f, ob, (uint8_t)cls);
        }
        if constexpr (!DL) sto(out.delay + f, ob * 4u, delay);
        // compaction: the frames that stay move to the front, in order (queues.py:105-110)
        if (!(delivered || timed || dropped)) {
            if (kept == 0) new_floor = qs;
            if (kept != f) {
                const int kr = kept * R;
                sto(lk.q_cap + kr, o_fr, cap); sto(lk.q_start + kr, o_fr, qs); sto(lk.q_end + kr, o_fr, qe);
                sto(lk.q_meta + kr, o_fr, (meta & ~1u) | (lost ? 1u : 0u));
                if constexpr (!DL) sto(st.q_hid + kr, o_fr, ldo(st.q_hid + fr, o_fr));
                sto(lk.q_fin + kr, o_fr, fin);
            } else {
                sto(lk.q_meta + fr, o_fr, (meta & ~1u) | (lost ? 1u : 0u));
                sto(lk.q_fin + fr, o_fr, fin);
            }
            ++kept;
        }
    }
    INET_PH(9);                                        // epilogue: frame replay, outputs, compaction
    if constexpr (DL) lost_new += lost_dl;             // marked in the slot loop
    // the slots past the queue get the outputs of an empty slot (not delivered / timed out / dropped, cap -1,
    // class 0, delay NaN): one frame at a time up to a multiple of 4, then 16-byte stores of 4 frames per array
    if (!DL && act) {
        const bool vec = (F & 3) == 0;
        const int fa = vec ? ((qv + 3) & ~3) : F;
        const uint32_t qnan = 0x7fc00000u;
        for (int f = qv; f < fa; ++f) {
            if (pm.out_ref) {
                sto(out.delivered + f, ob, (uint8_t)0); sto(out.timed_out + f, ob, (uint8_t)0);
                sto(out.dropped + f, ob, (uint8_t)0);
                sto(out.cap + f, ob * 8u, (int64_t)-1); sto(out.cls + f, ob * 8u, (int64_t)0);
            } else {
                sto(out.delivered + f, ob, (uint8_t)0); sto(out.cap32 + f, ob * 4u, (int32_t)-1);
                sto(out.cls8 + f, ob, (uint8_t)0);
            }
            sto(out.delay + f, ob * 4u, __uint_as_float(qnan));
        }
        const uint4 ones = make_uint4(~0u, ~0u, ~0u, ~0u), zeros = make_uint4(0u, 0u, 0u, 0u);
        const uint4 nans = make_uint4(qnan, qnan, qnan, qnan);
        for (int f = fa; f < F; f += 4) {
            if (pm.out_ref) {
                sto((uint32_t*)(out.delivered + f), ob, 0u);
                sto((uint32_t*)(out.timed_out + f), ob, 0u);
                sto((uint32_t*)(out.dropped + f), ob, 0u);
                sto((uint4*)(out.cap + f), ob * 8u, ones); sto((uint4*)(out.cap + f + 2), ob * 8u, ones);
                sto((uint4*)(out.cls + f), ob * 8u, zeros); sto((uint4*)(out.cls + f + 2), ob * 8u, zeros);
            } else {
                sto((uint32_t*)(out.delivered + f), ob, 0u);
                sto((uint4*)(out.cap32 + f), ob * 4u, ones);
                sto((uint32_t*)(out.cls8 + f), ob, 0u);
            }
            sto((uint4*)(out.delay + f), ob * 4u, nans);
        }
    }
    if constexpr (DL) {
        if (act && lk.out_delay)
            for (int f = qv; f < F; ++f) sto(lk.out_delay + f, ob * 4u, __uint_as_float(0x7fc00000u));
    }
    if (act) {                                         // vacated slots: empty, not completed
        for (int f = kept; f < qlen; ++f) { sto(lk.q_cap + f * R, o_fr, -1); sto(lk.q_fin + f * R, o_fr, (int)FIN_NONE); }
    }
    // compact(): floor, sent, dead processes, BSR (mac.py:610-616, mac_ul.py:255-257)
    floor_ = new_floor;
    sent = sent > floor_ ? sent : floor_;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        if (hm_state(hmeta[p]) == 1 && hhi[p] <= floor_ && hhi[p] > hlo[p]) {
            hmeta[p] = hm_pack(0, 0, hm_mcs(hmeta[p]), hm_nsb(hmeta[p]));
            hrdy[p] = 0; hcomb[p] = 0.f;
            if constexpr (IR) { hlexp[p] = -INFINITY; hnrb[p] = 0.f; }
        }
    }
    if constexpr (!DL) {
        int un = enq - sent;
        bsr = bsr < un ? bsr : un;
    }
    INET_PH(10);                                       // empty-slot outputs
    const int ack_new = ack_ptr();
    const int qb_end = enq - ack_new;                  // (queue_bytes: a difference of offsets)
    // The byte offsets stay in int32: once the floor reaches rebase_at, every offset of the robot moves down by the
    // floor and the robot's 64-bit base takes it (the reference's int64 offsets are base + offset). The queued frames
    // and the live HARQ processes lie at or within a TB of the floor; a free process's stale range is never read
    // again and is kept at most 2^30 below the floor.
    bool rebased = false;
    if (lk.base != nullptr && pm.rebase_at > 0 && act && floor_ >= pm.rebase_at) {
        const int b = floor_;
        rebased = true;
        sent -= b; enq -= b; floor_ = 0;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int64_t lo = (int64_t)hlo[p] - b, hi = (int64_t)hhi[p] - b;
            hlo[p] = (int)(lo < -(1ll << 30) ? -(1ll << 30) : lo);
            hhi[p] = (int)(hi < -(1ll << 30) ? -(1ll << 30) : hi);
        }
        for (int f = 0; f < kept; ++f) {
            const int fr = f * R;
            sto(lk.q_start + fr, o_fr, ldo(lk.q_start + fr, o_fr) - b);
            sto(lk.q_end + fr, o_fr, ldo(lk.q_end + fr, o_fr) - b);
        }
        sto(lk.base, o_r0 * 2u, ldo(lk.base, o_r0 * 2u) + (int64_t)b);
    }
    // ---------------- store state and per-robot outputs ----------------
    {
        // fresh copies of the per-lane offsets: the store addresses are recomputed here instead of being kept live
        // from the loads at the top of the kernel
        uint32_t o_r = o_r0, o_sr = o_sr0, o_pr = o_pr0;
        asm volatile("" : "+v"(o_r), "+v"(o_sr), "+v"(o_pr));
    if (act) {
        sto(lk.sent, o_r, sent); sto(lk.floor_, o_r, floor_);
        if constexpr (!DL) {
            sto(st.bsr, o_r, bsr); sto(st.sr_t, o_r, sr_t);
            if (pm.amc_prev) sto(st.last_nprb, o_r, lnp);
            if (kl) {
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const uint32_t oc = (uint32_t)((ee * NC + c) * R + rr0) * 4u;
                    sto(st.k_lin, oc, kk[c]); sto(st.k_from, oc, kf[c]); sto(st.k_g0, oc, kg[c]);
                }
            }
            if (fc2)
#pragma unroll
                for (int c = 0; c < NC; ++c) sto(st.fc_idx, o_rc(c), fci[c]);
        }
        sto(lk.last_tx, o_r, last_tx); sto(lk.qlen, o_r, kept); sto(lk.olla, o_r, olla); sto(lk.avg, o_r, avg);
        if (arr.counts || rebased) sto(lk.enq, o_r, enq);
#pragma unroll
        for (int s = 0; s < S; ++s) sto(lk.csi + s * R, o_sr, csi[s]);
        if constexpr (!DL) {
            if (pm.fading) {
                uint32_t o_hr = o_hr0;
                asm volatile("" : "+v"(o_hr));
#pragma unroll
                for (int q = 0; q < NCS; ++q) { sto(st.h_re + q * R, o_hr, hr[q]); sto(st.h_im + q * R, o_hr, hi[q]); }
            }
        }
        if constexpr (MC) {
            sto(cl.serv, o_r, serv); sto(cl.a3_cand, o_r, a3_cand); sto(cl.a3_cnt, o_r, a3_cnt);
            sto(cl.ho_end, o_r, ho_end); sto(cl.n_ho, o_r, n_ho);
            if (cl.rlf) {
                sto(cl.rlf_active, o_r, rlf_on ? 1 : 0); sto(cl.oos_cnt, o_r, oos_cnt); sto(cl.is_cnt, o_r, is_cnt);
                sto(cl.t310_end, o_r, t310_end); sto(cl.t311_end, o_r, t311_end); sto(cl.reest_end, o_r, reest_end);
                sto(cl.reest_cell, o_r, reest_cell); sto(cl.n_rlf, o_r, n_rlf);
                sto(cl.out_rlf, o_r >> 2, (uint8_t)(rlf_on ? 1 : 0));
            }
        }
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int pr = p * R;
            sto(lk.h_meta + pr, o_pr, hmeta[p]); sto(lk.h_lo + pr, o_pr, hlo[p]); sto(lk.h_hi + pr, o_pr, hhi[p]);
            sto(lk.h_ready + pr, o_pr, hrdy[p]); sto(lk.h_tbs + pr, o_pr, htbs[p]); sto(lk.h_comb + pr, o_pr, hcomb[p]);
            if constexpr (IR) { sto(lk.h_lexp + pr, o_pr, hlexp[p]); sto(lk.h_nrb + pr, o_pr, hnrb[p]); }
        }
        if constexpr (DL) {
            // NRNet.dl_newest (absolute) and the step outputs dl_newest (env clock) and dl_queue_len
            sto(lk.newest, o_r, newest);
            sto(lk.out_newest, o_r * 2u, (int64_t)(newest >= 0 ? newest - ep0 : -1));
            sto(lk.out_queue_len, o_r * 2u, (int64_t)kept);
        } else {
            sto(out.newest, o_r * 2u, (int64_t)(newest >= 0 ? newest - ep0 : -1));
            sto(out.queue_len, o_r * 2u, (int64_t)kept);
            sto(out.queue_bytes, o_r, (float)(qb_end > 0 ? qb_end : 0));
            sto(out.sinr_db, o_r, snr_out);
            if (out.serving_cell) sto(out.serving_cell, o_r * 2u, (int64_t)serv);
        }
    }
    }
    // per-env outputs and counters (segment reductions, written by robot 0)
    const bool det_any = env_any(det_hit);
    const int v_new = env_sum(act ? c_new : 0), v_retx = env_sum(act ? c_retx : 0);
    const int v_ok = env_sum(act ? c_ok : 0), v_fail = env_sum(act ? c_fail : 0);
    const int v_exh = env_sum(act ? c_exh : 0), v_lost = env_sum(act ? lost_new : 0);
    const int v_pend = env_sum(act ? c_new_pend : 0), v_bok = env_sum(act ? c_bytes_ok : 0);
    const int v_bnew = env_sum(act ? c_bytes_new : 0), v_prb = env_sum(act ? c_prb : 0);
    int v_tbb = 0, v_tbe = 0, v_blk = 0;
    if (lena) { v_tbb = env_sum(act ? c_tbb : 0); v_tbe = env_sum(act ? c_tbe : 0); v_blk = env_sum(act ? c_blk : 0); }
    __syncthreads();                                  // histogram atomics of every lane are done
    if constexpr (MC) {
        int v_rl[5] = {0, 0, 0, 0, 0};
        if (cl.rlf) {
#pragma unroll
            for (int k = 0; k < 5; ++k) v_rl[k] = env_sum(act ? c_rl[k] : 0);
        }
        if (e < E) {
            for (int q = r; q < NCS; q += rb) cl.ni_ul[(size_t)e * NCS + q] = s_ni[q];
            if (r == 0) { cl.pending[e] = 0; cl.ion[e] = ion; }
            if (cl.rlf && r == 0) {
#pragma unroll
                for (int k = 0; k < 5; ++k) cl.rlf_ctr[(size_t)e * 5 + k] += v_rl[k];
            }
        }
    }
    if (r == 0 && e < E) {
        if constexpr (!DL) {
            out.det_env[e] = det_any;
            out.t[e] = (int64_t)t - (int64_t)st.epoch[e];
            st.ctr_step[e] = st.ctr_step[e] + 1;      // rng.tick_step (nr_engine.py:847-848)
            if (kl && los_rep) st.k_fresh[e] = 0;      // the env's LOS state has arrived
        }
        int64_t* c = lk.ctr + (size_t)e * INET_NR_NCTR;
        c[0] += v_new; c[1] += v_retx; c[2] += v_ok; c[3] += v_fail; c[4] += v_exh;
        c[5] += v_bok; c[6] += v_bnew; c[7] += v_lost; c[8] += v_pend; c[9] += v_prb;
        c[10] += v_tbb; c[11] += v_tbe; c[12] += v_blk;
    }
    if (e < E && r < 3 * HB) lk.hist[(size_t)e * 3 * HB + r] += my_hist[r];
    if (e < E && rb < 3 * HB) {                       // segments narrower than the histogram: robot 0 adds the rest
        if (r == 0)
            for (int q = rb; q < 3 * HB; ++q) lk.hist[(size_t)e * 3 * HB + q] += my_hist[q];
    }
    INET_PH(11);                                      // state stores, per-env reductions and counters
    INET_PH_STORE;
}

// ---------------------------------------------------------------- launch plumbing
struct StepArgs {
    InetNrState st;
    const InetNrDlState* dl;          // NULL: the UL step; else the DL step of this link
    const InetNrCells* cells;         // NULL: one cell; else the multi-cell step (NRNet.step_cells)
    InetNrTables tb;
    InetNrParams pm;
    const InetNrRow* rows;
    int n_rows, n_data;
    InetNrArrivals arr;               // counts == NULL: no arrivals in the launch
    int64_t T;
    const float* x;
    const int64_t* hid;
    InetNrOutputs out;
    int rb;
    unsigned grid;
    size_t lds;
    hipStream_t stream;
};
typedef void (*StepFn)(const StepArgs&);

template <int S, int P, bool IR, bool VREF, int RBT, int FX = 0>
void launch_step(const StepArgs& a) {
    const InetNrCells none{};
    if (a.dl)
        hipLaunchKernelGGL((nr_step_kernel<S, P, IR, VREF, RBT, InetNrDlState, 1, FX>), dim3(a.grid),
                           dim3(STEP_WAVE), a.lds, a.stream, a.st, *a.dl, a.tb, a.pm, a.rows, a.n_rows, a.T, a.x,
                           a.hid, a.out, a.rb, a.n_data, a.arr, none);
    else
        hipLaunchKernelGGL((nr_step_kernel<S, P, IR, VREF, RBT, InetNrState, 1, FX>), dim3(a.grid), dim3(STEP_WAVE),
                           a.lds, a.stream, a.st, a.st, a.tb, a.pm, a.rows, a.n_rows, a.T, a.x, a.hid, a.out, a.rb,
                           a.n_data, a.arr, none);
}

// the build that fixes these parameters at compile time: 1 (with the Rician phasor) or 2 (without), 0 for none
inline int fx_profile(const InetNrParams& p) {
    const bool common = p.pf_rbg == 0 && p.pf_freeze == 0 && p.whole_band == 0 && p.pc1_on == 0 &&
                        p.retx_tdma == 0 && p.amc_prev == 0 && p.fc_on == 0 && p.los_sto == 0 && p.k_from_los == 0 &&
                        p.doppler == 0 && p.pf_wb == 0 &&
                        p.sched == 0 && p.comb == 1 && p.eesm == 1 && p.harq_drop == 0 && p.olla == 1 &&
                        p.phr_cap == 1 && p.retx_prio == 1 && p.fading == 1;
    return common ? (p.rician == 1 ? 1 : (p.rician == 0 ? 2 : 0)) : 0;
}

// envs of 65..128 (RBT = 128) or 129..256 robots (RBT = 256): one env per workgroup of two or four wavefronts (pose
// or SNR input; the UL, and with RBT = 128 the DL too)
template <int S, int P, bool IR, int FX = 0, int RBT = 128>
void launch_step_w2(const StepArgs& a) {
    const InetNrCells none{};
    if constexpr (RBT == 128)
        if (a.dl) {
            hipLaunchKernelGGL((nr_step_kernel<S, P, IR, false, RBT, InetNrDlState, 1, FX>), dim3(a.grid), dim3(RBT),
                               a.lds, a.stream, a.st, *a.dl, a.tb, a.pm, a.rows, a.n_rows, a.T, a.x, a.hid, a.out,
                               a.rb, a.n_data, a.arr, none);
            return;
        }
    hipLaunchKernelGGL((nr_step_kernel<S, P, IR, false, RBT, InetNrState, 1, FX>), dim3(a.grid), dim3(RBT), a.lds,
                       a.stream, a.st, a.st, a.tb, a.pm, a.rows, a.n_rows, a.T, a.x, a.hid, a.out, a.rb, a.n_data,
                       a.arr, none);
}

// the multi-cell step: NC cells, pose input, runtime segment width (RBT = 0) or one fixed at compile time
template <int S, int P, bool IR, int NC, int FX = 0, int RBT = 0>
void launch_step_mc(const StepArgs& a) {
    hipLaunchKernelGGL((nr_step_kernel<S, P, IR, false, RBT, InetNrState, NC, FX>), dim3(a.grid), dim3(STEP_WAVE), a.lds,
                       a.stream, a.st, a.st, a.tb, a.pm, a.rows, a.n_rows, a.T, a.x, a.hid, a.out, a.rb, a.n_data,
                       a.arr, *a.cells);
}

// every (P, IR, per-subband SNR) with a runtime segment width; plus, for 32-robot envs without IR or per-subband
// input, a build with the width fixed at compile time
template <int S>
StepFn pick_step_s(int P, bool ir, bool vref, int rb, int fx) {
    if constexpr (S == 13)                           // the common configuration at 13 RBGs, 8 HARQ, 32-robot envs
        if (fx == 1 && P == 8 && !ir && !vref && rb == 32) return &launch_step<13, 8, false, false, 32, 1>;
#define INET_PICK(PP)                                                                                 \
    if (P == PP) {                                                                                    \
        if (!ir && !vref && rb == 32) return &launch_step<S, PP, false, false, 32>;                  \
        return ir ? (vref ? &launch_step<S, PP, true, true, 0> : &launch_step<S, PP, true, false, 0>) \
                  : (vref ? &launch_step<S, PP, false, true, 0> : &launch_step<S, PP, false, false, 0>); \
    }
    INET_PICK(2) INET_PICK(4) INET_PICK(8) INET_PICK(16)
#undef INET_PICK
    return nullptr;
}

StepFn pick_step_s13(int P, bool ir, bool vref, int rb, int fx);   // nr_step_s13.hip
StepFn pick_step_s8(int P, bool ir, bool vref, int rb, int fx);    // nr_step_s8.hip
// the other RBG counts of one cell, each with its two-wavefront builds (nr_step_s<S>.hip): the counts of the standard
// carriers at 30 kHz (RBG configuration 1: 24, 38/78, 106/217, 133/65, 162, 245, 273 PRB)
#define INET_STEP_S_EXTRA(X) X(10) X(11) X(12) X(14) X(16) X(17) X(18)
#define INET_DECL_S(SS)                                                    \
    StepFn pick_step_s##SS(int P, bool ir, bool vref, int rb, int fx);   \
    StepFn pick_step_w2_s##SS(int P, bool ir, int fx);                   \
    StepFn pick_step_w4_s##SS(int P, bool ir);
INET_STEP_S_EXTRA(INET_DECL_S)
#undef INET_DECL_S


// multi-cell builds (NC cells): every (P, IR)
template <int S, int NC>
StepFn pick_step_mc_s(int P, bool ir, int fx, int rb) {
    if constexpr (S == 14 && NC == 3)                // config 3's switches (no Rician phasor), 8 HARQ, 64-robot envs
        if (fx == 2 && P == 8 && !ir && rb == 64) return &launch_step_mc<14, 8, false, 3, 2, 64>;
// (no HARQ-IR builds with several cells: refused, INET_NR_EUNSUPPORTED)
#define INET_PICK_MC(PP) \
    if (P == PP) return ir ? nullptr : &launch_step_mc<S, PP, false, NC>;
    INET_PICK_MC(2) INET_PICK_MC(4) INET_PICK_MC(8) INET_PICK_MC(16)
#undef INET_PICK_MC
    return nullptr;
}
StepFn pick_step_mc(int S, int C, int P, bool ir, int fx, int rb); // nr_step_mc.hip
StepFn pick_step_mc2(int S, int P, bool ir, int fx, int rb);       // nr_step_mc2.hip
StepFn pick_step_mc4(int S, int P, bool ir, int fx, int rb);       // nr_step_mc4.hip
StepFn pick_step_mc5(int S, int P, bool ir, int fx, int rb);       // nr_step_mc5.hip
StepFn pick_step_mc6(int S, int P, bool ir, int fx, int rb);       // nr_step_mc6.hip
StepFn pick_step_mc7(int S, int P, bool ir, int fx, int rb);       // nr_step_mc7.hip

// two-wavefront builds (R = 65..128): every (P, IR)
template <int S>
StepFn pick_step_w2_s(int P, bool ir, int fx) {
    if constexpr (S == 8)                            // config 5's switches without the Rician phasor, 8 HARQ
        if (fx == 2 && P == 8 && !ir) return &launch_step_w2<8, 8, false, 2>;
#define INET_PICK_W2(PP) \
    if (P == PP) return ir ? &launch_step_w2<S, PP, true> : &launch_step_w2<S, PP, false>;
    INET_PICK_W2(2) INET_PICK_W2(4) INET_PICK_W2(8) INET_PICK_W2(16)
#undef INET_PICK_W2
    return nullptr;
}
StepFn pick_step_w2(int S, int P, bool ir, int fx);        // nr_step_w2.hip
// four-wavefront builds (R = 129..256): every (P, IR)
template <int S>
StepFn pick_step_w4_s(int P, bool ir) {
#define INET_PICK_W4(PP) \
    if (P == PP) return ir ? &launch_step_w2<S, PP, true, 0, 256> : &launch_step_w2<S, PP, false, 0, 256>;
    INET_PICK_W4(2) INET_PICK_W4(4) INET_PICK_W4(8) INET_PICK_W4(16)
#undef INET_PICK_W4
    return nullptr;
}
StepFn pick_step_w4(int S, int P, bool ir);                // nr_step_w4.hip

// the one-cell step builds for S subbands: envs of up to 64 robots on one wavefront (nullptr: no build)
inline StepFn pick_step_one_cell(int S, int P, bool ir, bool vref, int rb, int fx) {
    switch (S) {
    case 8: return pick_step_s8(P, ir, vref, rb, fx);
    case 13: return pick_step_s13(P, ir, vref, rb, fx);
#define INET_CASE_S(SS) \
    case SS: return pick_step_s##SS(P, ir, vref, rb, fx);
    INET_STEP_S_EXTRA(INET_CASE_S)
#undef INET_CASE_S
    default: return nullptr;
    }
}
// envs of 65..128 robots on two wavefronts
inline StepFn pick_step_two_waves(int S, int P, bool ir, int fx) {
    switch (S) {
    case 8:
    case 13: return pick_step_w2(S, P, ir, fx);
#define INET_CASE_S(SS) \
    case SS: return pick_step_w2_s##SS(P, ir, fx);
    INET_STEP_S_EXTRA(INET_CASE_S)
#undef INET_CASE_S
    default: return nullptr;
    }
}

}  // namespace inet

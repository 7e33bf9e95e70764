// Device helpers of the NR uplink engine kernels (gfx950, wave64).
//
// * counter RNG: the lowbias32 hash, keys and Box-Muller normals of isaac_net/core/proto/rng.py:42-62, 164-185
//   (uniforms are bit-exact; normals use this device's logf / cosf / sqrtf);
// * ATen-order float reductions: torch's CPU sum over a short contiguous row (8-wide vectors, tail elements first,
//   then the vector lanes in order; rows under 8 elements in four interleaved partial sums) and logsumexp
//   (max, masked to 0 when infinite, + log of the sum of exp(x - max)). Replaying the reference's summation order
//   keeps the GPU bitwise equal to the CPU path wherever no transcendental function is involved;
// * segment collectives: a 64-lane wavefront holds 64 / RB envs, one robot per lane in a power-of-two segment of
//   RB lanes; reductions across the robots of one env are butterflies inside the segment (DPP and lane swaps)
//   or ballots (SALU).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#define DEV __device__ __forceinline__

namespace inet {

constexpr uint32_t GOLD = 0x9E3779B9u;
constexpr float INV24 = 5.9604644775390625e-08f;   // 2^-24
constexpr int32_t FIN_NONE = 0x7fffffff;            // frame not completed (fin = inf)
constexpr int64_t BIG = (int64_t)1 << 62;

DEV uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x21F0AAADu;
    x ^= x >> 15;
    x *= 0x735A2D97u;
    return x ^ (x >> 15);
}
DEV uint32_t salt32(uint32_t v) { return mix32(v) + GOLD; }
DEV uint32_t elem_hash(uint32_t base, uint32_t i) { return mix32(mix32(base + i * GOLD) ^ base); }
DEV float uniform_bits(uint32_t h) { return (float)(h >> 8) * INV24; }
// natural log of a normal, finite, positive u: v_log_f32 (log2) scaled by ln 2 in two parts with the product's
// rounding error recovered by an fma, the steps logf takes for such an argument (no denormal scaling and no
// infinity or NaN fix-up is needed there)
DEV float ln_unit(float u) {
    const float l2 = __builtin_amdgcn_logf(u);
    const float p = l2 * __int_as_float(0x3f317217);
    const float e = fmaf(__int_as_float(0x3377d1cf), l2, fmaf(l2, __int_as_float(0x3f317217), -p));
    return p + e;
}
// log10 of a finite p >= 1e-6 (a normal float): v_log_f32 (log2) scaled by log10(2) in two parts with the product's
// rounding error recovered by an fma, the steps log10f takes for such an argument
DEV float log10_pos(float p) {
    const float l2 = __builtin_amdgcn_logf(p);
    const float a = l2 * __int_as_float(0x3e9a209a);
    const float e = fmaf(__int_as_float(0x3284fbcf), l2, fmaf(l2, __int_as_float(0x3e9a209a), -a));
    return a + e;
}
// correctly rounded square root of x = +-0 or a normal positive float: the hardware estimate, then the neighbour one
// ulp below or above it when the residual x - s s' shows that it is nearer (the steps sqrtf takes for such an
// argument; no denormal scaling is needed on this range, and a zero returns itself)
DEV float sqrt_pos(float x) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const float sd = __int_as_float(__float_as_int(s) - 1), su = __int_as_float(__float_as_int(s) + 1);
    float r = fmaf(-sd, s, x) <= 0.0f ? sd : s;
    r = fmaf(-su, s, x) > 0.0f ? su : r;
    return x == 0.0f ? x : r;
}
// cos x for 0 <= x < 2 pi: the steps cosf takes for a finite argument below 2^17 (this build's device library):
// x reduced by the nearest multiple j of pi / 2 in three parts, then the sine or cosine polynomial of the remainder by
// the quadrant j mod 4. Without cosf's large-argument reduction and its NaN / infinity test, which never fire here.
DEV float cos_small(float x) {
    const float jf = rintf(x * __int_as_float(0x3f22f983));
    const int j = (int)jf;
    float r = fmaf(jf, __int_as_float(0xbfc90fda), x);
    r = fmaf(jf, __int_as_float(0xb3a22168), r);
    r = fmaf(jf, __int_as_float(0xa7c234c4), r);
    const float r2 = r * r;
    float sp = fmaf(r2, __int_as_float(0xb94c1982), __int_as_float(0x3c0881c4));
    sp = fmaf(r2, sp, __int_as_float(0xbe2aaa9d));
    const float sn = fmaf(r, r2 * sp, r);
    float cp = fmaf(r2, __int_as_float(0x37d75334), __int_as_float(0xbab64f3b));
    cp = fmaf(r2, cp, __int_as_float(0x3d2aabf7));
    cp = fmaf(r2, cp, __int_as_float(0xbf000004));
    const float cs = fmaf(r2, cp, 1.0f);
    const float v = (j & 1) ? -sn : cs;
    return __uint_as_float(__float_as_uint(v) ^ (((uint32_t)j << 30) & 0x80000000u));
}
// Box-Muller, cosine branch, from the hashes of elements 2j and 2j + 1 (u1 in [2^-24, 1], so -2 ln u1 is +-0 or a
// normal float in [1.2e-7, 33.3]; 2 pi u2 in [0, 2 pi))
DEV float normal_of(uint32_t h1, uint32_t h2) {
    float u1 = (float)((h1 >> 8) + 1u) * INV24;
    float u2 = (float)(h2 >> 8) * INV24;
    return sqrt_pos(-2.0f * ln_unit(u1)) * cos_small((float)6.283185307179586 * u2);
}
// element j of a normal draw uses hash elements 2j and 2j + 1
DEV float normal_at(uint32_t base, uint32_t j) { return normal_of(elem_hash(base, 2u * j), elem_hash(base, 2u * j + 1u)); }

// x / y for many x over one y, with x in [0, 2^60] and y normal in [2^-60, 2^60]: the Newton-Raphson steps of the
// IEEE division sequence (reciprocal, one refinement, then two residual corrections of the quotient), with the
// refined reciprocal shared by every x. On such operands that sequence's scaling and special-value fix-up steps
// change nothing, so the result is the IEEE quotient.
struct DivBy {
    float y, r;
    DEV explicit DivBy(float y_) : y(y_) {
        const float r0 = __builtin_amdgcn_rcpf(y_);
        r = fmaf(fmaf(-y_, r0, 1.0f), r0, r0);
    }
    DEV float operator()(float x) const {
        const float q0 = x * r;
        const float q1 = fmaf(fmaf(-y, q0, x), r, q0);
        return fmaf(fmaf(-y, q1, x), r, q1);
    }
};
// x / y rounded to nearest for a constant y with r = RN(1 / y): q = RN(x r), then one fma correction of the residual
// (Markstein). For the constants below this equals IEEE division for every float32 x; the check runs over every
// significand in tests/test_numerics.py.
DEV float div_const(float x, float y, float r) {
    float q = x * r;
    float e = fmaf(-q, y, x);
    return fmaf(e, r, q);
}
constexpr float SQRT2_F = (float)1.4142135623730951;
constexpr float INV_SQRT2_F = (float)(1.0 / (double)SQRT2_F);
constexpr float TEN_F = 10.0f;
constexpr float INV_TEN_F = (float)(1.0 / 10.0);
// base key of (seed key, env, episode, channel, counter, stream), proto/rng.py key_torch
DEV uint32_t base_key(uint32_t s0, uint32_t env, uint32_t ep, uint32_t channel, uint32_t ctr, uint32_t stream) {
    uint32_t h = mix32(s0 ^ salt32(env));
    h = mix32(h ^ salt32(ep));
    h = mix32(h ^ salt32(channel));
    h = mix32(h ^ salt32(ctr));
    return mix32(h ^ salt32(stream));
}

// torch clamp / maximum semantics: NaN propagates
DEV float clamp_min(float x, float lo) { return x < lo ? lo : x; }
DEV float clamp_max(float x, float hi) { return x > hi ? hi : x; }
DEV float clampf(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }
DEV float nan_to_num(float x, float nan, float pinf, float ninf) {
    return x != x ? nan : (x == INFINITY ? pinf : (x == -INFINITY ? ninf : x));
}
// log10 of x >= 1e-9 (after a clamp) that may also be +inf or NaN: log10_pos, with +inf kept (NaN stays NaN), as
// log10f gives
DEV float log10_clamped(float x) {
    const float l = log10_pos(x);
    return x == INFINITY ? x : l;
}
// phy._db: 10 log10(max(x, 1e-6)) with NaN -> -30, +inf -> 60, -inf -> -30
DEV float db_of(float lin) { return nan_to_num(10.0f * log10_clamped(clamp_min(lin, 1e-6f)), -30.0f, 60.0f, -30.0f); }
// 2^(y c) for the constant c = C1 + C2 (two parts) and y with y c well inside the float exponent range: the product
// split into an integer and a fraction, v_exp_f32 of the fraction scaled by ldexp, the steps expf / exp10f take
// for such an argument (their overflow and underflow fix-ups never fire there)
template <uint32_t C1, uint32_t C2>
DEV float exp2_scaled(float y) {
    const float c1 = __int_as_float(C1);
    const float t = y * c1;
    const float e = fmaf(__int_as_float(C2), y, fmaf(y, c1, -t));
    const float r = rintf(t);
    return ldexpf(__builtin_amdgcn_exp2f((t - r) + e), (int)r);
}
// exp(x) for a finite x <= 0 inside a sum with a term 1 (the log-sum-exp after its max): below -103.97 expf returns
// 0 where these steps can leave 2^-149, which the sum absorbs
DEV float exp_nonpos(float x) { return exp2_scaled<0x3fb8aa3bu, 0x32a5705fu>(x); }
// 10 ** (x / 10) for x in [-30, 60] (a clamped SINR in dB), as from_db below
DEV float from_db_mid(float x) { return exp2_scaled<0x40549a78u, 0x33979a37u>(div_const(x, 10.0f, 0.1f)); }
// 10 ** (x / 10) as torch evaluates it: x / 10 in float32, then 10 to that power (exp10, within an ulp)
DEV float from_db(float x) { return exp10f(div_const(x, TEN_F, INV_TEN_F)); }
// x ** n for the integer-valued float n >= 0 of a code-block count (torch pow(float, float)): binary powering in
// double precision, rounded once to float (correctly rounded unless the exact power lies within ~1e-15 relative of a
// rounding boundary); other exponents take powf
DEV float pow_count(float x, float nf) {
    int n = (int)nf;
    if (!(nf >= 0.0f && nf <= 4096.0f) || (float)n != nf) return powf(x, nf);
    double r = 1.0, b = (double)x;
    while (n) {
        if (n & 1) r *= b;
        b *= b;
        n >>= 1;
    }
    return (float)r;
}

// torch CPU float sum of a contiguous row of N elements (SumKernel.cpp vectorized_inner_sum / row_sum order)
template <int N>
DEV float aten_sum(const float* x) {
    if constexpr (N >= 8) {
        constexpr int VS = N / 8, SI = VS / 4;
        float p0[8], p1[8], p2[8], p3[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) { p0[l] = 0.f; p1[l] = 0.f; p2[l] = 0.f; p3[l] = 0.f; }
#pragma unroll
        for (int i = 0; i < SI; ++i) {
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                p0[l] += x[(i * 4 + 0) * 8 + l];
                p1[l] += x[(i * 4 + 1) * 8 + l];
                p2[l] += x[(i * 4 + 2) * 8 + l];
                p3[l] += x[(i * 4 + 3) * 8 + l];
            }
        }
#pragma unroll
        for (int i = SI * 4; i < VS; ++i) {
#pragma unroll
            for (int l = 0; l < 8; ++l) p0[l] += x[i * 8 + l];
        }
#pragma unroll
        for (int l = 0; l < 8; ++l) { p0[l] += p1[l]; p0[l] += p2[l]; p0[l] += p3[l]; }
        float fin = 0.f;
#pragma unroll
        for (int k = VS * 8; k < N; ++k) fin += x[k];
#pragma unroll
        for (int l = 0; l < 8; ++l) fin += p0[l];
        return fin;
    } else {
        constexpr int SI = N / 4;
        float q0 = 0.f, q1 = 0.f, q2 = 0.f, q3 = 0.f;
#pragma unroll
        for (int i = 0; i < SI; ++i) {
            q0 += x[i * 4 + 0];
            q1 += x[i * 4 + 1];
            q2 += x[i * 4 + 2];
            q3 += x[i * 4 + 3];
        }
#pragma unroll
        for (int i = SI * 4; i < N; ++i) q0 += x[i];
        return ((q0 + q1) + q2) + q3;
    }
}

// torch CPU float sum over the robots (dim 1) of an [E][R][C][S] tensor, column q = c S + s of the n_col = C S columns
// (the outer reduction of SumKernel.cpp as this build's CPU runs it, pinned against torch in
// tests/test_known_answers.py): the columns q < 32 floor(n_col / 32) add the rows in chunks of 16, each chunk from 0,
// accumulate the chunk sums in order from 0 and add that to the sum of the rows past the last full chunk; the other
// columns add row i into accumulator i mod 4 (the rows past the last group of four into accumulator 0) and return
// ((a0 + a1) + a2) + a3. x(i): the value of row i.
template <class X>
DEV float aten_outer_sum(int n_rows, bool chunked, X x) {
    if (chunked) {
        float acc = 0.f;
        int i = 0;
        for (; i + 16 <= n_rows; i += 16) {
            float c = 0.f;
            for (int k = 0; k < 16; ++k) c += x(i + k);
            acc += c;
        }
        float tail = 0.f;
        for (; i < n_rows; ++i) tail += x(i);
        return tail + acc;
    }
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    const int g4 = n_rows >> 2;
    for (int i = 0; i < g4; ++i) { a0 += x(4 * i); a1 += x(4 * i + 1); a2 += x(4 * i + 2); a3 += x(4 * i + 3); }
    for (int i = 4 * g4; i < n_rows; ++i) a0 += x(i);
    return ((a0 + a1) + a2) + a3;
}

// torch.logsumexp over a row of N
template <int N>
DEV float aten_lse(const float* x) {
    float mx = x[0];
#pragma unroll
    for (int k = 1; k < N; ++k) mx = x[k] > mx ? x[k] : mx;
    if (mx == INFINITY || mx == -INFINITY) mx = 0.f;
    float e[N];
#pragma unroll
    for (int k = 0; k < N; ++k) e[k] = expf(x[k] - mx);
    return logf(aten_sum<N>(e)) + mx;
}

// torch CPU float sum of a contiguous row of n < 512 elements x(0..n-1), n known at run time (same order as
// aten_sum<N>: rows of 8 or more are 8-lane vectors accumulated in four interleaved partial vectors, the tail elements
// summed first, then the vector lanes in order; shorter rows use four interleaved scalar partial sums)
template <class X>
DEV float aten_row_sum(int n, X x) {
    if (n < 8) {
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
        const int si = n >> 2;
        for (int i = 0; i < si; ++i) { a0 += x(i * 4); a1 += x(i * 4 + 1); a2 += x(i * 4 + 2); a3 += x(i * 4 + 3); }
        for (int i = si * 4; i < n; ++i) a0 += x(i);
        return ((a0 + a1) + a2) + a3;
    }
    const int nv = n >> 3, ni = nv >> 2;
    float fin = 0.f;
    for (int i = nv * 8; i < n; ++i) fin += x(i);
    for (int l = 0; l < 8; ++l) {
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
        for (int i = 0; i < ni; ++i) {
            a0 += x((i * 4) * 8 + l); a1 += x((i * 4 + 1) * 8 + l);
            a2 += x((i * 4 + 2) * 8 + l); a3 += x((i * 4 + 3) * 8 + l);
        }
        for (int i = ni * 4; i < nv; ++i) a0 += x(i * 8 + l);
        fin += ((a0 + a1) + a2) + a3;
    }
    return fin;
}

// aten_row_sum for a runtime n <= NMAX whose elements are LDS reads: every read is issued before the first add (a
// loop with a runtime bound waits for each read in turn), then the same additions in the same order. Elements past n
// read as +0.0 and are added where the loops above would not add anything: x + (+0.0) == x for every partial sum here
// (each starts at +0.0, so none is -0.0), so the result has the same bits.
template <int NMAX, class X>
DEV float aten_row_sum_u(int n, X x) {
    float v[NMAX];
#pragma unroll
    for (int i = 0; i < NMAX; ++i) v[i] = i < n ? x(i) : 0.0f;
    if (n < 8) {
        const int si = n >> 2;
        float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < (NMAX < 8 ? NMAX : 8); ++i) {
            if (i < 4) a[i] += si > 0 ? v[i] : 0.0f;
            a[0] += (i >= si * 4 && i < n) ? v[i] : 0.0f;
        }
        return ((a[0] + a[1]) + a[2]) + a[3];
    }
    const int nv = n >> 3, ni = nv >> 2;
    float fin = 0.f;
#pragma unroll
    for (int i = 0; i < NMAX; ++i) fin += (i >= nv * 8 && i < n) ? v[i] : 0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
        for (int i = 0; i < NMAX / 32; ++i) {
            const bool in = i < ni;
            a0 += in ? v[(i * 4) * 8 + l] : 0.0f;
            a1 += in ? v[(i * 4 + 1) * 8 + l] : 0.0f;
            a2 += in ? v[(i * 4 + 2) * 8 + l] : 0.0f;
            a3 += in ? v[(i * 4 + 3) * 8 + l] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < NMAX / 8; ++i) a0 += (i >= ni * 4 && i < nv) ? v[i * 8 + l] : 0.0f;
        fin += ((a0 + a1) + a2) + a3;
    }
    return fin;
}

// ---------------------------------------------------------------- radio (RadioMC.rx_dbm at one cell / AP)
// Received power (dBm) of a robot at (px, py) from the cell at (gx, gy): path loss and plane-wave shadowing
// (isaac_net/core/radio.py:238-272, channels/models.py:137-167, channels/tr38901.py:162-203 with a fixed LOS state).
// PM: a parameter struct with the radio fields of InetNrParams (hh2 ... pl_exp10, ue_tx, radio_model, n_modes);
// fld_env: the cell's fields of the env [n_fields][n_modes][3] (kx, ky, phase). The transcendental functions are evaluated in
// double precision and rounded once (the field arguments k . x reach 1e4 rad).
// the plane-wave field fld [n_modes][3] (kx, ky, phase) at (px, py): amp times the ATen-order row sum of the cosines
DEV float field_at(float px, float py, const float* fld, int n_modes, float amp) {
    float cs[16];
    for (int k = 0; k < n_modes; ++k) {
        float arg = (px * fld[k * 3 + 0] + py * fld[k * 3 + 1]) + fld[k * 3 + 2];
        cs[k] = (float)cos((double)arg);
    }
    // runtime-length ATen row sum (n_modes <= 16)
    float field;
    if (n_modes >= 8) {
        field = 0.f;
        for (int k = 8; k < n_modes; ++k) field += cs[k];
        for (int l = 0; l < 8; ++l) field += cs[l];
    } else {
        float q[4] = {0.f, 0.f, 0.f, 0.f};
        const int si = n_modes / 4;
        for (int i = 0; i < si; ++i)
            for (int k = 0; k < 4; ++k) q[k] += cs[i * 4 + k];
        for (int i = si * 4; i < n_modes; ++i) q[0] += cs[i];
        field = ((q[0] + q[1]) + q[2]) + q[3];
    }
    return amp * field;
}

// The TR 38.901 stochastic LOS state (models.py:121-135, tr38901.py:228-242): the LOS-state field value z through the
// empirical CDF of a unit sum of cosines (cdf: 65536 sorted samples), u = (index of the first sample >= z + 0.5) /
// 65537 as torch.searchsorted and float32 arithmetic give it, against Pr_LOS(d_2D) of the scenario (scn 0 UMi, 1 UMa
// with h_UT <= 13 m, 2 InH); true: LOS. on = false: the fixed LOS state of the parameters.
struct StoLos {
    const float* cdf;
    int scn;
    float sig_nlos;
    bool on;
};
DEV bool los_draw(const StoLos& sl, float z, float d2) {
    int lo = 0, hi = 1 << 16;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sl.cdf[mid] < z) lo = mid + 1;
        else hi = mid;
    }
    const float u = ((float)lo + 0.5f) / 65537.0f;
    float p;
    if (sl.scn <= 1) {
        const float d = d2 > 18.0f ? d2 : 18.0f;
        const float e = expf(-d / (sl.scn == 0 ? 36.0f : 63.0f));
        p = d2 <= 18.0f ? 1.0f : 18.0f / d + e * (1.0f - 18.0f / d);
    } else {
        p = d2 <= 1.2f ? 1.0f : (d2 < 6.5f ? expf(-(d2 - 1.2f) / 4.7f) : expf(-(d2 - 6.5f) / 32.6f) * 0.32f);
    }
    return u < p;
}

// Grid index of a link's delay spread (nr_engine.py:335-340, 352-356): lgDS = mu + sigma z, then
// round((lgDS + 9 - c1) c2) (half to even) clamped to [0, G - 1], every step a float32 operation as in torch
DEV int ds_index(float mu, float sig, float z, float c1, float c2, int G) {
    const float lg = mu + sig * z;
    float r = rintf(((lg + 9.0f) - c1) * c2);
    r = r > 0.0f ? r : 0.0f;
    r = r < (float)(G - 1) ? r : (float)(G - 1);
    return (int)r;
}

template <class PM>
DEV float radio_rx_dbm(const PM& pm, float px, float py, float gx, float gy, const float* fld_env,
                       const StoLos& sto = StoLos{nullptr, 0, 0.f, false}, bool* los_out = nullptr) {
    float dx = px - gx, dy = py - gy;
    float d2 = clamp_min(sqrtf(dx * dx + dy * dy), 1.0f);
    int fi = 0;
    float pl, sig = 0.f;
    if (pm.radio_model == 1) {                 // TR 38.901 (tr38901.py:162-203)
        float d3 = sqrtf(d2 * d2 + pm.hh2);
        float lg = (float)log10((double)d3);
        float pl1 = (pm.pl_a + pm.pl_n1 * lg) + pm.pl_c20;
        float pl2 = ((pm.pl_a + 40.0f * lg) + pm.pl_c20) - pm.pl_c2;
        pl = d2 <= pm.dbp ? pl1 : pl2;
        sig = pm.sig;
        // NLOS: the fixed NLOS state, or the stochastic state's draw (the LOS-state field is field 2)
        bool nlos = pm.nl_b1 != 0.0f;
        if (sto.on) {
            nlos = !los_draw(sto, field_at(px, py, fld_env + 2 * pm.n_modes * 3, pm.n_modes, pm.amp), d2);
            if (nlos) sig = sto.sig_nlos;
        }
        if (nlos) {                            // NLOS: max(PL_LOS, PL'_NLOS)
            float pn = ((pm.nl_b1 * lg + pm.nl_b0) + pm.nl_c) - pm.nl_d;
            pl = pn > pl ? pn : pl;
            fi = 1;
        }
        if (los_out) *los_out = !nlos;         // the link's LOS state (Radio.los_state)
    } else {
        pl = pm.pl_const + pm.pl_exp10 * (float)log10((double)d2);
    }
    const float field = field_at(px, py, fld_env + fi * pm.n_modes * 3, pm.n_modes, pm.amp);
    if (pm.radio_model == 1) {
        float loss = pl + sig * field;
        return pm.ue_tx + (-loss);
    }
    return (pm.ue_tx - pl) - field;
}

// One plane wave of shadowing field fi drawn for (seed key, env, episode) (channels/fields.py:38-58,
// radio.py:185-189): element kk = c K + k (cell c, wave k) of the RESET uniforms of stream LOG_DISTANCE (10) for the
// log-distance field, TR38901 + 3 fi for the TR 38.901 fields;
// spectrum 0 "sos" (wavelengths 20..60 m scaled by dcorr / 10.3), 1 "exp" (inverse CDF of the radial spectrum).
// Writes (kx, ky, phase) to fp; cos / sin / the phase product are evaluated as the reference's float32 torch ops,
// cos / sin in double precision rounded once.
DEV void draw_plane_wave(uint32_t s0, uint32_t env, uint32_t ep, int radio_model, int fi, int kk, float dc,
                         int spectrum, float* fp) {
    constexpr uint32_t CH_RESET_ = 3, LOG_DISTANCE_STREAM = 10, TR38901_STREAM = (0x52u << 16) + 16u;
    uint32_t st0 = radio_model == 1 ? TR38901_STREAM + 3u * fi : LOG_DISTANCE_STREAM;
    float u0 = uniform_bits(elem_hash(base_key(s0, env, ep, CH_RESET_, 0u, st0 + 0u), (uint32_t)kk));
    float u1 = uniform_bits(elem_hash(base_key(s0, env, ep, CH_RESET_, 0u, st0 + 1u), (uint32_t)kk));
    float u2 = uniform_bits(elem_hash(base_key(s0, env, ep, CH_RESET_, 0u, st0 + 2u), (uint32_t)kk));
    float ang = (u0 * 2.0f) * (float)3.141592653589793;          // rand * 2 * pi, in that order
    float kmag;
    if (spectrum == 0) {                                          // "sos": wavelengths 20..60 m
        float wl = 20.0f + 40.0f * u1;
        if (dc != 10.3f) wl = wl * (float)((double)dc / 10.3);
        kmag = (1.0f / wl) * (float)6.283185307179586;            // 2 pi / wl = reciprocal(wl) * 2 pi
    } else {                                                      // "exp": inverse CDF of the radial spectrum
        float u = clamp_max(u1, (float)(1.0 - 1e-6));
        float a = 1.0f - u;
        kmag = sqrtf(1.0f / (a * a) - 1.0f) / dc;
    }
    fp[0] = (float)cos((double)ang) * kmag;
    fp[1] = (float)sin((double)ang) * kmag;
    fp[2] = (u2 * 2.0f) * (float)3.141592653589793;
}

// exclusive prefix sum over the wavefront of a per-lane count 0 <= v < 64 and the wave total: one ballot per bit of
// v, counted below the lane (mbcnt), no LDS round trip
DEV int wave_prefix64(int v, int wl, int& total) {
    const unsigned long long below = wl ? (~0ull >> (64 - wl)) : 0ull;
    int pre = 0, tot = 0;
#pragma unroll
    for (int b = 0; b < 6; ++b) {
        const unsigned long long m = __ballot((v >> b) & 1);
        pre += __popcll(m & below) << b;
        tot += __popcll(m) << b;
    }
    total = tot;
    return pre;
}

// ---------------------------------------------------------------- segment collectives (RB lanes, power of two)
DEV unsigned long long seg_bits(int rb, int lane) {
    unsigned long long m = rb >= 64 ? ~0ull : ((1ull << rb) - 1ull);
    return m << (lane & ~(rb - 1) & 63);
}
DEV bool seg_any(bool p, int rb, int lane) { return (__ballot(p) & seg_bits(rb, lane)) != 0ull; }

DEV int seg_sum_i(int v, int rb) {
    for (int o = rb >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
DEV int64_t seg_sum_l(int64_t v, int rb) {
    for (int o = rb >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
DEV int seg_max_i(int v, int rb) {
    for (int o = rb >> 1; o > 0; o >>= 1) { int w = __shfl_xor(v, o, 64); v = w > v ? w : v; }
    return v;
}
// argmax with the first index on ties (torch max / argmax)
DEV void seg_argmax(float& v, int& i, int rb) {
    for (int o = rb >> 1; o > 0; o >>= 1) {
        float v2 = __shfl_xor(v, o, 64);
        int i2 = __shfl_xor(i, o, 64);
        bool take = (v2 > v) || (v2 == v && i2 < i);
        v = take ? v2 : v;
        i = take ? i2 : i;
    }
}

}  // namespace inet

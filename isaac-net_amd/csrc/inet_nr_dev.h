// Device helpers of the NR uplink engine kernels (gfx950, wave64).
//
// * counter RNG: the lowbias32 hash, keys and Box-Muller normals of isaac_net/core/proto/rng.py:42-62, 164-185
//   (uniforms are bit-exact; normals use this device's logf / cosf / sqrtf);
// * ATen-order float reductions: torch's CPU sum over a short contiguous row (8-wide vectors, tail elements first,
//   then the vector lanes in order; rows under 8 elements in four interleaved partial sums) and logsumexp
//   (max, masked to 0 when infinite, + log of the sum of exp(x - max)). Replaying the reference's summation order
//   keeps the GPU bitwise equal to the CPU path wherever no transcendental function is involved;
// * segment collectives: a 64-lane wavefront holds 64 / RB envs, one robot per lane in a power-of-two segment of
//   RB lanes; reductions across the robots of one env are butterflies inside the segment (ds_bpermute) or
//   ballots (SALU).
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
// Box-Muller, cosine branch, from the hashes of elements 2j and 2j + 1
DEV float normal_of(uint32_t h1, uint32_t h2) {
    float u1 = (float)((h1 >> 8) + 1u) * INV24;
    float u2 = (float)(h2 >> 8) * INV24;
    return sqrtf(-2.0f * logf(u1)) * cosf((float)6.283185307179586 * u2);
}
// element j of a normal draw uses hash elements 2j and 2j + 1
DEV float normal_at(uint32_t base, uint32_t j) { return normal_of(elem_hash(base, 2u * j), elem_hash(base, 2u * j + 1u)); }

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
// phy._db: 10 log10(max(x, 1e-6)) with NaN -> -30, +inf -> 60, -inf -> -30
DEV float db_of(float lin) { return nan_to_num(10.0f * log10f(clamp_min(lin, 1e-6f)), -30.0f, 60.0f, -30.0f); }
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

// Per-robot Doppler of the NR fading (channels/doppler.py:23-29): the AR(1) correlation per ms of a robot from its
// speed, in float32 as the reference's torch CPU operations compute it.
//
// Plain C++ (host and device): the same header is compiled into the step kernels and, by the CPU tests, with g++
// against torch.special.bessel_j0 and the oracle.
#pragma once

#include <math.h>

#ifndef INET_HD
#if defined(__HIPCC__)
#define INET_HD __host__ __device__
#else
#define INET_HD
#endif
#endif

namespace inet {

// Per-robot Doppler (channels/doppler.py:23-29). J0 as torch.special.bessel_j0 computes it in float32 on [0, 5]:
// Cephes's rational form (z - r1)(z - r2) P(z) / Q(z), z = x^2, Q monic, each polynomial by Horner steps that the
// CPU build fuses into fused multiply-adds; 1 - z / 4 below x = 1e-5.
INET_HD inline float bessel_j0_f32(float x) {
    if (x < 1e-5f) return 1.0f - x * x / 4.0f;
    const float z = x * x;
    float p = -4.79443220978201773821e9f;
    p = fmaf(p, z, 1.95617491946556577543e12f);
    p = fmaf(p, z, -2.49248344360967716204e14f);
    p = fmaf(p, z, 9.70862251047306323952e15f);
    float q = z + 4.99563147152651017219e2f;
    q = fmaf(q, z, 1.73785401676374683123e5f);
    q = fmaf(q, z, 4.84409658339962045305e7f);
    q = fmaf(q, z, 1.11855537045356834862e10f);
    q = fmaf(q, z, 2.11277520115489217587e12f);
    q = fmaf(q, z, 3.10518229857422583814e14f);
    q = fmaf(q, z, 3.18121955943204943306e16f);
    q = fmaf(q, z, 1.71086294081043136091e18f);
    return (((z - 5.78318596294678452118f) * (z - 3.04712623436620863991e1f)) * p) / q;
}

// x ** e of a float32 tensor and a scalar exponent as torch's CPU pow takes it: e = 1, 2, 3 and 0.5 as x, x x,
// (x x) x and sqrt(x); any other exponent within an ulp of the exact power (torch's vectorized pow), here correctly
// rounded (a double exp / log rounded once). x >= 0.
INET_HD inline float pow_scalar_f32(float x, float e) {
    if (e == 1.0f) return x;
    if (e == 2.0f) return x * x;
    if (e == 3.0f) return (x * x) * x;
    if (e == 0.5f) return sqrtf(x);
    if (x == 0.0f) return e > 0.0f ? 0.0f : 1.0f;
    return (float)exp((double)e * log((double)x));
}

// The AR(1) correlation per ms of a robot at speed v (m/s): J0(kx f_D)^(1 / 2.5), f_D = v kf (kf = f_c / c, kx =
// 2 pi 2.5 ms, float32 products as torch's tensor-scalar multiplies), 0 from the first zero of J0 on (the comparison in
// float32), J0 clamped to [0, 1] (NaN stays NaN)
INET_HD inline float doppler_rho_ms(float v, float kf, float kx) {
    const float fd = v * kf;
    const float x = kx * fd;
    float j = x >= 2.404825557695773f ? 0.0f : bessel_j0_f32(x);
    j = j < 0.0f ? 0.0f : (j > 1.0f ? 1.0f : j);
    return pow_scalar_f32(j, 0.4f);
}

}  // namespace inet

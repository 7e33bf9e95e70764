"""Per-robot Doppler (csrc/doppler.h, channels/doppler.py:23-29): the step kernels' float32 J0 equals
torch.special.bessel_j0 bit for bit on the whole range the correlation uses (0 .. the first zero of J0) but at two
points (an ulp), and the correlation per ms rho = J0(2 pi 2.5 ms v f_c / c)^(1 / 2.5) and the per-row power rho^(dt slot_ms) are within one
float32 ulp of torch's (whose vectorized pow is itself within an ulp of the exact power; the header's is correctly
rounded) and equal at the forms torch special-cases (exponents 1, 2, 3, 0.5). Compiled for the host with g++ (the
header is plain C++) with the library's flags for floating point (no contraction)."""
import math
import os
import subprocess

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
HDR = os.path.join(HERE, "..", "isaac-net_amd", "csrc")

DRIVER = r"""
#include <cstdio>
#include <cstring>
#include <vector>
#include "doppler.h"
// stdin: mode n then n hex float32 words (and for mode 2 the exponent as a hex word first); stdout: n hex words
int main() {
    int mode, n;
    while (scanf("%d %d", &mode, &n) == 2) {
        unsigned eu = 0, u;
        float e = 0.f, kf = 0.f, kx = 0.f;
        if (mode == 1) {
            unsigned a, b;
            if (scanf("%x %x", &a, &b) != 2) return 1;
            memcpy(&kf, &a, 4); memcpy(&kx, &b, 4);
        }
        if (mode == 2) { if (scanf("%x", &eu) != 1) return 1; memcpy(&e, &eu, 4); }
        for (int i = 0; i < n; ++i) {
            if (scanf("%x", &u) != 1) return 1;
            float x, y;
            memcpy(&x, &u, 4);
            if (mode == 0) y = inet::bessel_j0_f32(x);
            else if (mode == 1) y = inet::doppler_rho_ms(x, kf, kx);
            else y = inet::pow_scalar_f32(x, e);
            memcpy(&u, &y, 4);
            printf("%x ", u);
        }
        printf("\n");
    }
    return 0;
}
"""


@pytest.fixture(scope="module")
def drv(tmp_path_factory):
    d = tmp_path_factory.mktemp("doppler")
    src, exe = d / "drv.cpp", d / "drv"
    src.write_text(DRIVER)
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", f"-I{HDR}", "-o", str(exe), str(src)], check=True)
    return exe


def _hex(a):
    return " ".join(f"{b:x}" for b in np.asarray(a, dtype=np.float32).view(np.uint32))


def _run(exe, mode, x, extra=()):
    head = f"{mode} {len(x)} " + " ".join(extra)
    out = subprocess.run([str(exe)], input=head + " " + _hex(x) + "\n", capture_output=True, text=True, check=True)
    return np.array([int(w, 16) for w in out.stdout.split()], dtype=np.uint32).view(np.float32)


def _ulps(a, b):
    return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))


def test_j0_vs_torch(drv):
    """Every float32 step of 2^-21 in [0, 2.4049] and the smallest arguments (the 1 - x^2 / 4 branch below 1e-5):
    bitwise equal but at 2 of the 5,043,456 grid points (x = 2.2584953 and 2.356007, one ulp: a rounding inside
    torch's build that no order of these operations reproduces), never more than an ulp."""
    x = np.concatenate([np.arange(0, 2.4049, 2.0 ** -21, dtype=np.float64).astype(np.float32),
                        np.float32([0.0, 1e-30, 1e-7, 9.99999e-6, 1e-5, 1.00001e-5])])
    mine = _run(drv, 0, x)
    ref = torch.special.bessel_j0(torch.from_numpy(x)).numpy()
    u = _ulps(mine, ref)
    assert u.max() <= 1 and int((u > 0).sum()) <= 2, (int(u.max()), x[u > 0][:10])


def _torch_rho_ms(v, fc_ghz):
    """channels/doppler.py:23-29 in torch (float32 CPU)."""
    fd = torch.from_numpy(v) * (fc_ghz * 1e9 / 299_792_458.0)
    x = 2 * math.pi * 2.5 * 1e-3 * fd
    j0 = torch.where(x >= 2.404825557695773, torch.zeros_like(x), torch.special.bessel_j0(x))
    return (j0.clamp(0.0, 1.0) ** (1 / 2.5)).numpy()


@pytest.mark.parametrize("fc_ghz", [3.5, 2.4, 28.0])
def test_rho_per_ms_within_an_ulp(drv, fc_ghz):
    """Speeds 0 .. 30 m/s (past the first zero of J0 at every carrier) and the cut-off itself."""
    v = np.concatenate([np.linspace(0.0, 30.0, 300001, dtype=np.float32), np.float32([0.0, 1e-3, np.nan])])
    kf = np.float32(fc_ghz * 1e9 / 299_792_458.0)
    kx = np.float32(2 * math.pi * 2.5 * 1e-3)
    mine = _run(drv, 1, v, (_hex([kf]), _hex([kx])))
    ref = _torch_rho_ms(v, fc_ghz)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(mine), np.isnan(ref))
    u = _ulps(mine[fin], ref[fin])
    assert u.max() <= 1, int(u.max())
    assert (mine[fin] == 0).sum() == (ref[fin] == 0).sum() > 0       # the same robots past the first zero


@pytest.mark.parametrize("e", [0.25, 0.4, 0.5, 0.75, 1.0, 1.5, 2.0, 2.5, 3.0, 5.0])
def test_row_power_within_an_ulp(drv, e):
    """rho^(dt slot_ms) of the fading rows: exact at torch's special forms, else within an ulp."""
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.uniform(0, 1, 200000), [0.0, 1.0, 0.5]]).astype(np.float32)
    mine = _run(drv, 2, x, (_hex([np.float32(e)]),))
    ref = (torch.from_numpy(x) ** e).numpy()
    u = _ulps(mine, ref)
    if e in (1.0, 2.0, 3.0):
        assert u.max() == 0
    else:
        assert u.max() <= 1
    exact = (np.float64(x) ** np.float64(np.float32(e))).astype(np.float32)    # (the exponent as float32)
    if e not in (0.5, 3.0):                       # (torch's sqrt and (x x) x are not correctly rounded)
        assert np.array_equal(mine, exact)


def test_planted_error_in_j0_is_caught(drv):
    """A J0 without the fused Horner steps (separately rounded products and sums) differs from torch's: the bitwise
    check above pins the contraction, not only the coefficients."""
    x = np.arange(0.01, 2.4, 1e-4, dtype=np.float32)
    z = (x * x).astype(np.float32)
    p = np.float32(-4.79443220978201773821e9)
    for c in (1.95617491946556577543e12, -2.49248344360967716204e14, 9.70862251047306323952e15):
        p = (p * z + np.float32(c)).astype(np.float32)
    q = (z + np.float32(4.99563147152651017219e2)).astype(np.float32)
    for c in (1.73785401676374683123e5, 4.84409658339962045305e7, 1.11855537045356834862e10,
              2.11277520115489217587e12, 3.10518229857422583814e14, 3.18121955943204943306e16,
              1.71086294081043136091e18):
        q = (q * z + np.float32(c)).astype(np.float32)
    wrong = (((z - np.float32(5.78318596294678452118)) * (z - np.float32(30.4712623436620863991))) * p / q)
    ref = torch.special.bessel_j0(torch.from_numpy(x)).numpy()
    assert not np.array_equal(wrong.astype(np.float32), ref)
    assert np.array_equal(_run(drv, 0, x), ref)

"""Device arithmetic that replaces an IEEE operation by a cheaper exact one, checked exhaustively on the CPU.

div_const (isaac-net_amd/csrc/inet_nr_dev.h): x / y for a constant y as q = RN(x r), e = fma(-q, y, x),
RN(q + e r) with r = RN(1 / y). The check emulates the two fmas exactly (float64 products of float32 operands are
exact; the final sum is rounded once from its TwoSum representation) over every float32 significand, i.e. every
x in [1, 2); division by y is scale invariant, so this covers every normal x whose quotient is normal.
"""
import numpy as np
import pytest


def fma_div_mismatches(y):
    y = np.float32(y)
    r = np.float32(1.0) / y
    x = (np.arange(1 << 23, dtype=np.uint32) | np.uint32(0x3F800000)).view(np.float32)
    want = (x.astype(np.float64) / np.float64(y)).astype(np.float32)    # RN32(x / y): double suffices for float32
    q0 = (x * r).astype(np.float32)
    e = (x.astype(np.float64) - q0.astype(np.float64) * np.float64(y)).astype(np.float32)   # exact residual, RN32
    p = e.astype(np.float64) * np.float64(r)                                                 # exact product
    a = q0.astype(np.float64)
    s = a + p
    t = s - a
    err = (a - (s - t)) + (p - t)                                                            # s + err = a + p
    f = s.astype(np.float32)
    lo, hi = np.nextafter(f, np.float32(-np.inf)), np.nextafter(f, np.float32(np.inf))
    fd = f.astype(np.float64)
    tie_hi, tie_lo = s == (fd + hi.astype(np.float64)) / 2, s == (fd + lo.astype(np.float64)) / 2
    got = np.where(tie_hi & (err > 0), hi, np.where(tie_lo & (err < 0), lo, f))
    got = np.where(tie_hi & (err < 0), f, np.where(tie_lo & (err > 0), f, got))
    return int(np.count_nonzero(got != want)), int(np.count_nonzero(q0 != want))


@pytest.mark.parametrize("y", [1.4142135623730951, 10.0])
def test_div_const_exact(y):
    bad, bad_uncorrected = fma_div_mismatches(y)
    assert bad == 0
    assert bad_uncorrected > 0           # the check does see the error of the plain product q = RN(x r)

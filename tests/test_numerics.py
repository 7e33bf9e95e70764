"""Device arithmetic that replaces an IEEE operation by a cheaper exact one, checked exhaustively on the CPU.

div_const (isaac-net_amd/csrc/inet_nr_dev.h): x / y for a divisor y fixed per launch as q = RN(x r),
e = fma(-q, y, x), RN(fma(e, r, q)) with r = RN(1 / y) (Markstein's correction). A small C program (gcc, IEEE fmaf
and float division) compares it with x / y for every float32 significand, i.e. every x in [1, 2); float division
is scale invariant, so this covers every normal x with a normal quotient. The divisors are the ones the kernels use:
sqrt 2 (fading normals), 10 (dB to linear), the EESM beta of every MCS of the shipped tables, and the BLER table's
SINR and code-block grid steps.
"""
import os
import subprocess
import tempfile

import numpy as np
import pytest

from isaac_net_amd import phy

C_SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
int main(int argc, char** argv) {
    int n = argc - 1;
    for (int i = 0; i < n; ++i) {
        float y = strtof(argv[i + 1], NULL);
        float r = 1.0f / y;
        long bad = 0, bad_plain = 0;
        for (uint32_t m = 0; m < (1u << 23); ++m) {
            float x = f_of(0x3F800000u | m);
            float want = x / y;
            float q = x * r;
            float e = fmaf(-q, y, x);
            float got = fmaf(e, r, q);
            bad += got != want;
            bad_plain += q != want;
        }
        printf("%.9g %ld %ld\n", (double)y, bad, bad_plain);
    }
    return 0;
}
"""


def divisors():
    ys = [float(np.float32(np.sqrt(2.0))), 10.0]
    for mt in (1, 2):
        t = phy.PhyTables(mcs_table=mt)
        ys += [float(b) for b in t.beta] + [float(t.ds), float(t.dc)]
    return sorted(set(ys))


def test_div_const_exact_for_every_kernel_divisor():
    ys = divisors()
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "divcheck.c"), os.path.join(d, "divcheck")
        open(src, "w").write(C_SRC)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", exe, src, "-lm"], check=True)
        out = subprocess.run([exe] + [repr(np.float32(y).item()) for y in ys], check=True, capture_output=True,
                             text=True, timeout=600).stdout.split("\n")
    rows = [l.split() for l in out if l]
    assert len(rows) == len(ys)
    bad = [(y, b) for y, b, _ in rows if int(b) != 0]
    assert not bad, bad
    assert sum(int(p) for _, _, p in rows) > 0          # the plain product q = RN(x r) does differ: the check sees it


# cos_small (inet_nr_dev.h), the cosine of the Box-Muller angle x = RN(2 pi) u2 for the 2^24 values u2 = i 2^-24:
# the device steps restated in C with IEEE fmaf / rintf, their constants read from the header's source, against
# the double-precision cosine. A wrong constant, a dropped reduction part or a wrong quadrant sign fails by far more
# than the bound.
COS_SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
static float k[11];
static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static float cos_small(float x) {
    const float jf = rintf(x * k[0]);
    const int j = (int)jf;
    float r = fmaf(jf, k[1], x);
    r = fmaf(jf, k[2], r);
    r = fmaf(jf, k[3], r);
    const float r2 = r * r;
    float sp = fmaf(r2, k[4], k[5]);
    sp = fmaf(r2, sp, k[6]);
    const float sn = fmaf(r, r2 * sp, r);
    float cp = fmaf(r2, k[7], k[8]);
    cp = fmaf(r2, cp, k[9]);
    cp = fmaf(r2, cp, k[10]);
    const float cs = fmaf(r2, cp, 1.0f);
    float v = (j & 1) ? -sn : cs;
    uint32_t u;
    memcpy(&u, &v, 4);
    u ^= ((uint32_t)j << 30) & 0x80000000u;
    memcpy(&v, &u, 4);
    return v;
}
int main(int argc, char** argv) {
    for (int i = 0; i < 11; ++i) k[i] = f_of((uint32_t)strtoul(argv[i + 1], NULL, 16));
    const float two_pi = (float)6.283185307179586;
    double max_abs = 0.0, max_ulp = 0.0;
    long not_rn = 0;
    for (uint32_t i = 0; i < (1u << 24); ++i) {
        const float x = two_pi * ((float)i * 0x1p-24f);
        const float c = cos_small(x);
        const double ref = cos((double)x);
        const double err = fabs((double)c - ref);
        const float rf = (float)ref;
        const double ulp = (double)nextafterf(fabsf(rf), INFINITY) - (double)fabsf(rf);
        if (err > max_abs) max_abs = err;
        if (err / ulp > max_ulp) max_ulp = err / ulp;
        not_rn += c != rf;
    }
    printf("%.6g %.6g %ld\n", max_abs, max_ulp, not_rn);
    return 0;
}
"""


def cos_small_constants():
    """The eleven float constants of cos_small, in the order they appear in its body."""
    import re
    src = open(os.path.join(os.path.dirname(__file__), "..", "isaac-net_amd", "csrc", "inet_nr_dev.h")).read()
    body = src[src.index("DEV float cos_small(float x) {"):]
    body = body[:body.index("\n}\n")]
    return re.findall(r"__int_as_float\((0x[0-9a-f]{8})\)", body)


def _run_cos(consts):
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "coscheck.c"), os.path.join(d, "coscheck")
        open(src, "w").write(COS_SRC)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", exe, src, "-lm"], check=True)
        out = subprocess.run([exe] + consts, check=True, capture_output=True, text=True, timeout=600).stdout.split()
    return float(out[0]), float(out[1]), int(out[2])


def test_box_muller_cosine_over_every_u2():
    consts = cos_small_constants()
    assert len(consts) == 11
    max_abs, max_ulp, not_rn = _run_cos(consts)
    # within 2 ulp of the exact cosine (cosf's bound) and one ulp of 1.0 (2^-23) absolute: far inside the 1e-5
    # relative tolerance of the fading state the normals feed
    assert max_ulp <= 2.0 and max_abs <= 2.0 ** -23, (max_abs, max_ulp, not_rn)
    # a planted mistake (the second reduction part dropped) must fail the same bound
    bad = list(consts)
    bad[2] = "0x00000000"
    b_abs, b_ulp, _ = _run_cos(bad)
    assert b_ulp > 2.0 or b_abs > 2.0 ** -23

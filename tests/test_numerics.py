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

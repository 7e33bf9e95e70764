"""The step kernels' ranking of retransmission candidates (csrc/aten_sort.h, libstdc++'s std::sort over (key,
index) pairs as ATen's CPU sort runs it) against torch.argsort(descending=True) (isaac_net/core/mac.py:301, 307): the
same permutation, ties included, for the sizes the kernels rank (up to 256 robots) and for the tie patterns the
admission meets (equal metric sums, the -1 keys of robots that are not candidates, NaN). Compiled for the host with
g++ (the header is plain C++)."""
import os
import subprocess

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
HDR = os.path.join(HERE, "..", "isaac-net_amd", "csrc")

DRIVER = r"""
#include <cstdio>
#include <vector>
#include "aten_sort.h"
int main() {
    int t;
    if (scanf("%d", &t) != 1) return 1;
    while (t--) {
        int n;
        if (scanf("%d", &n) != 1) return 1;
        std::vector<float> k(n);
        std::vector<int> v(n), stk(64);
        for (int i = 0; i < n; ++i) {
            unsigned u;
            if (scanf("%x", &u) != 1) return 1;
            __builtin_memcpy(&k[i], &u, 4);
            v[i] = i;
        }
        inet::AtenSortDesc s{k.data(), v.data()};
        s.sort(n, stk.data());
        for (int i = 0; i < n; ++i) printf("%d ", v[i]);
        printf("\n");
    }
    return 0;
}
"""


@pytest.fixture(scope="module")
def sorter(tmp_path_factory):
    d = tmp_path_factory.mktemp("aten_sort")
    src, exe = d / "drv.cpp", d / "drv"
    src.write_text(DRIVER)
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{HDR}", "-o", str(exe), str(src)], check=True)
    return exe


def _run(exe, cases):
    lines = [str(len(cases))]
    for c in cases:
        bits = np.asarray(c, dtype=np.float32).view(np.uint32)
        lines.append(f"{len(c)} " + " ".join(f"{b:x}" for b in bits))
    out = subprocess.run([str(exe)], input="\n".join(lines) + "\n", capture_output=True, text=True, check=True)
    return [[int(x) for x in ln.split()] for ln in out.stdout.strip().split("\n")]


def test_matches_torch_argsort_descending(sorter):
    rs = np.random.default_rng(7)
    cases = []
    for n in (1, 2, 3, 8, 15, 16, 17, 18, 24, 31, 32, 33, 40, 47, 48, 63, 64, 65, 96, 100, 127, 128, 129, 200, 255, 256):
        for _ in range(40):
            pool = np.concatenate([rs.choice([-1.0, 0.0, 0.0, 1.5, 2.5], 3), rs.random(3)]).astype(np.float32)
            k = rs.choice(pool, n)
            if rs.random() < 0.1:
                k[rs.integers(0, n)] = np.nan
            cases.append(k)
    # long runs of one key (the non-candidates' -1 everywhere but a few ties), sorted and reversed inputs
    for n in (17, 48, 64, 128, 256):
        k = np.full(n, -1.0, np.float32)
        k[rs.choice(n, 5, replace=False)] = 0.0
        cases += [k, np.sort(rs.random(n)).astype(np.float32), np.sort(rs.random(n))[::-1].astype(np.float32),
                  np.zeros(n, np.float32)]
    got = _run(sorter, cases)
    for k, g in zip(cases, got):
        want = torch.from_numpy(np.ascontiguousarray(k)).argsort(-1, descending=True).tolist()
        assert g == want, (len(k), k.tolist())


def test_heapsort_branch_matches(sorter):
    """Keys that exhaust the introsort depth limit (tests/golden/sort_killers.npz, McIlroy's adversary against the
    same steps, checked there to reach the heapsort branch; the keys never fixed by the adversary are equal) and those
    keys with every second one tied: the order is still torch's."""
    from conftest import GOLDEN
    d = np.load(os.path.join(GOLDEN, "sort_killers.npz"))
    cases = []
    for n in (64, 128, 256):
        k = d[f"n{n}"]
        t = k.copy()
        t[::2] = np.floor(t[::2] / 4.0)
        cases += [k, t]
    got = _run(sorter, cases)
    for k, g in zip(cases, got):
        assert g == torch.from_numpy(k).argsort(-1, descending=True).tolist()


def test_index_order_differs_from_torch_above_16():
    """Why the kernels need the exact steps: beyond 16 elements torch's order of equal keys is not the index order."""
    k = torch.full((48,), -1.0)
    k[::3] = 0.0
    ties = [int(i) for i in k.argsort(descending=True) if k[i] == 0.0]
    assert ties != sorted(ties)

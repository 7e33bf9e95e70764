"""Build libinet_nr.so (the C-ABI HIP library) in-tree for gfx950.

    python isaac-net_amd/build.py            # or __graft_entry__.build()

Flags: -ffp-contract=off keeps every float multiply and add separately rounded (the op order mirrors the
reference's torch expressions), and packed FP32 instructions are disabled for this target.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libinet_nr.so")
SRC = [os.path.join(HERE, "csrc", "inet_nr.hip")]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function"]


def build(verbose=False):
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, "-o", tmp, *SRC]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

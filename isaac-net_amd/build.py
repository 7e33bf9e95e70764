"""Build libinet_nr.so (the C-ABI HIP library) in-tree for gfx950.

    python isaac-net_amd/build.py            # or __graft_entry__.build()
    python isaac-net_amd/build.py --phase-clocks   # libinet_nr_phase.so: the step kernels with per-phase clocks

The step-kernel instantiations are split over translation units (one per subband count) that compile in parallel
and link into one shared library. Flags: -ffp-contract=off keeps every float multiply and add separately rounded
(the op order mirrors the reference's torch expressions), and packed FP32 instructions are disabled for this target.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libinet_nr.so")
PHASE_LIB = os.path.join(HERE, "libinet_nr_phase.so")
# (the units with the most and the largest instantiations first: the pool's last unit sets the build's wall time)
UNITS = [f"nr_step_mc{c}.hip" for c in (7, 6, 5, 4)] + \
        ["nr_step_s13.hip", "nr_step_w2.hip", "nr_step_w4.hip", "nr_step_mc.hip", "nr_step_mc2.hip", "nr_step_s8.hip"] + \
        [f"nr_step_s{s}.hip" for s in (10, 11, 12, 14, 16, 17, 18)] + ["inet_nr.hip", "wifi.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function"]


def source_hash():
    """SHA-256 over the library's sources (csrc/*.h, csrc/*.hip, include/*.h, this file), in name order."""
    import glob
    import hashlib
    h = hashlib.sha256()
    files = sorted(glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(CSRC, "*.hip")) +
                   glob.glob(os.path.join(HERE, "..", "include", "*.h"))) + [os.path.abspath(__file__)]
    for f in files:
        h.update(os.path.basename(f).encode())
        with open(f, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def build(verbose=False, out_dir=None, phase_clocks=False):
    """Compile every unit and link the library. phase_clocks: the same sources with INET_PHASE_CLOCKS defined (every
    step-kernel wavefront records the shader clock spent in each phase of the step), linked as libinet_nr_phase.so
    for bench.py --phase-clocks; the product library is not touched."""
    obj_dir = out_dir or os.path.join(HERE, "_build_phase" if phase_clocks else "_build")
    os.makedirs(obj_dir, exist_ok=True)
    src = source_hash()
    extra = ["-DINET_PHASE_CLOCKS"] if phase_clocks else []

    def compile_unit(u):
        obj = os.path.join(obj_dir, u.replace(".hip", ".o"))
        cmd = [HIPCC, *FLAGS, *extra, f'-DINET_SRC_HASH="{src}"', "-c", "-o", obj, os.path.join(CSRC, u)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        return obj

    with cf.ThreadPoolExecutor(min(len(UNITS), os.cpu_count() or 8)) as ex:
        objs = list(ex.map(compile_unit, UNITS))
    lib = PHASE_LIB if phase_clocks else LIB
    tmp = lib + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, phase_clocks="--phase-clocks" in sys.argv))

"""The step kernels built for the common configurations (PF, chase combining, EESM, RLC AM, OLLA, PHR cap, retx
priority, fading; with a fixed Rician phasor: the RL-scale configuration at 13 RBGs, 8 HARQ processes, 32-robot envs;
without: config 5's two-wave kernel at 8 RBGs, 128-robot envs, and config 3's three-cell kernel at 14 RBGs) equal the
general builds bit for bit: outputs and every
state tensor, UL and with the downlink, through a partial reset. INET_NR_GENERIC=1 makes the library launch the
general build for the same call."""
import os

import numpy as np
import pytest
import torch

import isaac_net_amd as P

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def run(name, E, R, steps, generic):
    from isaac_net_amd import scenarios as S
    os.environ["INET_NR_GENERIC"] = "1" if generic else "0"
    try:
        wl = S.Workload(E, R, steps, seed=2, name=name, device=DEV)
        eng = P.make_engine("L2", E, R, DEV, wl.cfg, seed=2)
        outs = []
        for s in range(steps):
            if s == steps // 2:
                eng.reset([1, E - 2])
            if name == "rl_scale_dl":
                for i in range(wl.dl_bytes.shape[1]):
                    eng.add_dl_frames(None, wl.dl_bytes[s, i])
            o = eng.step(None, wl.poses[s], arrivals=wl.counts[s])
            outs.append({k: v.detach().cpu() for k, v in o.items()})
        st = {k: v.detach().cpu() for k, v in eng.owner_state().items()}
        return outs, st
    finally:
        os.environ.pop("INET_NR_GENERIC", None)


def same(a, b):
    if a.is_floating_point():
        return torch.equal(a.nan_to_num(-7.0).view(torch.int32) if a.dtype == torch.float32 else a.nan_to_num(-7.0),
                           b.nan_to_num(-7.0).view(torch.int32) if b.dtype == torch.float32 else b.nan_to_num(-7.0))
    return torch.equal(a, b)


@pytest.mark.parametrize("name", ["rl_scale", "rl_scale_dl", "freq_sel", "mc_interf"])
def test_common_configuration_build_equals_general_build(name):
    E, R, steps = {"freq_sel": (16, 128, 4), "mc_interf": (16, 64, 6)}.get(name, (64, 32, 8))
    print(f"{name} {E}x{R}, {steps} steps: common-configuration build vs general build", flush=True)
    o_fx, st_fx = run(name, E, R, steps, generic=False)
    o_gen, st_gen = run(name, E, R, steps, generic=True)
    for s in range(steps):
        for k in o_fx[s]:
            assert same(o_fx[s][k], o_gen[s][k]), (s, k)
    for k in st_fx:
        assert same(st_fx[k], st_gen[k]), k
    assert int(st_fx["ul.q.enq"].sum()) > 0

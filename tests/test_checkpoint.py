"""Checkpoint headers and checks on the CPU (no engine is stepped): the header of an engine, the kind / level / E / R
/ backend-family / config checks against a checkpoint, and the keys of the reference engine's checkpoint fixture that
the hip engine restores."""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN
import isaac_net_amd as P
from isaac_net_amd import checkpoint


class HipNREngine:
    """The header fields of a hip NR engine (no device state)."""
    level, backend, dev = "L2", "hip", None

    def __init__(self, E, R, config):
        self.E, self.R, self.config = E, R, config


def fake_engine(E=4, R=8, **cfg):
    return HipNREngine(E, R, P.NRConfig(n_prb=52, **cfg))


def test_header_and_checks():
    eng = fake_engine()
    h = checkpoint.header(eng)
    assert h["kind"] == "NREngine" and h["backend"] == "hip" and h["E"] == 4 and h["format"] == checkpoint.FORMAT
    checkpoint.check(eng, dict(h, backend="reference"))           # same bitwise family
    with pytest.raises(ValueError, match="E:"):
        checkpoint.check(eng, dict(h, E=5))
    with pytest.raises(ValueError, match="backend"):
        checkpoint.check(eng, dict(h, backend="triton"))
    other = checkpoint.header(fake_engine(scheduler="rr"))
    with pytest.raises(ValueError, match="scheduler"):
        checkpoint.check(eng, other)
    with pytest.warns(UserWarning):
        checkpoint.check(eng, other, strict=False)
    # fields only the reference's config has are not compared; the seed never is
    theirs = dict(h, config=dict(h["config"], seed=7, some_reference_only_field=1))
    checkpoint.check(eng, theirs)


def test_reference_checkpoint_holds_the_restored_state():
    """The reference engine's checkpoint (its state_dict after 10 steps) holds every key the hip engine restores."""
    z = np.load(os.path.join(GOLDEN, "ckpt_dl_c2.npz"), allow_pickle=False)
    keys = {k[3:] for k in z.files if k.startswith("ck/")}
    host = json.loads(bytes(z["host_json"]).decode())
    link = ("sent", "floor", "olla", "avg", "csi", "h_state", "h_lo", "h_hi", "h_ready", "h_ntx", "h_mcs", "h_tbs",
            "h_nsb", "h_comb", "h_lexp", "h_nrb", "last_tx", "q.cap", "q.start", "q.end", "q.lost", "q.fin",
            "q.cls", "q.enq", "ctr[tb_new]", "ctr[prb_avail]", "ntx_hist", "rv_tx", "rv_fail", "prb_used_env")
    for lk in ("ul", "dl"):
        for k in link:
            assert f"net.{lk}.{k}" in keys, (lk, k)
    for k in ("net.h", "epoch", "_last_snr", "_last_hid", "net.rng.episode", "net.rng.ctr[1]", "net.rng.ctr[2]",
              "net.rng.env", "net.dl_newest", "radio.ch.sf_los.k", "radio.ch.los_field.phi", "net.spec"):
        assert k in keys, k
    assert host["T"] == int(z["k_steps"]) and "net.last_g" in host and "net.rng.s0" in host


def test_reference_multicell_checkpoint_holds_the_restored_state():
    """With three cells the reference's checkpoint also holds the association, each gNB's N+I estimate, the
    interference statistic, the fading of every link [E,R,C,S,2] and one shadowing field per cell [C,E,K,2]."""
    z = np.load(os.path.join(GOLDEN, "ckpt_mc3_ho.npz"), allow_pickle=False)
    keys = {k[3:] for k in z.files if k.startswith("ck/")}
    for k in ("net.assoc.serv", "net.assoc.pending", "net.assoc.a3_cand", "net.assoc.a3_cnt", "net.assoc.ho_end",
              "net.assoc.n_ho", "net.ni_ul", "net.ioN[ul]", "net.h", "radio.k", "radio.phi"):
        assert k in keys, k
    E, R = int(json.loads(bytes(z["host_json"]).decode())["E"]), int(json.loads(bytes(z["host_json"]).decode())["R"])
    assert z["ck/net.h"].shape == (E, R, 3, 13, 2) and z["ck/radio.k"].shape[:2] == (3, E)

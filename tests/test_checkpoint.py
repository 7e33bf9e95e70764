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
    # the seed is never compared; a reference-only field at its reference default passes
    theirs = dict(h, config=dict(h["config"], seed=7, drx_cycle_ms=160.0))
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


def test_reference_only_fields_must_hold_their_reference_defaults():
    """A reference config field that this build does not model (DRX, RLF, TPC, MIMO, ...) passes the check only at
    its reference default; another value, or a field neither side knows, is refused."""
    from isaac_net_amd.config import REFERENCE_ONLY_DEFAULTS
    eng = fake_engine()
    h = checkpoint.header(eng)
    ref_cfg = dict(h["config"], **{k: checkpoint._plain(v) for k, v in REFERENCE_ONLY_DEFAULTS.items()})
    checkpoint.check(eng, dict(h, config=ref_cfg))                # every reference-only field at its default
    for k, v in (("drx_cycle_ms", 320.0), ("n310", 4), ("ul_mimo", True), ("rach_initial", "idle"),
                 ("qos_pdb_ms", [20.0, float("inf")])):
        with pytest.raises(ValueError, match=k):
            checkpoint.check(eng, dict(h, config=dict(ref_cfg, **{k: v})))
    with pytest.raises(ValueError, match="not_a_field"):
        checkpoint.check(eng, dict(h, config=dict(ref_cfg, not_a_field=1)))


def test_strict_state_loading_refuses_what_this_engine_does_not_run():
    """Under strict loading a state tensor the engine neither restores nor knows to skip, or a reference host switch
    that is on (a traffic model, an access procedure, a hook), is refused; generators, config-derived constants and
    the reference's per-step caches are skipped."""
    import torch
    from isaac_net_amd.engine import HipNREngine as E
    ok = {"net.ul.sent": torch.zeros(2), "gen": torch.zeros(3), "radio.ch.sf_los.gen": torch.zeros(3),
          "net.sizes": torch.zeros(2), "access": None, "_extras": False, "net.ul.slot_hook": None, "E": 4}
    assert E._strict_extra_keys(E, ok, {"net.ul.sent"}) == []
    # the LENA grant counters' switch must equal the config's: on only with a 5G-LENA MAC switch set
    lena = dict(ok, **{"net.ul._lena_mac": True})
    assert E._strict_extra_keys(E, lena, {"net.ul.sent"}) == ["net.ul._lena_mac=True"]

    class _Cfg(E):                                    # (the class attributes of the engine, a LENA config)
        config = P.NRConfig(ul_retx_sched="tdma")
    assert E._strict_extra_keys(_Cfg, lena, {"net.ul.sent"}) == []
    assert E._strict_extra_keys(_Cfg, dict(ok, **{"net.ul._lena_mac": False}), {"net.ul.sent"}) == \
        ["net.ul._lena_mac=False"]
    assert E._strict_extra_keys(E, dict(ok, **{"net.ul.tag": torch.zeros(2)}), {"net.ul.sent"}) == ["net.ul.tag"]
    bad = E._strict_extra_keys(E, dict(ok, access={"state": 1}, traffic="poisson"), {"net.ul.sent"})
    assert len(bad) == 2 and bad[0].startswith("access=")

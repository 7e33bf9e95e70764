"""Replay a golden trajectory (tests/golden/traj_*.npz) on an engine: same inputs, resets and submit order.
Test infrastructure only (see oracle/__init__.py)."""
from __future__ import annotations

import json

import numpy as np
import torch


def load_case(path):
    d = np.load(path, allow_pickle=False)
    cfg = json.loads(bytes(d["cfg_json"]).decode())
    for k in ("msg_sizes", "cell_positions_m", "cell_center_m"):
        if k in cfg:
            cfg[k] = tuple(tuple(v) if isinstance(v, list) else v for v in cfg[k])
    return d, cfg, bytes(d["kind"]).decode()


def submits(counts_s):
    """The harness's submit calls of one step: class 1 first, one call per message index. counts_s [E,R,NC]."""
    out = []
    for ci in range(counts_s.shape[-1]):
        n = counts_s[..., ci]
        for i in range(int(n.max()) if n.size else 0):
            out.append(np.where(n > i, ci + 1, 0).astype(np.int64))
    return out


def dl_frames(d, s):
    """The harness's add_dl_frames calls of step s: (bytes [E,R] float32, class [E,R] int64) per call, DL class 1
    first, one call per message index (empty without a downlink)."""
    if "dl_counts" not in d.files:
        return []
    out = []
    cnt, sizes = d["dl_counts"][s], d["dl_sizes"]
    for ci in range(cnt.shape[-1]):
        n = cnt[..., ci]
        for i in range(int(n.max()) if n.size else 0):
            out.append((np.where(n > i, sizes[ci], 0.0).astype(np.float32), np.where(n > i, ci + 1, 0).astype(np.int64)))
    return out


def run(eng, d, kind, steps=None, on_step=None, to=lambda a: torch.from_numpy(a)):
    """Drive eng (oracle or HIP engine) through the case; on_step(s, out, accepted_list) after every step."""
    T = int(d["steps"]) if steps is None else steps
    for s in range(T):
        ids = np.nonzero(d["reset_mask"][s])[0]
        if len(ids):
            eng.reset(ids.tolist())
        acc = [eng.submit(None, to(send)) for send in submits(d["counts"][s])]
        for nb, cls in dl_frames(d, s):
            eng.add_dl_frames(None, to(nb), to(cls))
        x = to(d["x"][s])
        if kind == "snr3":
            o = eng.step(None, snr_db=x)
        elif kind == "pg":
            o = eng.step(None, pathgain_db=x)
        elif "vel" in d.files:
            o = eng.step(None, x, vel=to(d["vel"][s]))
        else:
            o = eng.step(None, x)
        if on_step is not None:
            on_step(s, o, acc)


def load_wifi_case(path, NRConfig, WifiConfig):
    """(arrays, NRConfig with its WifiConfig, input kind "snr" | "pose") of a level WIFI trajectory."""
    d = np.load(path, allow_pickle=False)
    cfg = json.loads(bytes(d["cfg_json"]).decode())
    wc = json.loads(bytes(d["wifi_json"]).decode())
    for k in ("msg_sizes", "cell_positions_m"):
        if k in cfg:
            cfg[k] = tuple(tuple(v) if isinstance(v, list) else v for v in cfg[k])
    for k in ("class_ac", "ap_positions_m", "ap_channels"):
        if wc.get(k) is not None:
            wc[k] = tuple(tuple(v) if isinstance(v, list) else v for v in wc[k])
    return d, NRConfig(**cfg, wifi=WifiConfig(**wc), seed=0), bytes(d["kind"]).decode()

"""Checkpoints of a running engine to a file, with the reference's API and file layout (isaac_net/core/checkpoint.py).

    from isaac_net_amd import checkpoint
    checkpoint.save(eng, "isaac_net_100.pt", extra={"iter": 100})
    checkpoint.load(eng2, "isaac_net_100.pt")     # checks kind / level / E / R / config, then restores

The file is torch.save of {"isaac_net_amd": version, "format", "level", "backend", "device", "E", "R", "kind",
"config", "state": engine.state_dict() on the CPU, "global_rng", "extra"}: the reference's layout
(checkpoint.py:431-452), so one reader handles both. The NR engine's state_dict() uses the reference engine's
checkpoint keys ("net.ul.sent", "net.rng.ctr[2]", "radio.ch.sf_los.k", "T", ...): a checkpoint written by the
reference's NR engine (backend "reference", "eager" or "graph") loads into the hip engine and continues bit for bit,
since this backend is bitwise equal to those (the golden-trajectory parity tests); the reverse load needs the
reference's strict=False, since this engine keeps less host state (no torch generators, no trace hooks).
"""
from __future__ import annotations

import dataclasses
import math
import os
import warnings

import torch

FORMAT = 1
VERSION = "0.1"
# backends whose NR engines are bitwise equal to each other (the reference's family, plus this one)
BITWISE = ("reference", "eager", "graph", "hip")


def _plain(v):
    """A config value as plain data (dicts, lists, str, int, float, bool, None), loadable with weights_only=True."""
    if dataclasses.is_dataclass(v) and not isinstance(v, type):
        d = {f.name: _plain(getattr(v, f.name)) for f in dataclasses.fields(v)}
        d["__type__"] = type(v).__name__
        return d
    if isinstance(v, dict):
        return {str(k): _plain(x) for k, x in v.items()}
    if isinstance(v, (list, tuple)):
        return [_plain(x) for x in v]
    if isinstance(v, float) and math.isnan(v):
        return "nan"
    if isinstance(v, (bool, int, float, str, type(None))):
        return v
    if torch.is_tensor(v):
        return v.detach().cpu().tolist()
    return repr(v)


def _kind(engine):
    """The engine kind: the NR engines of every bitwise-equal backend are one kind ("NREngine")."""
    name = type(engine).__name__
    return "NREngine" if name == "HipNREngine" else name


def header(engine) -> dict:
    """The compatibility fields written next to the state: version, format, level, backend, device, E, R, kind,
    config."""
    dev = getattr(engine, "dev", None)
    return {"isaac_net_amd": VERSION, "format": FORMAT, "level": getattr(engine, "level", type(engine).__name__),
            "backend": getattr(engine, "backend", "hip"), "device": str(dev) if dev is not None else None,
            "E": int(engine.E), "R": int(engine.R), "kind": _kind(engine),
            "config": _plain(getattr(engine, "config", None))}


def save(engine, path, extra=None, *, state=None):
    """Write a checkpoint of engine to path (path + ".tmp", then renamed). extra: the caller's data (plain data or
    tensors keep the file loadable with weights_only=True). state: a state dict to write instead of
    engine.state_dict(). Returns path."""
    ck = header(engine)
    sd = engine.state_dict() if state is None else state
    ck["state"] = {k: (v.detach().cpu() if torch.is_tensor(v) else v) for k, v in sd.items()}
    rng = {"cpu": torch.get_rng_state()}
    if torch.cuda.is_available() and torch.cuda.is_initialized():
        rng["cuda"] = list(torch.cuda.get_rng_state_all())
    ck["global_rng"] = rng
    ck["extra"] = extra
    d = os.path.dirname(os.fspath(path))
    if d:
        os.makedirs(d, exist_ok=True)
    tmp = os.fspath(path) + ".tmp"
    torch.save(ck, tmp)
    os.replace(tmp, path)
    return path


def read(path, map_location="cpu"):
    """The checkpoint dict of a file written by save() (or by the reference's checkpoint.save). Loaded with
    weights_only=True: a file whose extra data needs unpickling is refused."""
    return torch.load(path, map_location=map_location, weights_only=True)


def _config_diff(mine, theirs, path=""):
    """Paths of the fields whose values differ between this build's config and the checkpoint's. At the top level a
    field only the checkpoint has must be one of the reference's fields this build does not model, at its reference
    default (config.REFERENCE_ONLY_DEFAULTS): otherwise the checkpoint ran a feature this engine does not, and the
    field is reported too."""
    if isinstance(mine, dict) and isinstance(theirs, dict):
        out = []
        for k in mine:
            if k in ("seed", "__type__") and path == "":
                continue
            if k in theirs:
                out += _config_diff(mine[k], theirs[k], f"{path}{k}.")
        if path == "" and mine.get("__type__") == "NRConfig":
            from .config import REFERENCE_ONLY_DEFAULTS
            for k in theirs:
                if k in mine or k == "__type__":
                    continue
                if k not in REFERENCE_ONLY_DEFAULTS or \
                        _config_diff(_plain(REFERENCE_ONLY_DEFAULTS[k]), theirs[k], f"{k}."):
                    out.append(f"{k} (not modelled by this engine; {theirs[k]!r})")
        return out
    if isinstance(mine, list) and isinstance(theirs, list):
        if len(mine) != len(theirs):
            return [path.rstrip(".")]
        out = []
        for i, (a, b) in enumerate(zip(mine, theirs)):
            out += _config_diff(a, b, f"{path}{i}.")
        return out
    if isinstance(mine, (int, float)) and isinstance(theirs, (int, float)) and not isinstance(mine, bool):
        return [] if float(mine) == float(theirs) else [path.rstrip(".")]
    return [] if mine == theirs else [path.rstrip(".")]


def check(engine, ck, strict=True):
    """Compare a checkpoint's header with engine: kind, level, E, R, the backend family and the config. Raises
    ValueError (strict) or warns on a mismatch."""
    h = header(engine)
    errs = [f"{k}: checkpoint {ck.get(k)!r}, engine {h[k]!r}" for k in ("kind", "level", "E", "R")
            if ck.get(k) != h[k]]
    if ck.get("backend") != h["backend"] and not (ck.get("backend") in BITWISE and h["backend"] in BITWISE):
        errs.append(f"backend: checkpoint {ck.get('backend')!r}, engine {h['backend']!r} (the state restores, but "
                    "the continuation is only as close as the two backends)")
    diff = _config_diff(h["config"], ck.get("config")) if isinstance(ck.get("config"), dict) else []
    if diff:
        errs.append("config differs: " + ", ".join(diff[:10]) + (" ..." if len(diff) > 10 else ""))
    if errs:
        msg = "checkpoint does not match the engine:\n  " + "\n  ".join(errs)
        if strict:
            raise ValueError(msg)
        warnings.warn(msg)


def load(engine, path, strict=True, global_rng=False):
    """Restore engine from a checkpoint file in place (check, then engine.load_state_dict(state, strict)).
    global_rng: also restore the global torch RNG state recorded by save(). Returns the checkpoint's extra."""
    ck = read(path)
    check(engine, ck, strict=strict)
    engine.load_state_dict(ck["state"], strict=strict)
    if global_rng and ck.get("global_rng"):
        torch.set_rng_state(ck["global_rng"]["cpu"])
        if "cuda" in ck["global_rng"] and torch.cuda.is_available():
            torch.cuda.set_rng_state_all(ck["global_rng"]["cuda"])
    return ck.get("extra")

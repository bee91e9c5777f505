"""Replay of the reference trajectories stored in tests/golden/traj_*.npz.

The fixture holds the seeds, the preset codebook and snapshots of the reference
CPU path; the parameter values and per-step gradients are regenerated here with
the integer-exact generator (``tests/golden/param_sets.py``).
"""

from __future__ import annotations

import numpy as np

import param_sets as ps
from golden_util import load

TRAJ_NAMES = ["gpt2mini_f32", "llamamini_bf16", "fp16mini", "groups_f32", "muon_bf16", "muon_f32",
              "tiny_e2e_f32", "llamamini_bf16_f32state"]


def group_options(meta, n_params):
    """Per-parameter hyperparameters exactly as the reference flattens its groups."""
    kw = dict(meta["kwargs"])
    kind = meta["kind"]
    if kind == "muon":
        lr = kw.get("lr", 1e-3)
        base = {"lr": lr, "beta1": kw.get("momentum", 0.95), "beta2": 0.0, "eps": kw.get("eps", 1e-7),
                "weight_decay": kw.get("weight_decay", 0.1)}
        return [dict(base) for _ in range(n_params)]
    base = {"lr": kw.get("lr", 1e-3), "beta1": 0.9, "beta2": 0.999, "eps": kw.get("eps", 1e-8),
            "weight_decay": kw.get("weight_decay", 0.0)}
    opts = [dict(base) for _ in range(n_params)]
    if kind == "gefen_groups":
        for i in (0, 1):
            opts[i].update(lr=3e-3, beta1=0.8, beta2=0.99, weight_decay=0.1)
        for i in range(2, 6):
            opts[i].update(eps=1e-6)
        for i in range(6, n_params):
            opts[i].update(lr=5e-4, weight_decay=0.01)
    return opts


def build(name):
    data, meta = load("traj_" + name)
    pset = getattr(ps, meta["param_set"])
    dtype = meta["dtype"]
    seed = meta["seed"]
    params = []
    for i, (pname, shape, mode) in enumerate(pset):
        params.append({"name": pname, "shape": tuple(shape), "mode": mode,
                       "p0": bits(ps.init_param(seed, i, shape, dtype)), "dtype": dtype})
    opts = group_options(meta, len(params))
    for prm, o in zip(params, opts):
        prm.update(o)
        if meta.get("f_fp32"):
            prm["sdtype"] = "f32"
    skip = {int(k): set(v) for k, v in meta["skip"].items()}
    return data, meta, params, skip


def grads_for(meta, params, step, skip):
    e_lo, e_hi = meta["e_range"]
    out = []
    for i, prm in enumerate(params):
        if i in skip.get(step, ()):
            out.append(None)
        else:
            out.append(bits(ps.grad_for_step(meta["seed"], i, step, prm["shape"], prm["dtype"], prm["mode"],
                                             e_lo, e_hi)))
    return out


def bits(a: np.ndarray) -> np.ndarray:
    """Storage convention of the oracle and the C-ABI: f16 and bf16 as uint16 bits."""
    a = np.asarray(a)
    return a.view(np.uint16) if a.dtype == np.float16 else a


def ulp_distance_bf16(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between two bf16 bit arrays (sign-magnitude aware)."""
    def key(x):
        x = x.astype(np.int32)
        return np.where(x & 0x8000, 0x8000 - (x & 0x7FFF), 0x8000 + (x & 0x7FFF))
    return np.abs(key(np.asarray(a_bits, dtype=np.uint16)) - key(np.asarray(b_bits, dtype=np.uint16)))


def ulp_distance_f16(a_bits, b_bits):
    return ulp_distance_bf16(a_bits, b_bits)

"""Write the golden fixtures of the reference's CPU path (``fused=False``).

Run in the survey container only, where the reference is mounted read-only:

    python tests/golden/make_golden.py [--reference /root/reference] [--only NAME]

The reference package maps ``gefen`` to its repository root, so it is imported
through a temporary directory holding a ``gefen`` symlink.  Only inputs and
outputs are written (``tests/golden/*.npz`` and ``*.json``); nothing from the
reference is copied.  The fixtures pin what no closed form can:

* period choices and divisor scores of ``find_period_by_block_variance``
  (numpy log + pairwise means; ``partitioning.py:119-167, 277-347``), also on
  full-size tensors of the BASELINE configs (``periods_full.npz``);
* the first-step codebook pipeline (torch histogram + exact DP;
  ``gefen.py:305-419``, ``quantization.py:206-258``);
* 20-step trajectories of ``Gefen`` / ``GefenMuon`` on the CPU path
  (``gefen.py:1208-1333``, ``gefen_muon.py:216-329``);
* the ``state_dict`` layout (``gefen.py:1343-1349``);
* every bf16 product of the reference's Newton-Schulz iterations
  (``gefen_muon.py:16-51``, ``ns_products.npz``) and, along the GefenMuon
  trajectories, each step's Newton-Schulz input and output and the parameter
  before and after its update (``gefen_muon.py:302-329``, ``muon_steps_*.npz``).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))
sys.path.insert(0, str(HERE))

from gefen_amd import synthetic as syn  # noqa: E402
import param_sets as ps  # noqa: E402

TORCH_DTYPE = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def import_reference(path: str):
    """Import the reference under its own package name ``gefen`` (its modules import
    each other as ``gefen.*``).  This repository's ``gefen`` package (the import
    surface over ``gefen_amd``) must not answer instead: the reference's directory
    goes first on sys.path, nothing named gefen may be imported yet, and the
    imported package must live under ``path``."""
    if any(name == "gefen" or name.startswith("gefen.") for name in sys.modules):
        raise RuntimeError("a module named gefen is already imported; run this script in a fresh process")
    tmp = tempfile.mkdtemp(prefix="gefen_ref_")
    os.symlink(path, os.path.join(tmp, "gefen"))
    sys.path.insert(0, tmp)
    import gefen  # noqa: F401
    if not os.path.realpath(gefen.__file__).startswith(os.path.realpath(path)):
        raise RuntimeError("imported {} instead of the reference at {}".format(gefen.__file__, path))
    import gefen.gefen as ref_gefen
    import gefen.gefen_muon as ref_muon
    import gefen.partitioning as ref_part
    import gefen.quantization as ref_quant
    return ref_gefen, ref_muon, ref_part, ref_quant


def to_torch(arr: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == "bf16":
        return torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(torch.bfloat16).clone()
    return torch.from_numpy(np.ascontiguousarray(arr)).clone()


def to_numpy(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def dtype_name(t: torch.dtype) -> str:
    return {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[t]


# --------------------------------------------------------------------------- periods
PERIOD_CASES = [
    # name, rows, cols, dtype, mode, e_lo, e_hi
    ("rowscaled_96x768_f32", 96, 768, "f32", "row", -14, -4),
    ("rowscaled_64x1152_bf16", 64, 1152, "bf16", "row", -14, -4),
    ("rowscaled_50x300_f32", 50, 300, "f32", "row", -14, -4),
    ("rowscaled_12x2304_bf16", 12, 2304, "bf16", "row", -14, -4),
    ("rowscaled_8x4096_f32", 8, 4096, "f32", "row", -14, -4),
    ("rowscaled_40x3072_bf16", 40, 3072, "bf16", "row", -14, -4),
    ("rowscaled_200x12_f32", 200, 12, "f32", "row", -14, -4),
    ("iid_4096_f32", 1, 4096, "f32", "row", -7, -7),
    ("iid_64x1000_bf16", 64, 1000, "bf16", "tensor", -9, -9),
    ("colscaled_256x96_f32", 256, 96, "f32", "col", -14, -4),
    ("tiny_48_f32", 1, 48, "f32", "row", -7, -7),
    ("tiny_7_f32", 1, 7, "f32", "row", -7, -7),
    ("prime_1031x3_f32", 3, 1031, "f32", "row", -14, -4),
    ("zeros_1024_f32", 1, 1024, "f32", "zero", 0, 0),
    ("rowscaled_33x1536_f16", 33, 1536, "f16", "row", -12, -4),
]


def period_case_grad(seed: int, i: int, rows: int, cols: int, dtype: str, mode: str, e_lo: int, e_hi: int):
    if mode == "zero":
        g = np.zeros(rows * cols)
    elif mode == "col":
        z = syn.normal(syn.make_key(seed, 77 + i), rows * cols).reshape(rows, cols)
        s = syn.dyadic_scale(syn.make_key(seed, 99 + i), cols, e_lo, e_hi)
        g = (z * s[None, :]).ravel()
    elif mode == "tensor":
        g = syn.row_scaled_normal(seed, 55 + i, 1, rows * cols, e_lo, e_hi).ravel()
    else:
        g = syn.row_scaled_normal(seed, 55 + i, rows, cols, e_lo, e_hi).ravel()
    return syn.round_to(g, dtype)


def make_periods(ref, out: Path) -> None:
    ref_gefen, _, ref_part, _ = ref
    seed = 1234
    data = {}
    manifest = []
    for i, (name, rows, cols, dtype, mode, e_lo, e_hi) in enumerate(PERIOD_CASES):
        g = period_case_grad(seed, i, rows, cols, dtype, mode, e_lo, e_hi)
        grad = to_torch(g, dtype)
        # exactly the CPU branch of Gefen._predict_period_from_grad_sq (gefen.py:812-828)
        period_input = grad.detach().float().square().reshape(-1).cpu().numpy()
        period = ref_part.find_period_by_block_variance(
            period_input, print_results=False, parameter_name=name,
            parameter_shape=(rows, cols), backend="cpu", input_is_squared=True,
            max_period=None)
        n = period_input.size
        divs = [p for p in ref_part.divisors(n) if n // p >= ref_part.DMNB]
        scores = [float(ref_part.average_within_block_variance_cpu(period_input, None, p)) for p in divs]
        data[name + "/grad"] = g
        data[name + "/divisors"] = np.array(divs, dtype=np.int64)
        data[name + "/scores"] = np.array(scores, dtype=np.float64)
        data[name + "/period"] = np.array(period, dtype=np.int64)
        manifest.append({"name": name, "dtype": dtype, "shape": [rows, cols], "mode": mode,
                         "period": int(period), "checksum": syn.checksum(g)})
        print("period", name, period, flush=True)
    np.savez_compressed(out / "periods.npz", **data)
    (out / "periods.json").write_text(json.dumps(manifest, indent=1))


# Full-size tensors of the BASELINE configs, generated as bench.py generates
# them (seed 2026, stream = the tensor's index in bench.py's parameter list):
# (name, bench config, index, shape, dtype, rows of the gradient scale, e_lo, e_hi)
PERIOD_FULL_CASES = [
    ("gpt2_wte_f32", "gpt2", 0, (50257, 768), "f32", 50257, -14, -4),
    ("llama8b_k_proj_bf16", "llama8b", 2, (1024, 4096), "bf16", 1, -17, -7),
    ("llama8b_down_proj_bf16", "llama8b", 7, (4096, 14336), "bf16", 1, -17, -7),
]


def period_full_grad(case):
    name, cfg, index, shape, dtype, rows, e_lo, e_hi = case
    n = int(np.prod(shape))
    return syn.round_to(syn.row_scaled_normal(2026, index, rows, n // rows, e_lo, e_hi), dtype).reshape(-1)


def make_periods_full(ref, out: Path) -> None:
    """Scores of every divisor and the chosen period of full-size config tensors
    (partitioning.py:119-167, 277-347 on the CPU path of gefen.py:812-828).
    Only scores and choices are stored; tests regenerate the inputs."""
    _, _, ref_part, _ = ref
    data = {}
    manifest = []
    for case in PERIOD_FULL_CASES:
        name, cfg, index, shape, dtype = case[:5]
        t0 = time.time()
        g = period_full_grad(case)
        grad = to_torch(g, dtype)
        period_input = grad.detach().float().square().reshape(-1).cpu().numpy()
        period = ref_part.find_period_by_block_variance(
            period_input, print_results=False, parameter_name=name, parameter_shape=shape, backend="cpu",
            input_is_squared=True, max_period=None)
        n = period_input.size
        divs = [p for p in ref_part.divisors(n) if n // p >= ref_part.DMNB]
        scores = [float(ref_part.average_within_block_variance_cpu(period_input, None, p)) for p in divs]
        data[name + "/divisors"] = np.array(divs, dtype=np.int64)
        data[name + "/scores"] = np.array(scores, dtype=np.float64)
        data[name + "/period"] = np.array(period, dtype=np.int64)
        manifest.append({"name": name, "config": cfg, "index": index, "shape": list(shape), "dtype": dtype,
                         "period": int(period), "checksum": syn.checksum(g), "seconds": round(time.time() - t0, 1)})
        print("full period", name, period, flush=True)
    np.savez_compressed(out / "periods_full.npz", **data)
    (out / "periods_full.json").write_text(json.dumps(manifest, indent=1))


# --------------------------------------------------------------------------- DP
def make_dp(ref, out: Path) -> None:
    ref_gefen, _, ref_part, ref_quant = ref
    data = {}
    manifest = []
    rng_seed = 4321

    # (1) the first-step pipeline on a few small tensors (histogram + exact DP)
    pipe_cases = [
        ("pipe_f32", [((16, 24), 24, "f32"), ((40,), 8, "f32"), ((6, 10), 10, "f32")]),
        ("pipe_bf16", [((12, 32), 32, "bf16"), ((64,), 16, "bf16")]),
        ("pipe_small_padded", [((5, 6), 6, "f32")]),
    ]
    for ci, (name, tensors) in enumerate(pipe_cases):
        grad_periods = []
        for ti, (shape, period, dtype) in enumerate(tensors):
            rows = shape[0] if len(shape) > 1 else 1
            cols = int(np.prod(shape)) // rows
            g = syn.round_to(syn.row_scaled_normal(rng_seed, 100 * ci + ti, rows, cols, -14, -4), dtype).reshape(shape)
            data["{}/grad{}".format(name, ti)] = g
            data["{}/period{}".format(name, ti)] = np.array(period, dtype=np.int64)
            t = to_torch(g, dtype)
            grad_periods.append(("t{}".format(ti), t.reshape(-1), period, t))
        t0 = time.time()
        cb = ref_gefen.learn_gefen_exact_codebook_from_grad_periods(
            grad_periods=iter(grad_periods), codebook_device=torch.device("cpu"),
            num_codebooks=256, force_endpoints=True, verbose=False,
            compute_mse_logging=False, use_fused_histogram=True)
        data[name + "/codebook"] = cb.numpy().astype(np.float32)
        manifest.append({"name": name, "kind": "pipeline", "ntensors": len(tensors),
                         "seconds": round(time.time() - t0, 1)})
        print("dp", name, "done in", round(time.time() - t0, 1), "s", flush=True)

    # (2) exact_dp on synthetic histograms (both endpoint modes, several K)
    hist_cases = [
        ("hist_k16_free", 500, 16, False, 1.0),
        ("hist_k64_forced", 700, 64, True, 1.0),
        ("hist_k256_forced", 420, 256, True, 1.0),
        ("hist_k8_forced_big", 300, 8, True, 3.0e7),
        ("hist_k256_padded", 100, 256, True, 1.0),
        ("hist_k4_free_tiny", 9, 4, False, 1.0),
    ]
    for hi, (name, nactive, k, force, mult) in enumerate(hist_cases):
        w = syn.words(syn.make_key(rng_seed, 9000 + hi), 0, 4096 + nactive)
        perm = np.argsort(w[:4096], kind="stable")[:nactive]
        active = np.sort(perm)
        counts = np.zeros(4096, dtype=np.float32)
        vals = (1 + (w[4096:] % np.uint64(1000)).astype(np.float64)) * mult
        counts[active] = vals.astype(np.float32)
        edges = torch.linspace(-1.0, 1.0, steps=4097, dtype=torch.float32)
        centers = 0.5 * (edges[:-1] + edges[1:])
        ct = torch.from_numpy(counts)
        act = ct > 0
        stats = {"bin_edges": edges, "bin_centers": centers, "bin_counts": ct, "active_bins": act,
                 "active_centers": centers[act], "active_counts": ct[act],
                 "active_sums": centers[act] * ct[act]}
        t0 = time.time()
        cb = ref_quant.exact_dp(histogram_stats=stats, num_codebooks=k, force_endpoints=force)
        data[name + "/counts"] = counts
        data[name + "/k"] = np.array(k, dtype=np.int64)
        data[name + "/force"] = np.array(int(force), dtype=np.int64)
        data[name + "/codebook"] = cb.numpy().astype(np.float32)
        manifest.append({"name": name, "kind": "exact_dp", "nactive": nactive, "k": k, "force": force,
                         "seconds": round(time.time() - t0, 1)})
        print("dp", name, "done in", round(time.time() - t0, 1), "s", flush=True)
    np.savez_compressed(out / "exact_dp.npz", **data)
    (out / "exact_dp.json").write_text(json.dumps(manifest, indent=1))


# --------------------------------------------------------------------------- trajectories
TRAJ_CASES = {
    # name: (param set, dtype, optimizer, steps, kwargs, grad e-range, snapshot steps)
    "gpt2mini_f32": ("GPT2_MINI", "f32", "gefen", 20, {}, (-14, -4)),
    "llamamini_bf16": ("LLAMA_MINI", "bf16", "gefen", 20, {}, (-17, -7)),
    "fp16mini": ("FP16_MINI", "f16", "gefen", 20, {"lr": 2e-3, "weight_decay": 0.05}, (-10, -4)),
    "groups_f32": ("GPT2_MINI", "f32", "gefen_groups", 20, {}, (-14, -4)),
    "muon_bf16": ("MUON_MINI", "bf16", "muon", 20, {}, (-10, -10)),
    "muon_f32": ("MUON_MINI", "f32", "muon", 10, {"nesterov": False, "weight_decay": 0.0, "lr": 2e-2}, (-10, -10)),
    "tiny_e2e_f32": ("TINY_E2E", "f32", "gefen_learn", 20, {"weight_decay": 0.1}, (-14, -4)),
    "llamamini_bf16_f32state": ("LLAMA_MINI", "bf16", "gefen", 20, {"weight_decay": 0.01}, (-17, -7)),
}
# trajectories run with the reference's module flag F_FP32 = True (float32
# optimizer state for reduced-precision parameters, gefen.py:53-69)
F_FP32_CASES = {"llamamini_bf16_f32state"}
SNAP_STEPS = (1, 2, 5, 10, 20)
STATE_STEPS = (1, 2, 20)


def _run_traj(opt, params, data, name, seed, steps, skip, dtype, e_lo, e_hi) -> None:
    for step in range(1, steps + 1):
        for i, (pname, t, mode) in enumerate(params):
            if i in skip.get(step, ()):
                t.grad = None
                continue
            g = ps.grad_for_step(seed, i, step, tuple(t.shape), dtype, mode, e_lo, e_hi)
            t.grad = to_torch(g, dtype)
        opt.step()
        if step in SNAP_STEPS:
            for i, (pname, t, _) in enumerate(params):
                data["p{}/step{}".format(i, step)] = to_numpy(t)
        if step in STATE_STEPS:
            for i, (pname, t, _) in enumerate(params):
                st = opt.state[t]
                for key in ("m_codebook", "m_magnitude", "vmean"):
                    if key in st:
                        data["s{}/{}/step{}".format(i, key, step)] = to_numpy(st[key])


def make_traj(ref, out: Path, name: str, codebook: np.ndarray) -> None:
    ref_gefen, ref_muon, _, _ = ref
    set_name, dtype, kind, steps, kwargs, (e_lo, e_hi) = TRAJ_CASES[name]
    pset = getattr(ps, set_name)
    seed = 2024 + sum(map(ord, name))
    params = []
    for i, (pname, shape, mode) in enumerate(pset):
        p0 = ps.init_param(seed, i, shape, dtype)
        t = to_torch(p0, dtype).requires_grad_(True)
        params.append((pname, t, mode))
    data = {"codebook_in": codebook.astype(np.float32)}
    data["meta/seed"] = np.array(seed, dtype=np.int64)
    skip = {}
    if kind == "muon":
        opt = ref_muon.GefenMuon([(n, t) for n, t, _ in params], **kwargs)
    elif kind == "gefen_groups":
        frozen = torch.zeros(3, requires_grad=False)
        groups = [
            {"params": [(params[0][0], params[0][1]), (params[1][0], params[1][1])], "lr": 3e-3,
             "betas": (0.8, 0.99), "weight_decay": 0.1},
            {"params": [t for _, t, _ in params[2:6]] + [frozen], "eps": 1e-6},
            {"params": [(n, t) for n, t, _ in params[6:]], "lr": 5e-4, "weight_decay": 0.01},
        ]
        opt = ref_gefen.Gefen(groups, lr=1e-3)
        skip = {3: {2, 7}, 7: {4}}  # step -> param indices without grad
    else:
        opt = ref_gefen.Gefen([(n, t) for n, t, _ in params], **kwargs)
    if kind != "gefen_learn":
        opt._gefen_codebook = torch.from_numpy(codebook.astype(np.float32)).clone()
    t0 = time.time()
    if name in F_FP32_CASES:
        ref_gefen.F_FP32 = True
    try:
        _run_traj(opt, params, data, name, seed, steps, skip, dtype, e_lo, e_hi)
    finally:
        ref_gefen.F_FP32 = False
    periods = [int(opt.state[t]["automatic_period"]) for _, t, _ in params]
    data["periods"] = np.array(periods, dtype=np.int64)
    data["codebook_out"] = opt._gefen_codebook.numpy().astype(np.float32)
    sd = opt.state_dict()
    layout = {"top_keys": sorted(k for k in sd.keys()),
              "gefen_global_step": int(sd["gefen_global_step"]),
              "param_groups": [{k: (v if not isinstance(v, tuple) else list(v)) for k, v in g.items()}
                               for g in sd["param_groups"]],
              "state": {str(k): {kk: ({"tensor": True, "dtype": str(vv.dtype), "shape": list(vv.shape)}
                                      if torch.is_tensor(vv) else
                                      {"tensor": False, "type": type(vv).__name__,
                                       "value": list(vv) if isinstance(vv, tuple) else vv})
                                 for kk, vv in v.items()} for k, v in sd["state"].items()}}
    np.savez_compressed(out / "traj_{}.npz".format(name), **data)
    (out / "traj_{}.json".format(name)).write_text(json.dumps(
        {"name": name, "param_set": set_name, "dtype": dtype, "kind": kind, "steps": steps,
         "kwargs": kwargs, "e_range": [e_lo, e_hi], "seed": seed, "skip": {str(k): sorted(v) for k, v in skip.items()},
         "f_fp32": name in F_FP32_CASES,
         "periods": periods, "seconds": round(time.time() - t0, 1), "state_dict": layout}, indent=1, default=str))
    print("traj", name, "periods", periods, "in", round(time.time() - t0, 1), "s", flush=True)


# --------------------------------------------------------------------------- Newton-Schulz
# (name, rows, cols, seed stream): the bf16 products of every iteration of
# _zeropower_via_newtonschulz (gefen_muon.py:16-51) on seeded bf16 inputs
NS_CASES = [
    ("ns_256x512", 256, 512, 1),
    ("ns_512x256", 512, 256, 2),
    ("ns_128x384", 128, 384, 3),
]
NS_COEFFS = (3.4445, -4.7750, 2.0315)
NS_STEPS = 5
NS_EPS = 1e-7


class _AddmmSpy:
    """Stands in for the reference module's ``torch``: records the operands and
    result of every torch.addmm call; every other attribute is torch's."""

    def __init__(self):
        self.calls = []

    def addmm(self, inp, mat1, mat2, *, beta=1, alpha=1):
        out = torch.addmm(inp, mat1, mat2, beta=beta, alpha=alpha)
        self.calls.append((inp.clone(), mat1.clone(), mat2.clone(), beta, alpha, out.clone()))
        return out

    def __getattr__(self, name):
        return getattr(torch, name)


def make_ns(ref, out: Path) -> None:
    """Each iteration k of the reference's Newton-Schulz on bf16 input G:
    X_{k-1} (ortho_grad entering the iteration), A_k = X X^T (the operand of the
    first addmm), B_k = addmm(A, A, A, beta=b, alpha=c) and X_k = addmm(X, B, X,
    beta=a); X_0 is the normalised input, and ``out`` the function's result."""
    _, ref_muon, _, _ = ref
    seed = 5150
    data = {}
    manifest = []
    real_torch = ref_muon.torch
    for name, rows, cols, stream in NS_CASES:
        g = syn.round_to(syn.normal(syn.make_key(seed, stream), rows * cols) * 1e-3, "bf16").reshape(rows, cols)
        spy = _AddmmSpy()
        ref_muon.torch = spy
        try:
            res = ref_muon._zeropower_via_newtonschulz(to_torch(g, "bf16"), NS_COEFFS, NS_STEPS, NS_EPS)
        finally:
            ref_muon.torch = real_torch
        calls = spy.calls
        assert len(calls) == 2 * NS_STEPS, len(calls)
        data[name + "/g"] = g
        data[name + "/x0"] = to_numpy(calls[1][2])  # mat2 of the first X update: the normalised X
        for k in range(NS_STEPS):
            gram_in, _, _, beta_b, alpha_c, b_out = calls[2 * k]
            x_in, b_in, x_in2, beta_a, _, x_out = calls[2 * k + 1]
            assert beta_b == NS_COEFFS[1] and alpha_c == NS_COEFFS[2] and beta_a == NS_COEFFS[0]
            assert torch.equal(x_in.view(torch.int16), x_in2.view(torch.int16))
            assert torch.equal(b_in.view(torch.int16), b_out.view(torch.int16))
            data["{}/a{}".format(name, k + 1)] = to_numpy(gram_in)
            data["{}/b{}".format(name, k + 1)] = to_numpy(b_out)
            data["{}/x{}".format(name, k + 1)] = to_numpy(x_out)
            if k > 0:
                assert torch.equal(x_in.view(torch.int16), calls[2 * k - 1][5].view(torch.int16))
        data[name + "/out"] = to_numpy(res)
        manifest.append({"name": name, "shape": [rows, cols], "seed": seed, "stream": stream,
                         "coefficients": list(NS_COEFFS), "steps": NS_STEPS, "eps": NS_EPS,
                         "checksum_g": syn.checksum(g.reshape(-1))})
        print("ns", name, flush=True)
    np.savez_compressed(out / "ns_products.npz", **data)
    (out / "ns_products.json").write_text(json.dumps(manifest, indent=1))


# GefenMuon steps at which the Newton-Schulz input / output and the parameter
# before / after the update are recorded (muon trajectories)
MUON_STEP_CAPTURE = (1, 2, 10)


def make_muon_steps(ref, out: Path, name: str, codebook: np.ndarray) -> None:
    """Replays the GefenMuon trajectory `name` on the reference and records, at
    MUON_STEP_CAPTURE, every tensor's Newton-Schulz input (the Nesterov blend,
    gefen_muon.py:312-316), its output, and the parameter before and after the
    step (gefen_muon.py:318-329)."""
    ref_gefen, ref_muon, _, _ = ref
    set_name, dtype, kind, steps, kwargs, (e_lo, e_hi) = TRAJ_CASES[name]
    assert kind == "muon"
    pset = getattr(ps, set_name)
    seed = 2024 + sum(map(ord, name))
    params = []
    for i, (pname, shape, mode) in enumerate(pset):
        t = to_torch(ps.init_param(seed, i, shape, dtype), dtype).requires_grad_(True)
        params.append((pname, t, mode))
    opt = ref_muon.GefenMuon([(n, t) for n, t, _ in params], **kwargs)
    opt._gefen_codebook = torch.from_numpy(codebook.astype(np.float32)).clone()
    real_ns = ref_muon._zeropower_via_newtonschulz
    seen = []

    def spy(grad, coeffs, ns_steps, eps):
        # the input first: for a bf16 input, grad.bfloat16() is grad itself, which
        # the normalisation then divides in place (gefen_muon.py:33-37)
        ns_in = grad.detach().clone()
        res = real_ns(grad, coeffs, ns_steps, eps)
        seen.append((ns_in, res.detach().clone()))
        return res

    data = {}
    last = max(MUON_STEP_CAPTURE)
    ref_muon._zeropower_via_newtonschulz = spy
    try:
        for step in range(1, last + 1):
            for i, (pname, t, mode) in enumerate(params):
                g = ps.grad_for_step(seed, i, step, tuple(t.shape), dtype, mode, e_lo, e_hi)
                t.grad = to_torch(g, dtype)
            before = [to_numpy(t) for _, t, _ in params]
            seen.clear()
            opt.step()
            assert len(seen) == len(params)
            if step in MUON_STEP_CAPTURE:
                for i, (pname, t, _) in enumerate(params):
                    data["p{}/step{}/before".format(i, step)] = before[i]
                    data["p{}/step{}/after".format(i, step)] = to_numpy(t)
                    data["p{}/step{}/ns_in".format(i, step)] = to_numpy(seen[i][0])
                    data["p{}/step{}/ns_out".format(i, step)] = to_numpy(seen[i][1])
    finally:
        ref_muon._zeropower_via_newtonschulz = real_ns
    np.savez_compressed(out / "muon_steps_{}.npz".format(name), **data)
    (out / "muon_steps_{}.json".format(name)).write_text(json.dumps(
        {"name": name, "steps": list(MUON_STEP_CAPTURE), "ns_in_dtype": "bf16" if dtype == "bf16" else dtype,
         "ns_out_dtype": "bf16"}, indent=1))
    print("muon steps", name, flush=True)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--only", default=None)
    args = ap.parse_args()
    torch.set_num_threads(1)
    ref = import_reference(args.reference)
    out = HERE
    if args.only in (None, "periods"):
        make_periods(ref, out)
    if args.only in (None, "periods_full"):
        make_periods_full(ref, out)
    if args.only in (None, "dp"):
        make_dp(ref, out)
    if args.only in (None, "ns"):
        make_ns(ref, out)
    if args.only in (None, "muon_steps"):
        dp = np.load(out / "exact_dp.npz")
        codebook = dp["hist_k256_forced/codebook"]
        for name in ("muon_bf16", "muon_f32"):
            make_muon_steps(ref, out, name, codebook)
    if args.only is None or args.only.startswith("traj"):
        dp = np.load(out / "exact_dp.npz")
        codebook = dp["hist_k256_forced/codebook"]
        names = list(TRAJ_CASES) if args.only in (None, "traj") else [args.only[len("traj_"):]]
        for name in names:
            make_traj(ref, out, name, codebook)


if __name__ == "__main__":
    main()

"""Gefen optimizer-step benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config llama8b|llama1.5b|gpt2|muon|kernels]

Prints ONE JSON line.  The default workload is BASELINE.json's north star: a
Llama-3-8B-shaped parameter set (291 tensors, 8.03e9 bf16 parameters, bf16
gradients, untied embed / lm_head).  Inputs are synthetic (integer-exact
generator, gefen_amd/synthetic.py) and created in HBM before timing:
parameters ~ N(0, 0.02), gradients ~ N(0, 1) times a per-tensor dyadic
log-uniform scale in [2^-17, 2^-7] (~[7.6e-6, 7.8e-3]; BASELINE.json names
[1e-5, 1e-2]).  Before every step after the first, new gradient values are
written into the same gradient buffers (outside the timed region).

* value / ms_per_step: median wall time of one ``optimizer.step()`` over the
  timed steps (synchronised per step), steady state (steps after the first).
* roofline: algorithmic HBM bytes of one step (p read+write, g read, 8-bit
  index read+write, per-block state read+write with the chosen periods) divided
  by the GPU time of the step's launches inside real ``optimizer.step()`` calls
  (each after a gradient refill), from HIP events the kept step plan records on
  the launch stream right before its first launch and after its last (median
  over a second pass of timed steps).  step_frac: the same bytes divided by
  ms_per_step (host time included).  frac_back_to_back: the launches repeated
  back to back on unchanged gradients.  copy_kernel_gbs: a plain 2 GiB device
  copy (16-byte vectors) timed on the same box, and frac_of_copy the step's
  bandwidth as a fraction of it.  host_ms_per_step: host time of the
  optimizer.step() call; host_ms_plan_run / host_ms_step_tasks: host time of
  the one C call that launches a cached step (gefen_step_plan_run) and of
  gefen_step_tasks, which plans every launch anew (medians over calls issued
  back to back).
* cpu_baseline: the CPU oracle (C restatement of the reference CPU path,
  OpenMP) on a bounded sample of the same tensors, scaled to a full step.
* other_configs (default config only, unless --headline-only): the metric's
  other named shapes, GPT-2 124M (fp32) and Llama-3 1.5B (bf16), and the
  GefenMuon Qwen3-1.7B step, each measured the same way in the same run after
  the 8B tensors are freed (step ms, kernel roofline, and a CPU baseline on a
  smaller time budget).
"""

from __future__ import annotations

import argparse
import ctypes
import gc
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np
import torch

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "optimizer step ms at GPT-2 125M / Llama-1.5B / 8B shapes; % HBM roofline"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA, MI355X
FP64_PEAK_TFLOPS = 78.6  # float64, MI355X (vector and matrix)


def llama_shapes(hidden, layers, q_out, kv_out, inter, vocab):
    shapes = [("embed_tokens", (vocab, hidden))]
    for i in range(layers):
        pre = "layers.{}.".format(i)
        shapes += [(pre + "self_attn.q_proj", (q_out, hidden)), (pre + "self_attn.k_proj", (kv_out, hidden)),
                   (pre + "self_attn.v_proj", (kv_out, hidden)), (pre + "self_attn.o_proj", (hidden, q_out)),
                   (pre + "mlp.gate_proj", (inter, hidden)), (pre + "mlp.up_proj", (inter, hidden)),
                   (pre + "mlp.down_proj", (hidden, inter)), (pre + "input_layernorm", (hidden,)),
                   (pre + "post_attention_layernorm", (hidden,))]
    shapes += [("norm", (hidden,)), ("lm_head", (vocab, hidden))]
    return shapes


def gpt2_shapes():
    shapes = [("wte", (50257, 768)), ("wpe", (1024, 768))]
    for i in range(12):
        pre = "h.{}.".format(i)
        shapes += [(pre + "attn.c_attn.weight", (768, 2304)), (pre + "attn.c_attn.bias", (2304,)),
                   (pre + "attn.c_proj.weight", (768, 768)), (pre + "mlp.c_fc.weight", (768, 3072)),
                   (pre + "mlp.c_proj.weight", (3072, 768)), (pre + "ln_1.weight", (768,)),
                   (pre + "ln_1.bias", (768,)), (pre + "ln_2.weight", (768,)), (pre + "ln_2.bias", (768,))]
    shapes += [("ln_f.weight", (768,))]
    return shapes


def qwen_muon_shapes():
    shapes = []
    for i in range(28):
        pre = "layers.{}.".format(i)
        shapes += [(pre + "q_proj", (2048, 2048)), (pre + "k_proj", (1024, 2048)), (pre + "v_proj", (1024, 2048)),
                   (pre + "o_proj", (2048, 2048)), (pre + "gate_proj", (6144, 2048)), (pre + "up_proj", (6144, 2048)),
                   (pre + "down_proj", (2048, 6144))]
    return shapes


CONFIGS = {
    "llama8b": dict(shapes=lambda: llama_shapes(4096, 32, 4096, 1024, 14336, 128256), dtype=torch.bfloat16,
                    grad="tensor", opt="gefen",
                    workload="Llama-3-8B-shaped Gefen step: 291 tensors, 8.03e9 bf16 params + bf16 grads"),
    "llama1.5b": dict(shapes=lambda: llama_shapes(2048, 16, 2048, 512, 8192, 128256), dtype=torch.bfloat16,
                      grad="tensor", opt="gefen",
                      workload="Llama-3-1.5B-shaped Gefen step: 147 tensors, 1.50e9 bf16 params + bf16 grads"),
    "gpt2": dict(shapes=gpt2_shapes, dtype=torch.float32, grad="row", opt="gefen",
                 workload="GPT-2 124M Gefen step: 111 fp32 tensors, row-scaled grads"),
    "muon": dict(shapes=qwen_muon_shapes, dtype=torch.bfloat16, grad="muon", opt="muon",
                 workload="GefenMuon step on Qwen3-1.7B-shaped 2D matrices (196 tensors, bf16)"),
}
PUBLISHED_MS = {"gpt2": 3.0, "llama1.5b": 29.0}  # README.md:142-145 (hardware not stated)
KERNELS_WORKLOAD = "Isolated kernel workload: one fp32 tensor of 64M elements (8192x8192), 1e-3 * Student-t(3)"


def bench_kernels(args, dev):
    """the first-step kernels on one 64M-element fp32 tensor,
    each timed with HIP events on the launch stream (median of reps)."""
    from gefen_amd import synthetic as syn
    from gefen_amd.gefen import Gefen
    from gefen_amd.kernels.exact_histogram_fused import gefen_exact_histogram_cuda
    from gefen_amd.kernels.lloyd_max_fused import gefen_lloyd_accumulate_cuda, gefen_lloyd_mse_cuda
    from gefen_amd.kernels.period_variance import (average_within_block_variance_cuda_kernel, period_scores_launch,
                                                   period_scores_workspace_bytes)
    from gefen_amd.partitioning import PeriodScorer, candidate_divisors
    from gefen_amd.quantization import exact_dp_from_counts

    n = 8192 * 8192
    g = torch.empty(n, dtype=torch.float32, device=dev)
    syn.fill_device(g, 2026, 2, syn.KIND_STUDENT_T3, mult=1e-3)
    stream = torch.cuda.current_stream()
    reps = max(args.steps, 3)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        ms = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            torch.cuda.synchronize()
            ms.append(e0.elapsed_time(e1))
        return statistics.median(ms)

    divs = candidate_divisors(n)
    ws = torch.empty(period_scores_workspace_bytes(n, divs), dtype=torch.uint8, device=dev)
    sc = torch.empty(len(divs) + 1, dtype=torch.float64, device=dev)
    scorer = PeriodScorer(mode=1)
    scorer.add(g)
    period = scorer.finish()[0]
    hist_period = period
    counts = torch.zeros(4096, dtype=torch.int64, device=dev)
    gefen_exact_histogram_cuda(g, hist_period, counts)
    cb = exact_dp_from_counts(counts.float(), 256, True)
    sums = torch.zeros(256, dtype=torch.float32, device=dev)
    lc = torch.zeros(256, dtype=torch.int64, device=dev)
    m1 = torch.zeros(1, dtype=torch.float32, device=dev)
    m2 = torch.zeros(1, dtype=torch.float32, device=dev)
    vper = period if period > 1 else 256
    nbytes = 4.0 * n
    res = {}
    res["period_scores"] = timed(lambda: period_scores_launch(g, divs, 1, 1e-12, sc, ws))
    res["histogram"] = timed(lambda: gefen_exact_histogram_cuda(g, hist_period, counts))
    res["exact_dp"] = timed(lambda: exact_dp_from_counts(counts.float(), 256, True))
    res["lloyd_accumulate"] = timed(lambda: gefen_lloyd_accumulate_cuda(g, cb, hist_period, sums, lc))
    res["lloyd_mse"] = timed(lambda: gefen_lloyd_mse_cuda(g, cb, cb, hist_period, m1, m2))
    res["block_variance"] = timed(lambda: average_within_block_variance_cuda_kernel(g, vper, input_is_squared=False))

    p = torch.empty(8192, 8192, dtype=torch.float32, device=dev)
    syn.fill_device(p, 2026, 3, syn.KIND_NORMAL, mult=0.02)
    p.requires_grad_(True)
    p.grad = g.view(8192, 8192)

    def first_step():
        opt = Gefen([("w", p)])
        opt.step()

    res["gefen_first_step"] = timed(first_step)
    kernels = {}
    for k, ms in res.items():
        kernels[k] = {"ms": round(ms, 4)}
        if k in ("period_scores", "histogram", "lloyd_accumulate", "lloyd_mse", "block_variance"):
            kernels[k]["read_GB_s"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    pipeline = res["period_scores"] + res["histogram"] + res["exact_dp"]
    # the dominant kernel is the exact DP (quantization.py:158-186): for each of K
    # levels and each end e, every start s is a float64 candidate dp + cost with
    # 7 arithmetic operations (3 prefix differences, a square, a division, two
    # additions); N active bins give sum_c (N-c+1)(N-c+2)/2 candidates
    nact = int((counts > 0).sum().item())
    K = 256
    cands = sum((nact - c + 1) * (nact - c + 2) // 2 for c in range(1, K + 1)) if nact >= K else 0
    dp_flops = 7.0 * cands
    ach = dp_flops / (res["exact_dp"] * 1e-3) / 1e12
    out = {"metric": METRIC, "value": round(pipeline, 4), "unit": "ms", "n_gpus": 1, "steps": reps,
           "warmup": 1, "ms_per_step": round(pipeline, 4), "higher_is_better": False, "scaling": "weak",
           "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": KERNELS_WORKLOAD, "value_is": "period scores (all {} divisors) + histogram + "
                      "exact DP, the codebook pipeline of a first step".format(len(divs)),
                      "period": period, "divisors": len(divs)},
           "kernels": kernels,
           "roofline": {"bound": "mfma", "achieved": round(ach, 3), "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(ach / FP64_PEAK_TFLOPS, 4), "traffic": None,
                        "kernel": "exact DP (k_dp_level): {} active bins, K = {}, {:.3e} float64 candidates".format(
                            nact, K, cands),
                        "note": "compute-bound in float64 on the vector ALU, not MFMA: the peak is MI355X's fp64 "
                                "figure (78.6 TFLOP/s, vector and matrix alike); a division counts as one "
                                "operation though the IEEE float64 quotient takes about 11 instructions; the "
                                "operands sit in LDS, so HBM traffic is negligible",
                        "algorithmic_flops": dp_flops}}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_kernels(g.cpu().numpy(), divs)
    print(json.dumps(out), flush=True)



def fill_grad(cfg, g, index, step=0, seed=2026):
    """Gradient `index` of the config for `step` (0: the gradient of the first step,
    stream = index; later steps use streams step * 100000 + index), in place:
    "row": N(0,1) times a dyadic log-uniform scale per row in [2^-14, 2^-4] (GPT-2,
    ~[6e-5, 6e-2]); "tensor": one scale per tensor in [2^-17, 2^-7] (~[7.6e-6, 7.8e-3]);
    "muon": N(0, 1e-3) (2^-10 ~ 0.98e-3)."""
    from gefen_amd import synthetic as syn

    stream = index if step == 0 else step * 100_000 + index
    n = g.numel()
    if cfg["grad"] == "row":
        cols = g.shape[-1] if g.dim() > 1 else n
        syn.fill_device(g, seed, stream, syn.KIND_ROW_SCALED, cols=cols, e_lo=-14, e_hi=-4)
    elif cfg["grad"] == "muon":
        syn.fill_device(g, seed, stream, syn.KIND_ROW_SCALED, cols=n, e_lo=-10, e_hi=-10)
    else:
        syn.fill_device(g, seed, stream, syn.KIND_ROW_SCALED, cols=n, e_lo=-17, e_hi=-7)


def build_problem(cfg, dev, seed=2026):
    from gefen_amd import synthetic as syn

    params = []
    for i, (name, shape) in enumerate(cfg["shapes"]()):
        p = torch.empty(shape, dtype=cfg["dtype"], device=dev)
        syn.fill_device(p, seed, 1_000_000 + i, syn.KIND_NORMAL, mult=0.02)
        g = torch.empty(shape, dtype=cfg["dtype"], device=dev)
        fill_grad(cfg, g, i, 0, seed)
        p.requires_grad_(True)
        p.grad = g
        params.append((name, p))
    torch.cuda.synchronize()
    return params


def step_bytes(opt, params):
    """Algorithmic HBM bytes of one steady-state step with the chosen periods."""
    total = 0
    for _, p in params:
        st = opt.state[p]
        n = p.numel()
        sd = p.element_size()
        ss = st["m_magnitude"].element_size()
        P = st["automatic_period"]
        if P > 1:
            total += n * (3 * sd + 2) + (n // P) * 2 * (ss + ss)
        else:
            d = st["period_one_divisor"]
            total += n * (3 * sd + 2 + 2 * ss) + (n // d) * 2 * ss
    return total


STEP_KERNEL_SOURCES = ("gefen_amd/csrc/step_kernels.h", "gefen_amd/csrc/common.h")


def step_kernel_sources_sha256():
    """sha256 of the step kernels' sources: a traffic record applies only to the
    kernels it was measured on."""
    import hashlib

    h = hashlib.sha256()
    for rel in STEP_KERNEL_SOURCES:
        h.update(rel.encode())
        h.update((REPO / rel).read_bytes())
    return h.hexdigest()


def measured_traffic(cfg, nbytes):
    """HBM bytes per step of the k_gefen_step launches from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (scaled by a copy kernel of known
    size), when they were taken on this workload with the same algorithmic bytes
    and the same kernel sources (else None: a stale record is never reported)."""
    path = REPO / "profiles" / "k_gefen_step_llama8b_traffic.json"
    if not path.exists():
        return None
    rec = json.loads(path.read_text())
    if rec.get("workload") != cfg["workload"] or rec.get("algorithmic_bytes_per_step") != int(nbytes):
        return None
    if rec.get("sources_sha256") != step_kernel_sources_sha256():
        return None
    return rec["traffic_bytes_per_step"]


def kernel_tasks(opt, params):
    """The task array the optimizer passes to gefen_step_tasks (for direct timing)."""
    from gefen_amd import _lib

    tasks = np.zeros(len(params), dtype=_lib.STEP_TASK)
    for i, (_, p) in enumerate(params):
        st = opt.state[p]
        g = opt.param_groups[i]
        t = tasks[i]
        t["p"], t["grad"] = p.data_ptr(), p.grad.data_ptr()
        t["m_codebook"], t["m_magnitude"], t["vmean"] = (st["m_codebook"].data_ptr(), st["m_magnitude"].data_ptr(),
                                                         st["vmean"].data_ptr())
        t["numel"], t["period"] = p.numel(), st["automatic_period"]
        t["period_one_divisor"] = st.get("period_one_divisor", 0) if st["automatic_period"] == 1 else 0
        code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
        t["param_dtype"] = code[p.dtype]
        t["state_dtype"] = code[st["m_magnitude"].dtype]
        t["beta1"], t["beta2"], t["lr"], t["eps"], t["weight_decay"] = (g["beta1"], g["beta2"], g["lr"], g["eps"],
                                                                         g["weight_decay"])
        t["bias_correction_1"] = 1 - g["beta1"] ** (st["step"] + 1)
        t["bias_correction_2"] = 1 - g["beta2"] ** (st["step"] + 1)
    return tasks


def muon_ns_roofline(opt, params, reps=3):
    """Newton-Schulz of one GefenMuon step (the batched stacks the optimizer builds,
    on bf16 inputs of the same shapes) timed with HIP events on the launch stream.
    Algorithmic flops per matrix and iteration: 2 (m^2 n + m^3 + m^2 n), m = min
    dim, n = max dim (X X^T, A A, B X), as the reference computes them."""
    from gefen_amd.newton_schulz import batched_shape_ok, newton_schulz_batched

    groups = {}
    for _, p in params:
        rows, cols = p.shape
        if batched_shape_ok(rows, cols):
            groups[(rows, cols)] = groups.get((rows, cols), 0) + 1
    g0 = opt.param_groups[0]
    coeffs, steps, eps = tuple(g0["ns_coefficients"]), g0["ns_steps"], g0["eps"]
    dev = params[0][1].device
    stacks = {k: (torch.randn(n, k[0], k[1], device=dev) * 1e-3).bfloat16() for k, n in groups.items()}
    # the matrices' sums of squares, which the optimizer's momentum kernels gather
    # while writing the stacks (computed here once, outside the timed region)
    sums = {k: torch.nn.functional.pad((x.double() ** 2).sum(dim=(1, 2))[:, None], (0, 127)).reshape(-1)
            for k, x in stacks.items()}  # laid out as GEFEN_SUMSQ_STRIDE (128) entries per matrix
    flops = 0.0
    for (rows, cols), n in groups.items():
        m, nn = min(rows, cols), max(rows, cols)
        flops += n * steps * 2.0 * (m * m * nn + m * m * m + m * m * nn)
    stream = torch.cuda.current_stream()

    def run():  # x is renormalised in place each time: the same work every call
        for k, x in stacks.items():
            newton_schulz_batched(x, coeffs, steps, eps, sumsq=sums[k])

    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    achieved = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
            "kernel_ms_per_step": round(ms, 3), "algorithmic_flops_per_step": flops,
            "note": "Newton-Schulz of every stack of one step, normalisation included"}


def copy_ceiling_gbs(dev, nbytes=1 << 31, reps=5):
    """HBM bandwidth of a plain 16-byte-vector copy kernel on this box (bytes read +
    written per second, HIP events on the launch stream): the ceiling the step
    kernels' streaming traffic is also compared against."""
    from gefen_amd import synthetic as syn

    src = torch.ones(nbytes // 2, dtype=torch.int16, device=dev)
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream()
    syn.copy_device(src, dst)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        syn.copy_device(src, dst)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    torch.cuda.empty_cache()
    return 2.0 * nbytes / (ms * 1e-3) / 1e9


def cpu_baseline(opt, params, budget_s=20.0):
    """Oracle (reference CPU path restated in C, OpenMP over blocks) on a sample
    of the tensors, scaled by bytes to one full step."""
    from oracle import oracle as orc

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    cb = opt._gefen_codebook.detach().cpu().numpy().astype(np.float32)
    # a contiguous run of transformer tensors (the embedding first in the list is skipped)
    sample, sample_elems = [], 0
    target = 60_000_000  # elements in the sample
    for i in range(1, len(params)):
        sample.append(i)
        sample_elems += params[i][1].numel()
        if sample_elems >= target:
            break
    host = []
    for i in sample:
        _, p = params[i]
        st = opt.state[p]
        conv = (lambda t: t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
                if t.dtype != torch.float32 else t.detach().contiguous().cpu().numpy().reshape(-1))
        host.append((i, conv(p), conv(p.grad), st["m_codebook"].cpu().numpy().reshape(-1).copy(),
                     conv(st["m_magnitude"]), conv(st["vmean"])))
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

    def one_rep(threads):
        t0 = time.perf_counter()
        for i, pp, gg, idx, mag, vm in host:
            _, p = params[i]
            st = opt.state[p]
            g = opt.param_groups[i]
            P = st["automatic_period"]
            rc = orc.lib().orc_gefen_step(code[p.dtype], code[st["m_magnitude"].dtype], orc._ptr(pp), orc._ptr(gg),
                                          orc._ptr(idx), orc._ptr(mag), orc._ptr(vm), p.numel(), P,
                                          st.get("period_one_divisor", 0) if P == 1 else 0, orc._ptr(cb), cb.size,
                                          g["beta1"], g["beta2"], g["lr"], g["eps"], g["weight_decay"], 0.5, 0.5,
                                          threads)
            assert rc == 0
        return time.perf_counter() - t0

    reps, elapsed = 0, 0.0
    while elapsed < budget_s / 2 and reps < 50:
        elapsed += one_rep(cores)
        reps += 1
    per_rep = elapsed / reps
    single = one_rep(1)  # the same sample once on one core
    full = sum(p.numel() for _, p in params)
    scale = 1000.0 * full / sample_elems
    return {"value": round(per_rep * scale, 1), "unit": "ms per full step (scaled by elements)", "cores": cores,
            "kind": "port", "single_core_value": round(single * scale, 1),
            "sample": "{} consecutive tensors after the first, {:.3g} elements, {} repetitions of the oracle step "
                      "(OpenMP over blocks; one more on one core for single_core_value), scaled to {:.3g} "
                      "elements".format(len(sample), sample_elems, reps, full)}


def cpu_baseline_muon(opt, params, budget_s=20.0):
    """The GefenMuon step of the reference's CPU path on one matrix of each shape,
    scaled by Newton-Schulz flops to one full step: quantised momentum and the
    Nesterov blend from the oracle (C), Newton-Schulz as the reference computes it
    on the CPU (gefen_muon.py:16-51: torch bf16 tensors, X @ X.T and two addmm
    per iteration, each product accumulated in float32 by torch's CPU GEMM and
    rounded to bf16, on torch's intra-op threads), the parameter update from the
    oracle (gefen_muon.py:325-329)."""
    from oracle import oracle as orc

    threads = torch.get_num_threads()
    cb = opt._gefen_codebook.detach().cpu().numpy().astype(np.float32)
    g0 = opt.param_groups[0]
    (a, b, c), steps, eps = tuple(g0["ns_coefficients"]), g0["ns_steps"], g0["eps"]

    def ns_flops(shape):
        m, n = min(shape), max(shape)
        return steps * 2.0 * (m * m * n + m * m * m + m * m * n)

    def newton_schulz_cpu(u_bits, shape):
        x = torch.from_numpy(u_bits.view(np.int16).reshape(shape)).view(torch.bfloat16)
        if shape[0] > shape[1]:
            x = x.T
        x = x / x.norm().clamp(min=eps)
        for _ in range(steps):
            am = x @ x.T
            bm = torch.addmm(am, am, am, beta=b, alpha=c)
            x = torch.addmm(x, bm, x, beta=a)
        if shape[0] > shape[1]:
            x = x.T
        return x.contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)

    sample, seen = [], set()
    for i, (_, p) in enumerate(params):
        if tuple(p.shape) not in seen:
            seen.add(tuple(p.shape))
            sample.append(i)
    host = []
    for i in sample:
        _, p = params[i]
        st = opt.state[p]
        conv = (lambda t: t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1))
        tstate = orc.TensorState(p.numel(), st["automatic_period"], "bf16", "bf16")
        tstate.m_codebook = st["m_codebook"].cpu().numpy().reshape(-1).copy()
        tstate.m_magnitude = conv(st["m_magnitude"]).copy()
        tstate.pod = st.get("period_one_divisor")
        host.append((i, conv(p).copy(), conv(p.grad).copy(), tstate))
    reps, elapsed = 0, 0.0
    while elapsed < budget_s and reps < 5:
        t0 = time.perf_counter()
        for i, pp, gg, tstate in host:
            shape = tuple(params[i][1].shape)
            blend = orc.muon_momentum(gg, "bf16", tstate, cb, g0["momentum"], g0["nesterov"])
            u = newton_schulz_cpu(blend, shape)
            orc.muon_apply(pp, u, "bf16", shape, g0["lr"], g0["weight_decay"],
                           orc.adjust_lr(g0["lr"], g0["adjust_lr_fn"], shape))
        elapsed += time.perf_counter() - t0
        reps += 1
    per_rep = elapsed / reps
    scale = sum(ns_flops(tuple(p.shape)) for _, p in params) / sum(ns_flops(tuple(params[i][1].shape))
                                                                    for i in sample)
    return {"value": round(per_rep * scale * 1000.0, 1), "unit": "ms per full step (scaled by Newton-Schulz flops)",
            "cores": threads, "kind": "port",
            "sample": "one matrix of each shape ({}), {} repetitions of the reference CPU path's GefenMuon step "
                      "(Newton-Schulz as torch bf16 CPU products on {} intra-op threads, momentum and update from "
                      "the C oracle), scaled by Newton-Schulz flops to all {} matrices".format(
                          ", ".join("{}x{}".format(*params[i][1].shape) for i in sample), reps, threads,
                          len(params))}


def cpu_baseline_kernels(g_host, period_divs):
    """The same first-step codebook pipeline (period scores of every divisor,
    histogram, exact DP) on the same 64M-element tensor with the oracle (C,
    OpenMP for scores and histogram, one thread for the DP)."""
    from oracle import oracle as orc

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    t0 = time.perf_counter()
    sc = orc.period_scores(g_host, "f32", period_divs, mode=1)
    period = orc.finalize_period(list(zip(period_divs, sc.tolist())), g_host.size)
    t1 = time.perf_counter()
    counts = orc.histogram(g_host, "f32", period)
    t2 = time.perf_counter()
    orc.exact_dp(counts.astype(np.float32), 256, True)
    t3 = time.perf_counter()
    return {"value": round((t3 - t0) * 1000.0, 1), "unit": "ms (period scores + histogram + exact DP)",
            "cores": cores, "kind": "port",
            "sample": "the whole 64M-element tensor: scores {:.0f} ms, histogram {:.0f} ms, DP {:.0f} ms (one "
                      "thread)".format((t1 - t0) * 1e3, (t2 - t1) * 1e3, (t3 - t2) * 1e3)}


def measure(name, args, dev, with_cpu, copy_gbs=None, cpu_budget_s=20.0):
    """One config's JSON object: median step() latency over args.steps timed steps
    after args.warmup untimed ones (new gradients before every step), the
    kernel roofline, and (with_cpu) the CPU baseline."""
    cfg = CONFIGS[name]
    from gefen_amd.gefen import Gefen
    from gefen_amd.gefen_muon import GefenMuon
    from gefen_amd import _lib

    params = build_problem(cfg, dev)

    def set_grads(k):
        """The gradients of step k + 1, written into the same gradient buffers before
        the step (outside the timed region): every step sees new values at the
        addresses a training loop's caching allocator typically hands back."""
        for i, (_, p) in enumerate(params):
            fill_grad(cfg, p.grad, i, k)
        torch.cuda.synchronize()

    Opt = GefenMuon if cfg["opt"] == "muon" else Gefen
    opt = Opt(params)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    opt.step()
    torch.cuda.synchronize()
    first_ms = (time.perf_counter() - t0) * 1000.0
    step_no = 1
    for _ in range(args.warmup):
        set_grads(step_no)
        step_no += 1
        opt.step()
    torch.cuda.synchronize()
    times = []
    for _ in range(args.steps):
        set_grads(step_no)
        step_no += 1
        t0 = time.perf_counter()
        opt.step()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1000.0)
    med = statistics.median(times)
    q = np.percentile(times, [10, 90]).tolist()
    out = {"metric": METRIC, "value": round(med, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(med, 4), "higher_is_better": False, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16" if cfg["dtype"] == torch.bfloat16 else "f32", "data": "synthetic",
           "config": {"workload": cfg["workload"], "tensors": len(params),
                      "params": int(sum(p.numel() for _, p in params))},
           "p10_ms": round(q[0], 4), "p90_ms": round(q[1], 4), "first_step_ms": round(first_ms, 1)}
    if name in PUBLISHED_MS:
        out["vs_baseline"] = round(PUBLISHED_MS[name] / med, 3)
    periods = {}
    for _, p in params:
        P = opt.state[p]["automatic_period"]
        periods[P] = periods.get(P, 0) + 1
    out["config"]["periods"] = {str(k): v for k, v in sorted(periods.items())}
    if cfg["opt"] == "gefen":
        lib = _lib.load()
        # the step's launches timed inside real optimizer.step() calls (each after a
        # gradient refill, like the timed steps): the kept plan records HIP events on
        # the launch stream right before its first launch and after its last
        # (a second pass, so that the timed steps above carry no event records)
        plan = opt._plan
        if plan is None or not plan.handle:
            raise RuntimeError("the optimizer did not keep a step plan")
        _lib.check(lib.gefen_step_plan_time_runs(plan.handle, 1))
        in_step, host, outside = [], [], []
        cur = torch.cuda.current_stream()
        for _ in range(args.steps):
            set_grads(step_no)
            step_no += 1
            # also: the host time of the step() call, and the GPU time between an
            # event recorded right before the call and one recorded right after it
            # that the step's launches do not cover (the host's work before the
            # first launch reaches the GPU, and the join of the side stream)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(cur)
            t0 = time.perf_counter()
            opt.step()
            t1 = time.perf_counter()
            e1.record(cur)
            if opt._plan is not plan:
                raise RuntimeError("the step plan was rebuilt during the timed steps")
            torch.cuda.synchronize()
            ms = ctypes.c_float()
            _lib.check(lib.gefen_step_plan_last_ms(plan.handle, ctypes.byref(ms)))
            in_step.append(ms.value)
            host.append((t1 - t0) * 1000.0)
            outside.append(e0.elapsed_time(e1) - ms.value)
        _lib.check(lib.gefen_step_plan_time_runs(plan.handle, 0))
        kms = statistics.median(in_step)
        # the same launches back to back on unchanged gradients (the kernels' own
        # rate at the shader clock of a busy GPU; not the reported figure)
        tasks = kernel_tasks(opt, [(n, p) for n, p in params])
        tables = opt._codebook_tables()
        stream = torch.cuda.current_stream()
        for _ in range(2):
            _lib.check(lib.gefen_step_tasks(tasks.ctypes.data, len(params), tables.data_ptr(), stream.cuda_stream))
        reps = max(args.steps, 5)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        host_tasks = []
        e0.record(stream)
        for _ in range(reps):
            t0 = time.perf_counter()
            rc = lib.gefen_step_tasks(tasks.ctypes.data, len(params), tables.data_ptr(), stream.cuda_stream)
            host_tasks.append((time.perf_counter() - t0) * 1000.0)
            _lib.check(rc)
        e1.record(stream)
        torch.cuda.synchronize()
        kms_b2b = e0.elapsed_time(e1) / reps
        # host time of the C call that launches a cached step (gefen_step_plan_run on
        # the plan's table as the last step refreshed it), beside that of
        # gefen_step_tasks above, which plans every launch anew: each call timed
        # alone on the host, issued back to back
        host_run = []
        for _ in range(reps):
            t0 = time.perf_counter()
            rc = lib.gefen_step_plan_run(plan.handle, plan.tptr, len(plan.tasks), stream.cuda_stream)
            host_run.append((time.perf_counter() - t0) * 1000.0)
            _lib.check(rc)
        torch.cuda.synchronize()
        nbytes = step_bytes(opt, params)
        achieved = nbytes / (kms * 1e-3) / 1e9
        if copy_gbs is None:
            copy_gbs = copy_ceiling_gbs(dev)
        out["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(cfg, nbytes),
                           "kernel_ms_per_step": round(kms, 4), "algorithmic_bytes_per_step": int(nbytes),
                           "step_frac": round(nbytes / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "kernel_ms_back_to_back": round(kms_b2b, 4),
                           "frac_back_to_back": round(nbytes / (kms_b2b * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "copy_kernel_gbs": round(copy_gbs, 1), "frac_of_copy": round(achieved / copy_gbs, 4),
                           "host_ms_per_step": round(statistics.median(host), 4),
                           "gpu_ms_outside_launches": round(statistics.median(outside), 4),
                           "host_ms_plan_run": round(statistics.median(host_run), 4),
                           "host_ms_step_tasks": round(statistics.median(host_tasks), 4)}
        if with_cpu:
            out["cpu_baseline"] = cpu_baseline(opt, params, budget_s=cpu_budget_s)
    else:
        out["roofline"] = muon_ns_roofline(opt, params)
        if with_cpu:
            out["cpu_baseline"] = cpu_baseline_muon(opt, params, budget_s=cpu_budget_s)
    return out


def compact(out):
    """The figures of a further config's line that the headline line carries."""
    r = out["roofline"]
    keep = ("bound", "achieved", "peak", "unit", "frac", "kernel_ms_per_step", "step_frac", "frac_back_to_back",
            "frac_of_copy", "host_ms_per_step", "gpu_ms_outside_launches", "host_ms_plan_run", "host_ms_step_tasks")
    return {"workload": out["config"]["workload"], "ms_per_step": out["value"], "p10_ms": out["p10_ms"],
            "p90_ms": out["p90_ms"], "first_step_ms": out["first_step_ms"], "dtype": out["dtype"],
            "vs_readme": out["vs_baseline"], "periods": out["config"]["periods"],
            "roofline": {k: r[k] for k in keep if k in r}, "cpu_baseline": out.get("cpu_baseline")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="llama8b", choices=sorted(CONFIGS) + ["kernels"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--headline-only", action="store_true",
                    help="with the default config, skip the GPT-2, Llama-1.5B and GefenMuon lines that the "
                         "headline line otherwise carries under other_configs")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also copy 2 GiB once with k_copy16 (a kernel of known traffic for scaling HBM counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the step would shard by partition "
              "block, with no communication between GPUs). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    if args.config == "kernels":
        bench_kernels(args, dev)
        return
    if args.copy_probe:
        from gefen_amd import synthetic as syn

        src = torch.ones(1 << 30, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        syn.copy_device(src, dst)  # k_copy16: 2 GiB read + 2 GiB written
        torch.cuda.synchronize()
        del src, dst
    out = measure(args.config, args, dev, not args.no_cpu_baseline)
    if args.config == "llama8b" and not args.headline_only:
        # the metric's other named shapes (and GefenMuon), each measured the same
        # way after the headline's tensors are freed; value stays the 8B step
        others = {}
        for name in ("gpt2", "llama1.5b", "muon"):
            gc.collect()
            torch.cuda.empty_cache()
            try:
                others[name] = compact(measure(name, args, dev, not args.no_cpu_baseline,
                                               out["roofline"].get("copy_kernel_gbs"), cpu_budget_s=5.0))
            except Exception as e:  # the headline line is printed regardless
                others[name] = {"error": repr(e)[:300]}
        out["other_configs"] = others
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

"""GefenMuon on MI355X (reference: gefen_muon.py, ndvbd/Gefen 1.2.3).

Muon with Gefen's 8-bit quantised momentum.  Per step, one batched HIP launch
updates the quantised momentum of every tensor and writes the Nesterov blend
(gefen_muon.py:302-316, CPU-path rounding); Newton-Schulz orthogonalisation
(gefen_muon.py:16-51) runs batched over same-shaped matrices on MFMA; the
parameter update is one batched launch with the reference's CPU arithmetic
(gefen_muon.py:325-329).
"""

from __future__ import annotations

import math
from typing import Iterable, Optional, Tuple, Union

import numpy as np
import torch
import torch.nn as nn

from gefen_amd import _lib
from gefen_amd.gefen import (Gefen, _DTYPE_CODE, _distinct, _gefen_host, _plan_checks_python, _step_entry,
                             _kernel_weight_decay, automatic_partition_view)

EPS = 1e-7
_SUMSQ_STRIDE = 128  # GEFEN_SUMSQ_STRIDE (include/gefen_hip.h): sum-of-squares entries per momentum task
DEFAULT_A = 3.4445
DEFAULT_B = -4.7750
DEFAULT_C = 2.0315
DEFAULT_NS_STEPS = 5


def _check_ns_args(ns_coefficients, ns_steps: int) -> None:
    """The argument checks of gefen_muon.py:23-30."""
    if ns_steps >= 100:
        raise ValueError("Number of steps must be less than 100 for computational efficiency")
    if len(ns_coefficients) != 3:
        raise ValueError("Coefficients must be a tuple of exactly 3 values")


def _zeropower_via_newtonschulz(grad: torch.Tensor, ns_coefficients: Tuple[float, float, float], ns_steps: int,
                                eps: float) -> torch.Tensor:
    """Quintic Newton-Schulz iteration in bf16 (gefen_muon.py:16-51)."""
    if ns_steps >= 100:
        raise ValueError("Number of steps must be less than 100 for computational efficiency")
    if len(grad.shape) != 2:
        raise ValueError("Input tensor gradient must be a 2D matrix")
    if len(ns_coefficients) != 3:
        raise ValueError("Coefficients must be a tuple of exactly 3 values")
    from gefen_amd.newton_schulz import newton_schulz_bf16

    return newton_schulz_bf16(grad, ns_coefficients, ns_steps, eps)


def _adjust_lr(lr: float, adjust_lr_fn: Optional[str], param_shape: torch.Size) -> float:
    """gefen_muon.py:54-67."""
    if isinstance(lr, torch.Tensor):
        lr = lr.item()
    rows, cols = param_shape[:2]
    if adjust_lr_fn is None or adjust_lr_fn == "original":
        ratio = math.sqrt(max(1, rows / cols))
    elif adjust_lr_fn == "match_rms_adamw":
        ratio = 0.2 * math.sqrt(max(rows, cols))
    else:
        ratio = 1.0
    return lr * ratio


class GefenMuon(Gefen):
    """GefenMuon (gefen_muon.py:70-350)."""

    def __init__(self, params: Iterable[Union[nn.Parameter, Tuple[str, nn.Parameter]]],
                 lr: Union[float, torch.Tensor] = 1e-3, weight_decay: float = 0.1, momentum: float = 0.95,
                 nesterov: bool = True,
                 ns_coefficients: Tuple[float, float, float] = (DEFAULT_A, DEFAULT_B, DEFAULT_C), eps: float = EPS,
                 ns_steps: int = DEFAULT_NS_STEPS, adjust_lr_fn: Optional[str] = None, *, fused: bool = True,
                 verbose: bool = False) -> None:
        if isinstance(lr, torch.Tensor) and lr.numel() != 1:
            raise ValueError("Tensor lr must be 1-element")
        if not 0.0 <= lr:
            raise ValueError("Learning rate should be >= 0 but is: {}".format(lr))
        if not 0.0 <= momentum:
            raise ValueError("momentum should be >= 0 but is: {}".format(momentum))
        if not 0.0 <= weight_decay:
            raise ValueError("weight decay should be >= 0 but is: {}".format(weight_decay))
        if adjust_lr_fn is not None and adjust_lr_fn not in ["original", "match_rms_adamw"]:
            raise ValueError("Adjust learning rate function {} is not supported".format(adjust_lr_fn))
        super().__init__(params, lr=lr, betas=(momentum, 0.0), eps=eps, weight_decay=weight_decay, fused=fused,
                         verbose=verbose)
        for group in self.param_groups:
            group["momentum"] = momentum
            group["nesterov"] = nesterov
            group["ns_coefficients"] = ns_coefficients
            group["ns_steps"] = ns_steps
            group["adjust_lr_fn"] = adjust_lr_fn
            for p in group["params"]:
                if p.ndim != 2:
                    raise ValueError("GefenMuon only supports 2D parameters whereas we found a parameter with size: "
                                     "{}".format(p.size()))

    def _init_gefen_muon_state(self, state, grad_view: torch.Tensor) -> None:
        self._init_gefen_state(state, grad_view)

    def _init_states(self, pending) -> None:
        need = [(p, grad) for (group, p, local_p, grad) in pending
                if "automatic_period" not in self.state[p] and grad.numel() > 1]
        periods = self._predict_periods(need) if need else []
        for (p, _), period in zip(need, periods):
            self.state[p]["automatic_period"] = period
        for group, p, local_p, grad in pending:
            st = self.state[p]
            n = grad.numel()
            if "automatic_period" not in st:
                st["automatic_period"] = 1
            period = st["automatic_period"]
            if n % period != 0:
                raise ValueError("Automatic partition period {} does not divide local shard of parameter {} with "
                                 "numel {}".format(period, group["name"], n))
            st["step"] = 0
            self._init_gefen_muon_state(st, automatic_partition_view(grad.reshape(-1), period))
            self._print_period(group["name"], local_p, period)

    def _step_all(self) -> None:
        """Quantised momentum, Newton-Schulz and the parameter update of every
        tensor.  While the same parameters carry gradients of the same layout and
        the state tensors and Newton-Schulz settings are unchanged, a cached plan
        (_MuonPlan) reuses the task tables and stacked buffers and only refreshes
        gradient addresses, step counts and hyperparameters."""
        plan = self._plan
        if plan is not None and plan.refresh(self):
            plan.run(self)
            return
        self._plan = None
        self._step_all_build()

    def _step_all_build(self) -> None:
        items = []
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                name = group["name"]
                local_p = self._resolve_local_tensor(p, "parameter {}".format(name))
                grad = self._resolve_local_tensor(p.grad, "gradient {}".format(name))
                if torch.is_complex(local_p):
                    raise RuntimeError("GefenMuon does not support complex parameters")
                if grad.is_sparse:
                    raise RuntimeError("GefenMuon does not support sparse gradients")
                if grad.ndim != 2:
                    raise ValueError("GefenMuon gradient must be a 2D matrix for {}".format(name))
                if local_p.numel() != grad.numel():
                    raise ValueError("Local parameter shard numel {} does not match local gradient numel {} for {}."
                                     .format(local_p.numel(), grad.numel(), name))
                if grad.numel() == 0:
                    continue
                if grad.device.type != "cuda":
                    raise RuntimeError("gefen_amd runs on HIP devices; {} is on {}".format(name, grad.device))
                items.append((group, p, local_p, grad))
        if not items:
            return
        fresh = [it for it in items if "step" not in self.state[it[1]]]
        if fresh:
            self._init_states(fresh)
        if self._gefen_codebook is None:
            raise ValueError("Expected Gefen codebook to be initialized before fused GefenMuon update.")
        tables = self._codebook_tables()
        tasks = np.zeros(len(items), dtype=_lib.MUON_TASK)
        # Matrices of one shape, dtype and Newton-Schulz setting share a stacked
        # buffer: the momentum kernel writes each one's Nesterov blend into its
        # slice and Newton-Schulz runs on the whole stack.
        from gefen_amd.newton_schulz import batched_shape_ok

        stacks = {}
        for i, (group, p, local_p, grad) in enumerate(items):
            rows, cols = grad.shape
            if batched_shape_ok(rows, cols):
                key = (rows, cols, grad.dtype, tuple(group["ns_coefficients"]), group["ns_steps"], group["eps"])
                stacks.setdefault(key, []).append(i)
        where = {}
        bufs = {}
        for key, idx in stacks.items():
            rows, cols, dtype = key[0], key[1], key[2]
            bufs[key] = torch.empty(len(idx), rows, cols, dtype=dtype, device=items[idx[0]][3].device)
            for slot, i in enumerate(idx):
                where[i] = (key, slot)
        outs = []
        keep = []
        for i, (group, p, local_p, grad) in enumerate(items):
            st = self.state[p]
            period = st["automatic_period"]
            flat = grad.reshape(-1)
            if not flat.is_contiguous():
                flat = flat.contiguous()
            keep.append(flat)
            if i in where:
                key, slot = where[i]
                out = bufs[key][slot].view(-1)
            else:
                out = torch.empty_like(flat)
            outs.append(out)
            t = tasks[i]
            t["grad"] = flat.data_ptr()
            t["m_codebook"] = st["m_codebook"].data_ptr()
            t["m_magnitude"] = st["m_magnitude"].data_ptr()
            t["out"] = out.data_ptr()
            t["numel"] = flat.numel()
            t["block"] = self._period_one_divisor_from_state(st, flat.numel()) if period == 1 else period
            t["grad_dtype"] = _DTYPE_CODE[flat.dtype]
            t["state_dtype"] = _DTYPE_CODE[st["m_magnitude"].dtype]
            t["momentum"] = group["momentum"]
            t["nesterov"] = 1 if group["nesterov"] else 0
        dev = items[0][3].device
        lib = _lib.load()
        # the sums of squares of the written blends of bf16 stacks, for the
        # Newton-Schulz normalisation (gathered by the momentum kernels)
        sumsq = torch.empty(len(items) * _SUMSQ_STRIDE, dtype=torch.float64, device=dev)
        sum_index = {key: torch.tensor(idx, dtype=torch.int32, device=dev)
                     for key, idx in stacks.items() if key[2] == torch.bfloat16}
        with torch.cuda.device(dev):
            rc = lib.gefen_muon_tasks_sumsq(tasks.ctypes.data, len(items), tables.data_ptr(), sumsq.data_ptr(),
                                            torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(rc, "gefen_muon_tasks_sumsq")
        updates = {}
        works = {}
        if stacks:
            from gefen_amd.newton_schulz import newton_schulz_batched

            for key, idx in stacks.items():
                coeffs, steps, eps = key[3], key[4], key[5]
                _check_ns_args(coeffs, steps)
                x = bufs[key] if key[2] == torch.bfloat16 else bufs[key].bfloat16()
                works[key] = {}
                si = sum_index.get(key)
                res = newton_schulz_batched(x, coeffs, steps, eps, work=works[key],
                                            sumsq=sumsq if si is not None else None, index=si)
                for slot, i in enumerate(idx):
                    updates[i] = res[slot]
        apply = np.zeros(len(items), dtype=_lib.MUON_APPLY_TASK)
        copy_back = []
        for i, ((group, p, local_p, grad), out) in enumerate(zip(items, outs)):
            st = self.state[p]
            st["step"] += 1
            update = updates.get(i)
            if update is None:
                update = _zeropower_via_newtonschulz(out.view_as(grad), group["ns_coefficients"], group["ns_steps"],
                                                     group["eps"]).contiguous()
            keep.append(update)
            lr_group = group["lr"]
            lr = float(lr_group.item()) if torch.is_tensor(lr_group) else float(lr_group)
            adjusted = _adjust_lr(lr, group["adjust_lr_fn"], p.shape)
            if local_p.is_contiguous():
                target = local_p
            elif hasattr(p, "to_local") and hasattr(p, "placements"):
                target = local_p.contiguous()
                copy_back.append((local_p, target))
            else:
                raise ValueError("GefenMuon fused update requires a contiguous parameter tensor for {}.".format(
                    group["name"]))
            keep.append(target)
            wd = _kernel_weight_decay(lr_group, group["weight_decay"])
            if wd is None:
                # p.mul_(1 - lr * wd) with a 16-bit tensor lr (gefen_muon.py:325-326): the
                # factor in the tensor's dtype, as torch forms it; the apply kernel skips its decay
                target.mul_(1 - lr_group * group["weight_decay"])
                wd = 0.0
            t = apply[i]
            t["p"] = target.data_ptr()
            t["update"] = update.data_ptr()
            t["numel"] = target.numel()
            t["param_dtype"] = _DTYPE_CODE[target.dtype]
            t["transposed"] = 1 if grad.size(0) > grad.size(1) else 0
            t["lr"] = lr
            t["weight_decay"] = wd
            t["adjusted_lr"] = adjusted
        with torch.cuda.device(dev):
            rc = lib.gefen_muon_apply_tasks(apply.ctypes.data, len(items), torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(rc, "gefen_muon_apply_tasks")
        for local_p, target in copy_back:
            local_p.copy_(target)
        plain = (not copy_back
                 and all(local_p is p and grad is p.grad and grad.is_contiguous() for (_, p, local_p, grad) in items))
        if plain:
            # matrices off the batched path keep their momentum output buffer and take
            # the one-matrix Newton-Schulz in every run
            solo = [(i, outs[i], tuple(items[i][0]["ns_coefficients"]), items[i][0]["ns_steps"], items[i][0]["eps"])
                    for i in range(len(items)) if i not in where]
            self._plan = _MuonPlan(self, items, tasks, apply, [(key, idx, bufs[key], works[key], sum_index.get(key))
                                                                 for key, idx in stacks.items()], dev, sumsq, solo)
        del keep

    @_step_entry
    @torch.no_grad()
    def step(self, closure=None):
        """gefen_muon.py:331-350: closure first, then the codebook refresh."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self._maybe_refresh_gefen_codebook()
        self._maybe_save_gefen_grad_histogram()
        self._step_all()
        self._gefen_global_step += 1
        return loss


class _MuonPlan:
    """Cached task tables of GefenMuon._step_all (the GefenMuon counterpart of
    gefen._StepPlan): the momentum and update task tables, the stacked Newton-
    Schulz buffers and their work buffers.  ``refresh`` applies while every
    parameter with a gradient is the recorded one with a gradient of the recorded
    layout, the state tensors are the same objects and each group's Newton-Schulz
    settings (coefficients, steps, eps, lr adjustment) are unchanged; it then
    refreshes gradient addresses, step counts, lr, weight decay, momentum and
    Nesterov, and returns True.  Otherwise it changes nothing and returns False.
    A stack with Newton-Schulz steps applies its parameters' updates inside its
    last product (gefen_gemm_bf16_nt_batched_apply), so the updates are never
    stored and read back; the first step (the table build) applies them with
    gefen_muon_apply_tasks, which the plan's results equal bit for bit.  Matrices
    off the batched path keep their momentum output buffer and take the
    one-matrix Newton-Schulz and gefen_muon_apply_tasks, as in the build."""

    def __init__(self, opt, items, mtasks, apply, stacks, device, sumsq, solo=()):
        self.params = [it[1] for it in items]
        self.pptr = [it[1].data_ptr() for it in items]
        self.numel = [it[3].numel() for it in items]
        self.gdtype = [it[3].dtype for it in items]
        self.states = [opt.state[it[1]] for it in items]
        self.state_keys = ("m_codebook", "m_magnitude")
        self.srefs = [tuple(st[k] for k in self.state_keys) for st in self.states]
        self.grads = [None] * len(items)
        self.gptr = [0] * len(items)
        self.device = device
        self.dev_index = device.index if device.index is not None else torch.cuda.current_device()
        groups = [it[0] for it in items]
        self.distinct = _distinct(groups)
        self.group_index = np.array([next(i for i, d in enumerate(self.distinct) if d is g) for g in groups])
        self.shapes = [tuple(it[1].shape) for it in items]
        self.mtasks = mtasks.copy()
        self.apply = apply.copy()
        self.stacks = stacks
        # stacks with Newton-Schulz steps apply their updates in their last product
        # (gefen_gemm_bf16_nt_batched_apply); the other tensors take gefen_muon_apply_tasks
        # (parameters of 8-element aligned addresses, as that epilogue's vector
        # accesses need; a stack with another parameter keeps the separate pass)
        fused = np.zeros(len(items), dtype=bool)
        self.fuse = []
        for key, idx, _, _, _ in stacks:
            ok = key[4] > 0 and all(items[i][1].data_ptr() % (8 * items[i][1].element_size()) == 0 for i in idx)
            self.fuse.append(ok)
            if ok:
                fused[idx] = True
        self.rest = np.nonzero(~fused)[0]
        # (item, momentum output, coefficients, steps, eps) of the matrices outside
        # the stacks: one-matrix Newton-Schulz, then gefen_muon_apply_tasks
        self.solo = [(i, out.view(items[i][3].shape), c, st, e) for i, out, c, st, e in solo]
        self.sumsq = sumsq
        self.settings = self._settings()
        self.core = None if _gefen_host is None else _gefen_host.PlanCore(self.params, self.states, self.state_keys)
        self.steps = np.zeros(len(items), dtype=np.int64)
        self.mcols = (self.mtasks.dtype.fields["grad"][1],)

    def _settings(self):
        """Per distinct group: (lr, weight_decay, momentum, nesterov) and the
        Newton-Schulz settings that shape the plan."""
        out = []
        for g in self.distinct:
            lr = g["lr"]
            out.append(((float(lr.item()) if torch.is_tensor(lr) else float(lr),
                         _kernel_weight_decay(lr, g["weight_decay"]), g["momentum"], bool(g["nesterov"])),
                        (tuple(g["ns_coefficients"]), g["ns_steps"], g["eps"], g["adjust_lr_fn"])))
        return out

    def refresh(self, opt) -> bool:
        settings = self._settings()
        if any(a[1] != b[1] or a[0][1] is None for a, b in zip(settings, self.settings)):
            return False
        if self.core is not None:
            if not self.core.refresh(opt.param_groups, self.mtasks.ctypes.data, self.mtasks.itemsize, self.mcols,
                                     self.steps.ctypes.data):
                return False
        else:
            if _plan_checks_python(self, opt) is None:
                return False
            self.mtasks["grad"] = self.gptr
        if settings != self.settings:
            gi = self.group_index
            hyper = [s[0] for s in settings]
            lr = np.array([h[0] for h in hyper])[gi]
            self.apply["lr"] = lr
            self.apply["weight_decay"] = np.array([h[1] for h in hyper])[gi]
            self.apply["adjusted_lr"] = [_adjust_lr(float(v), self.distinct[g]["adjust_lr_fn"], shape)
                                         for v, g, shape in zip(lr, gi, self.shapes)]
            self.mtasks["momentum"] = np.array([h[2] for h in hyper])[gi]
            self.mtasks["nesterov"] = np.array([1 if h[3] else 0 for h in hyper])[gi]
            self.settings = settings
        return True

    def run(self, opt) -> None:
        from gefen_amd.newton_schulz import newton_schulz_batched

        lib = _lib.load()
        tables = opt._codebook_tables()
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            _lib.check(lib.gefen_muon_tasks_sumsq(self.mtasks.ctypes.data, len(self.mtasks), tables.data_ptr(),
                                                  self.sumsq.data_ptr(), stream), "gefen_muon_tasks_sumsq")
            # newton_schulz_batched may return its input (a bf16 copy of a non-bf16
            # stack, with an even or zero step count): every input and result stays
            # referenced here until the launch that reads them is enqueued
            keep = []
            for (key, idx, buf, work, sum_index), fuse in zip(self.stacks, self.fuse):
                coeffs, steps, eps = key[3], key[4], key[5]
                x = buf if key[2] == torch.bfloat16 else buf.bfloat16()
                sums = self.sumsq if sum_index is not None else None
                if fuse:  # the last product updates the parameters (gefen_muon.py:47, 325-329)
                    newton_schulz_batched(x, coeffs, steps, eps, work=work, sumsq=sums, index=sum_index,
                                          apply=self.apply[idx])
                    keep.append(x)
                    continue
                res = newton_schulz_batched(x, coeffs, steps, eps, work=work, sumsq=sums, index=sum_index)
                keep.append((x, res))
                slot_bytes = res[0].numel() * res.element_size()
                self.apply["update"][idx] = res.data_ptr() + np.arange(len(idx), dtype=np.uint64) * slot_bytes
            for i, out, coeffs, steps, eps in self.solo:
                upd = _zeropower_via_newtonschulz(out, coeffs, steps, eps).contiguous()
                keep.append(upd)
                self.apply["update"][i] = upd.data_ptr()
            if len(self.rest):
                rest = np.ascontiguousarray(self.apply[self.rest])
                _lib.check(lib.gefen_muon_apply_tasks(rest.ctypes.data, len(rest), stream), "gefen_muon_apply_tasks")
            del keep

"""The Gefen optimizer on MI355X (reference: gefen.py, ndvbd/Gefen 1.2.3).

Drop-in for ``gefen.Gefen``: same constructor, param-group flattening (one
group per tensor), ``step()``, state keys / shapes / dtypes and
``state_dict()``.  Every tensor op of the step runs on the HIP device:

* first step (gefen.py:969-980, 305-419): period scores of every gradient
  (one host sync), block-normalised histograms, fp32 count accumulation and
  the exact-DP codebook, all on the device;
* each step (gefen.py:1208-1333): one fused kernel pass per tensor (vmean EMA,
  weight decay, stepsize, momentum, 8-bit quantisation, parameter update),
  with all tensors of a dtype class batched into a few launches.

The arithmetic is the reference's CPU path (``fused=False``): codebook indices
and magnitudes are bit-identical to it, parameters agree to fp32 rtol 1e-5 /
1 bf16 ulp.  There is no CPU implementation: parameters must live on a HIP
device.
"""

from __future__ import annotations

import ctypes
import functools
import math
from itertools import chain
from pathlib import Path
from typing import Iterable, List, Optional, Tuple, Union

import numpy as np
import torch
import torch.nn as nn

from gefen_amd import _lib
from gefen_amd import quantization as quantization_module

try:  # host-side plan checks in C++ (gefen_amd/csrc/host_plan.cpp); the Python checks otherwise
    from gefen_amd import _gefen_host
except ImportError:
    _gefen_host = None
from gefen_amd.partitioning import PeriodScorer, divisors

FIND_PERIOD_BACKEND = None

FUSE_AUTOMATIC_VMEAN_UPDATE = True
FUSE_GEFEN_AUTOMATIC_STEP = True
FUSE_HISTOGRAM_FOR_EXACT = True
F_FP32 = False

_DTYPE_CODE = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


# --------------------------------------------------------------------------- helpers
def automatic_partition_view(flat_tensor: torch.Tensor, period: int) -> torch.Tensor:
    """[numel / period, period] view of a flat tensor (gefen.py:21-39)."""
    if flat_tensor.dim() != 1:
        raise ValueError("Automatic partition view expects a 1D tensor, got dim={}".format(flat_tensor.dim()))
    if period <= 0:
        raise ValueError("Automatic partition period must be positive, got {}".format(period))
    if flat_tensor.numel() % period != 0:
        raise ValueError("Automatic partition expects numel {} to be divisible by period {}".format(
            flat_tensor.numel(), period))
    return flat_tensor.view(-1, period)


def automatic_partition_reduce(flat_tensor: torch.Tensor, period: int, reduce_op: str) -> torch.Tensor:
    """Per-block mean or max (gefen.py:42-50)."""
    view = automatic_partition_view(flat_tensor, period)
    if reduce_op == "mean":
        return view.mean(dim=1, keepdim=True)
    if reduce_op == "max":
        return view.max(dim=1, keepdim=True).values
    raise ValueError("Unexpected reduce_op: {}".format(reduce_op))


def gefen_state_dtype_from_grad(grad_view: torch.Tensor) -> torch.dtype:
    """State dtype = gradient dtype unless F_FP32 (gefen.py:53-69)."""
    force_fp32 = globals().get("F_FP32", False)
    if not isinstance(force_fp32, bool):
        raise TypeError("F_FP32 must be a bool, got {}".format(type(force_fp32).__name__))
    if force_fp32:
        return torch.float32
    if grad_view.dtype in (torch.float32, torch.float16, torch.bfloat16):
        return grad_view.dtype
    raise ValueError("Gefen state dtype is undefined for gradient dtype {}".format(grad_view.dtype))


def largest_divisor_at_most(value: int, limit: int) -> int:
    """gefen.py:72-82."""
    if value <= 0:
        raise ValueError("Expected value to be positive, got {}".format(value))
    elif limit <= 0:
        raise ValueError("Expected limit to be positive, got {}".format(limit))
    if value <= limit:
        return value
    found = divisors(value, max_divisor=limit)
    if len(found) == 0:
        raise ValueError("Could not find a positive divisor for value {}".format(value))
    return found[-1]


def _safe_filename(text: str) -> str:
    return "".join(c if c.isalnum() or c in "._" else "_" for c in text).strip("_")


def automatic_vmean_update(vmean: torch.Tensor, grad_view: torch.Tensor, beta2: float, *, use_fused: bool) -> None:
    """vmean EMA of gefen.py:91-119 (always the HIP kernel)."""
    from gefen_amd.kernels.automatic_vmean import automatic_vmean_update_cuda

    automatic_vmean_update_cuda(vmean, grad_view, beta2)


def gefen_nearest_codebook_indices(codebook: torch.Tensor, normalized_vals: torch.Tensor) -> torch.Tensor:
    """Nearest codeword, lower-bound search with ties to the left (gefen.py:122-143)."""
    if codebook.device != normalized_vals.device:
        raise ValueError("Gefen codebook device {} does not match normalized_vals device {}.".format(
            codebook.device, normalized_vals.device))
    k = codebook.numel()
    flat = normalized_vals.reshape(-1).float()
    idx = torch.searchsorted(codebook, flat)
    left = (idx - 1).clamp(0, k - 1)
    right = idx.clamp(0, k - 1)
    pick = torch.where((flat - codebook[left]).abs() <= (flat - codebook[right]).abs(), left, right)
    return pick.to(torch.uint8).view(normalized_vals.shape)


def gefen_dequantize_unpacked_indices(codebook: torch.Tensor, stored_indices: torch.Tensor,
                                      like_tensor: torch.Tensor) -> torch.Tensor:
    """codebook[idx] in the dtype of like_tensor (gefen.py:146-169)."""
    if codebook.device != stored_indices.device:
        raise ValueError("Gefen codebook device {} does not match stored index device {}.".format(
            codebook.device, stored_indices.device))
    coeff = codebook[stored_indices.long()].to(device=like_tensor.device, dtype=like_tensor.dtype)
    if hasattr(like_tensor, "device_mesh") and hasattr(like_tensor, "placements"):
        cls = type(like_tensor)
        if hasattr(cls, "from_local"):
            return cls.from_local(coeff, like_tensor.device_mesh, like_tensor.placements)
    return coeff


def gefen_set_unpacked_indices(stored_indices: torch.Tensor, indices: torch.Tensor) -> None:
    stored_indices.copy_(indices.to(torch.uint8))


def gefen_automatic_fused_update(*, p, grad_view, m_codebook, m_magnitude, stepsize, codebook, packed_indices,
                                 beta1, lr) -> None:
    """gefen.py:178-212."""
    if grad_view.device.type != "cuda":
        raise ValueError("Fused automatic Gefen update requires CUDA tensors.")
    if codebook.device != grad_view.device:
        raise ValueError("Gefen codebook device {} does not match grad_view device {}.".format(
            codebook.device, grad_view.device))
    from gefen_amd.kernels.automatic_gefen_fused import automatic_gefen_fused_update_cuda

    automatic_gefen_fused_update_cuda(p, grad_view, m_codebook, m_magnitude, stepsize, codebook, packed_indices,
                                      beta1, lr)


def gefen_automatic_fused_update_from_vmean(*, p, grad_view, m_codebook, m_magnitude, vmean, codebook,
                                            packed_indices, beta1, lr, bias_correction_1, bias_correction_2,
                                            eps) -> None:
    """gefen.py:215-257."""
    if grad_view.device.type != "cuda":
        raise ValueError("Fused automatic Gefen update requires CUDA tensors.")
    if codebook.device != grad_view.device:
        raise ValueError("Gefen codebook device {} does not match grad_view device {}.".format(
            codebook.device, grad_view.device))
    from gefen_amd.kernels.automatic_gefen_fused import automatic_gefen_fused_update_from_vmean_cuda

    automatic_gefen_fused_update_from_vmean_cuda(p, grad_view, m_codebook, m_magnitude, vmean, codebook,
                                                 packed_indices, beta1, lr, bias_correction_1, bias_correction_2,
                                                 eps)


def gefen_automatic_period1_update(*, p, grad_flat, m_codebook, m_magnitude, vmean, codebook, period_one_divisor,
                                   beta1, beta2, lr, bias_correction_1, bias_correction_2, eps) -> None:
    """gefen.py:260-302."""
    if grad_flat.device.type != "cuda":
        raise ValueError("Fused period-1 Gefen update requires CUDA tensors.")
    if codebook.device != grad_flat.device:
        raise ValueError("Gefen codebook device {} does not match grad_flat device {}.".format(
            codebook.device, grad_flat.device))
    from gefen_amd.kernels.automatic_gefen_fused import automatic_gefen_period1_update_cuda

    automatic_gefen_period1_update_cuda(p, grad_flat, m_codebook, m_magnitude, vmean, codebook, period_one_divisor,
                                        beta1, beta2, lr, bias_correction_1, bias_correction_2, eps)


def learn_gefen_exact_codebook_from_grad_periods(*, grad_periods, codebook_device: torch.device, num_codebooks: int,
                                                 force_endpoints: bool, verbose: bool, compute_mse_logging: bool,
                                                 use_fused_histogram: bool = FUSE_HISTOGRAM_FOR_EXACT
                                                 ) -> Optional[torch.Tensor]:
    """gefen.py:305-419 on the device: per-tensor histograms of block-normalised
    gradients, fp32 accumulation in parameter order, exact DP."""
    if hasattr(quantization_module, "SAVE_CODEBOOK_PREFIX"):
        prefix = quantization_module.SAVE_CODEBOOK_PREFIX
        if prefix is not None:
            if not hasattr(quantization_module, "LIST_STEPS_SAVE_HIST_GRAD"):
                raise ValueError(
                    "Gefen exact codebook learning does not support SAVE_CODEBOOK_PREFIX exports. "
                    "Disable exports or define LIST_STEPS_SAVE_HIST_GRAD for the explicit histogram export path.")
            elif quantization_module.LIST_STEPS_SAVE_HIST_GRAD is None:
                raise ValueError(
                    "Gefen exact codebook learning does not support SAVE_CODEBOOK_PREFIX exports. "
                    "Disable exports or use a non-exact research path outside the publishable Gefen optimizer.")
    from gefen_amd.kernels.exact_histogram_fused import gefen_exact_histogram_cuda

    bins = num_codebooks * 16
    lib = _lib.load()
    acc = None
    local = None
    total = 0
    for _, flat, period, _ in grad_periods:
        if flat.device.type != "cuda":
            raise ValueError("gefen_amd learns the codebook from HIP device gradients, got {}".format(flat.device))
        if acc is None:
            acc = torch.zeros(bins, dtype=torch.float32, device=flat.device)
            local = torch.zeros(bins, dtype=torch.int64, device=flat.device)
        else:
            local.zero_()
        gefen_exact_histogram_cuda(flat, period, local)
        with torch.cuda.device(flat.device):
            _lib.check(lib.gefen_accumulate_counts(acc.data_ptr(), local.data_ptr(), bins,
                                                   torch.cuda.current_stream(flat.device).cuda_stream))
        total += flat.numel()
    if total == 0:
        return None
    codebook = quantization_module.exact_dp_from_counts(acc, num_codebooks, force_endpoints).to(codebook_device)
    if verbose and compute_mse_logging:
        edges = torch.linspace(-1.0, 1.0, steps=bins + 1, dtype=torch.float32)
        centers = 0.5 * (edges[:-1] + edges[1:])
        counts = acc.cpu()
        active = counts > 0
        ac = centers[active]
        cb = codebook.cpu()
        idx = torch.searchsorted(cb, ac)
        left = (idx - 1).clamp(0, cb.numel() - 1)
        right = idx.clamp(0, cb.numel() - 1)
        assign = torch.where((ac - cb[left]).abs() <= (ac - cb[right]).abs(), left, right)
        err = ac - cb[assign]
        print("  exact DP: MSE_normalized={:.6e}".format((err.square() * counts[active]).sum().item() / total))
    return codebook


def _resolve_find_period_backend(grad: torch.Tensor) -> str:
    global FIND_PERIOD_BACKEND
    if FIND_PERIOD_BACKEND is not None:
        return FIND_PERIOD_BACKEND
    work = grad.to_local() if hasattr(grad, "to_local") else grad
    FIND_PERIOD_BACKEND = "cuda_kernel" if work.device.type == "cuda" else "cpu"
    return FIND_PERIOD_BACKEND


def _flat_with_data(grad: torch.Tensor) -> torch.Tensor:
    """grad.detach().reshape(-1), after touching its data: a gradient whose storage
    is not allocated yet raises here, where the reference's first kernel call
    would raise."""
    flat = grad.detach().reshape(-1)
    flat.data_ptr()
    return flat


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(index: int) -> int:
    """The hipStream_t of the current stream of device `index` (without building a
    torch.cuda.Stream object when torch offers the raw handle)."""
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def _step_entry(impl):
    """Optimizer.step of the Gefen optimizers.  torch.optim.Optimizer wraps a
    subclass's step in profile_hook_step: a record_function range around the step
    pre-hooks, the step and the post-hooks.  This entry runs that same wrapper
    whenever a step hook is registered (on the optimizer or globally) or a
    profiler is running, and the step alone otherwise, which keeps the
    record_function dispatch off every step's host path.  ``hooked`` tells
    Optimizer.__init__ not to wrap it again."""
    from torch.optim import optimizer as _optim

    hooked = torch.optim.Optimizer.profile_hook_step(impl)
    # without torch's profiler query (or its global hook tables) every step takes the wrapper
    profiling = getattr(getattr(torch._C, "_autograd", None), "_profiler_enabled", None)
    pre = getattr(_optim, "_global_optimizer_pre_hooks", None)
    post = getattr(_optim, "_global_optimizer_post_hooks", None)
    if profiling is None or pre is None or post is None:
        hooked.hooked = True
        return hooked

    @functools.wraps(impl)
    def step(self, *args, **kwargs):
        if (self._optimizer_step_pre_hooks or self._optimizer_step_post_hooks or pre or post or profiling()):
            return hooked(self, *args, **kwargs)
        return impl(self, *args, **kwargs)

    step.hooked = True
    return step


def _local(tensor):
    if hasattr(tensor, "to_local"):
        tensor = tensor.to_local()
    if hasattr(tensor, "wait"):
        tensor = tensor.wait()
    return tensor


# state entries a cached plan requires to stay the same objects
_GEFEN_STATE_KEYS = ("m_codebook", "m_magnitude", "vmean")


class _StepPlan:
    """Cached task table of Gefen._step_all.

    Valid while the optimizer's parameters with a gradient are the same objects
    in the same order, each parameter keeps its storage, each gradient is a
    plain contiguous tensor of the same dtype, size and device, and each
    parameter's state tensors are the same objects.  ``refresh`` checks exactly
    that, then advances the step counts and returns the table with the current
    gradient addresses, hyperparameters and bias corrections; it returns None
    (and changes nothing) when the plan no longer applies.
    """

    __slots__ = ("params", "pptr", "numel", "gdtype", "states", "state_keys", "srefs", "groups", "tasks", "device",
                 "dev_index",
                 "grads", "gptr", "distinct", "group_index", "hyper", "core", "steps", "columns", "tables", "handle",
                 "lib", "run_fn", "tptr")

    def __init__(self, opt, items, tasks, device, tables):
        self.params = [it[1] for it in items]
        self.pptr = [it[1].data_ptr() for it in items]
        self.numel = [it[3].numel() for it in items]
        self.gdtype = [it[3].dtype for it in items]
        self.states = [opt.state[it[1]] for it in items]
        self.state_keys = _GEFEN_STATE_KEYS
        self.srefs = [tuple(st[k] for k in self.state_keys) for st in self.states]
        self.groups = [it[0] for it in items]
        # position of each tensor's group among the distinct groups (hyperparameters are per group)
        self.distinct = _distinct(self.groups)
        self.group_index = [next(i for i, d in enumerate(self.distinct) if d is grp) for grp in self.groups]
        self.tasks = tasks.copy()
        self.device = device
        self.dev_index = device.index if device.index is not None else torch.cuda.current_device()
        # gradient tensors of the last Python refresh: the same object again needs fewer checks
        self.grads = [None] * len(items)
        self.gptr = [0] * len(items)
        self.hyper = None  # per-group hyperparameters last written into the table
        self.core = None if _gefen_host is None else _gefen_host.PlanCore(self.params, self.states, self.state_keys)
        self.steps = np.zeros(len(items), dtype=np.int64)
        fields = self.tasks.dtype.fields
        self.columns = tuple(fields[c][1] for c in ("grad", "lr", "beta1", "beta2", "eps", "weight_decay",
                                                     "bias_correction_1", "bias_correction_2"))
        # the launches of this table, kept by the library (gefen_step_plan): a step
        # only rewrites gradient addresses and scalars before launching
        self.lib = _lib.load()
        self.tables = tables
        self.handle = None
        handle = ctypes.c_void_p()
        with torch.cuda.device(device):
            _lib.check(self.lib.gefen_step_plan_create(self.tasks.ctypes.data, len(self.tasks), tables.data_ptr(),
                                                       ctypes.byref(handle)), "gefen_step_plan_create")
        self.handle = handle.value
        self.run_fn = ctypes.cast(self.lib.gefen_step_plan_run, ctypes.c_void_p).value
        self.tptr = self.tasks.ctypes.data

    def step(self, opt, tables, stream) -> bool:
        """One cached step on `stream` (the plan's device current): the checks and
        refresh of ``refresh``, then the kept launches; False (nothing changed or
        launched) when the plan no longer applies.  With the host extension both
        happen in one call (PlanCore.step)."""
        if self.core is not None and tables is self.tables:
            rc = self.core.step(opt.param_groups, self.tptr, self.tasks.itemsize, self.columns,
                                self.steps.ctypes.data, self.run_fn, self.handle, stream)
            if rc == -1:
                return False
            _lib.check(rc, "gefen_step_plan_run")
            return True
        tasks = self.refresh(opt)
        if tasks is None:
            return False
        self.run(tasks, tables, stream)
        return True

    def __del__(self):
        handle = getattr(self, "handle", None)
        if handle:
            self.handle = None
            try:
                self.lib.gefen_step_plan_destroy(handle)
            except Exception:  # interpreter shutdown: the library may already be gone
                pass

    def run(self, tasks, tables, stream) -> None:
        """Steps the refreshed table on `stream` (the plan's device current):
        through the kept launches, or with gefen_step_tasks when the codebook
        tables are no longer the plan's."""
        if tables is self.tables:
            _lib.check(self.lib.gefen_step_plan_run(self.handle, tasks.ctypes.data, len(tasks), stream),
                       "gefen_step_plan_run")
        else:
            _lib.check(self.lib.gefen_step_tasks(tasks.ctypes.data, len(tasks), tables.data_ptr(), stream),
                       "gefen_step_tasks")

    def refresh(self, opt):
        t = self.tasks
        if self.core is not None:
            # checks, gradient addresses, hyperparameters, bias corrections and the
            # step counts in C++ (gefen_amd/csrc/host_plan.cpp)
            if not self.core.refresh(opt.param_groups, t.ctypes.data, t.itemsize, self.columns,
                                     self.steps.ctypes.data):
                return None
            return t
        # hyperparameters once per distinct group (the table's columns are rewritten
        # only when they change), bias corrections once per (group, step)
        hyper = []
        for grp in self.distinct:
            glr = grp["lr"]
            wd = _kernel_weight_decay(glr, grp["weight_decay"])
            if wd is None:
                return None
            hyper.append((float(glr.item()) if torch.is_tensor(glr) else float(glr), grp["beta1"], grp["beta2"],
                          grp["eps"], wd))
        steps = _plan_checks_python(self, opt)
        if steps is None:
            return None
        t["grad"] = self.gptr
        t = self.tasks
        if hyper != self.hyper:
            gi = self.group_index
            for col, j in (("lr", 0), ("beta1", 1), ("beta2", 2), ("eps", 3), ("weight_decay", 4)):
                t[col] = [hyper[i][j] for i in gi]
            self.hyper = hyper
        if not isinstance(steps, np.ndarray):
            steps = np.asarray(steps, dtype=np.int64)
        s0 = int(steps[0])
        if len(hyper) == 1 and int(steps.min()) == s0 == int(steps.max()):
            b1, b2 = hyper[0][1], hyper[0][2]
            t["bias_correction_1"] = 1 - b1 ** s0
            t["bias_correction_2"] = 1 - b2 ** s0
        else:
            corr = {}
            bc1, bc2 = [], []
            for gi, step in zip(self.group_index, steps.tolist()):
                c = corr.get((gi, step))
                if c is None:
                    c = corr[(gi, step)] = (1 - hyper[gi][1] ** step, 1 - hyper[gi][2] ** step)
                bc1.append(c[0])
                bc2.append(c[1])
            t["bias_correction_1"] = bc1
            t["bias_correction_2"] = bc2
        return t


def _plan_checks_python(plan, opt):
    """The checks of PlanCore.refresh (gefen_amd/csrc/host_plan.cpp) in Python, for
    a plan with params, pptr, numel, gdtype, grads, gptr, states, state_keys,
    srefs and dev_index (used when the host extension is not built): fills plan.gptr and
    returns the advanced step counts, or None (changing nothing) when the plan no
    longer applies."""
    params, pptr, numel, gdtype, grads, gptr = plan.params, plan.pptr, plan.numel, plan.gdtype, plan.grads, plan.gptr
    n = len(params)
    dev = plan.dev_index
    k = 0
    for group in opt.param_groups:
        for p in group["params"]:
            g = p.grad
            if g is None:
                continue
            if k == n or p is not params[k]:
                return None
            if g is not grads[k]:
                if (type(g) is not torch.Tensor or g.dtype is not gdtype[k] or g.numel() != numel[k]
                        or not g.is_contiguous() or g.get_device() != dev):
                    return None
                grads[k] = g
            elif g.numel() != numel[k] or not g.is_contiguous():  # resized or restrided in place
                return None
            if p.data_ptr() != pptr[k] or not p.is_contiguous():
                return None
            gptr[k] = g.data_ptr()
            k += 1
    if k != n:
        return None
    keys = plan.state_keys
    for st, refs in zip(plan.states, plan.srefs):
        if any(st.get(k) is not r for k, r in zip(keys, refs)):
            return None
        if type(st.get("step")) is not int:
            return None
    steps = []
    for st in plan.states:
        step = st["step"] + 1
        st["step"] = step
        steps.append(step)
    return steps


def _kernel_weight_decay(lr, weight_decay):
    """The weight decay to hand the kernels for a group (gefen.py:1280-1281,
    p.mul_(1 - lr * wd)).  The kernels form the factor as (float)(1 - lr * wd) in
    double.  For a float32 tensor lr torch forms it in float32,
    f = fl32(1 - fl32(lr * fl32(wd))), which differs from the double expression in
    about 1% of cases; the kernels then get wd' = (1 - f) / lr, for which the double
    expression lies within ~2^-51 (relative) of f, far inside half a float ulp, so
    it rounds to f exactly.  Returns wd' (wd itself for a number or float64 lr),
    or None where that cannot hold (a tensor lr of a 16-bit dtype, lr <= 0, f zero
    or not finite): torch then applies the factor before the launch."""
    if not (weight_decay > 0.0 and torch.is_tensor(lr) and lr.dtype != torch.float64):
        return weight_decay
    if lr.dtype != torch.float32:
        return None
    lr_v = float(lr.item())
    f = np.float32(np.float32(1.0) - np.float32(np.float32(lr_v) * np.float32(weight_decay)))
    if not (lr_v > 0.0 and np.isfinite(f) and f != 0.0):
        return None
    return (1.0 - float(f)) / lr_v


def _distinct(objs):
    """The distinct objects of a list by identity, in first-appearance order."""
    out = []
    for o in objs:
        if not any(o is d for d in out):
            out.append(o)
    return out


# --------------------------------------------------------------------------- optimizer
class Gefen(torch.optim.Optimizer):
    """Gefen (gefen.py:435-1420): AdamW with an 8-bit codebook first moment and
    a block-shared second moment, on MI355X."""

    def __init__(self, params: Iterable[Union[nn.Parameter, Tuple[str, nn.Parameter]]],
                 lr: Union[float, torch.Tensor] = 1e-3, betas: Tuple[float, float] = (0.9, 0.999),
                 eps: float = 1e-8, weight_decay: float = 0.0, *, fused: bool = True, verbose: bool = False):
        print("Initializing Gefen optimizer (fused={}).".format(fused))
        if not 0.0 <= lr:
            raise ValueError("Invalid learning rate: {}".format(lr))
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError("Invalid beta parameter at index 0: {}".format(betas[0]))
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError("Invalid beta parameter at index 1: {}".format(betas[1]))
        if not 0.0 <= weight_decay:
            raise ValueError("Invalid weight_decay value: {}".format(weight_decay))

        def validate(glr, gbetas, geps, gwd):
            if not 0.0 <= glr:
                raise ValueError("Invalid learning rate: {}".format(glr))
            elif not 0.0 <= gbetas[0] < 1.0:
                raise ValueError("Invalid beta parameter at index 0: {}".format(gbetas[0]))
            elif not 0.0 <= gbetas[1] < 1.0:
                raise ValueError("Invalid beta parameter at index 1: {}".format(gbetas[1]))
            elif not 0.0 <= gwd:
                raise ValueError("Invalid weight_decay value: {}".format(gwd))
            elif not 0.0 <= geps:
                raise ValueError("Invalid epsilon value: {}".format(geps))

        def named(group_params):
            if isinstance(group_params, torch.Tensor):
                yield None, group_params
                return
            for item in group_params:
                if isinstance(item, tuple):
                    name, param = item
                else:
                    name, param = None, item
                if not isinstance(param, torch.Tensor):
                    raise TypeError("Gefen can only optimize Tensors, but one of the params is {}".format(
                        type(param).__name__))
                yield name, param

        groups = []

        def add(name, param, glr, gbetas, geps, gwd):
            if not param.requires_grad:
                return
            groups.append({"name": str(name).lower(), "params": param, "lr": glr, "beta1": gbetas[0],
                           "beta2": gbetas[1], "eps": geps, "weight_decay": gwd})

        self.fused = fused
        self.verbose = verbose
        self._printed_optimizer_memory = False
        self._gefen_codebook = None
        self._gefen_global_step = 0
        self._printed_gefen_materialization = False
        self._exit_after_grad_sq_save = False
        self._tables = None
        self._tables_key = None
        self._plan = None

        for gi, item in enumerate(params):
            if isinstance(item, dict):
                if "params" not in item:
                    raise ValueError("Gefen parameter group {} is missing the 'params' key.".format(gi))
                glr = item.get("lr", lr)
                gbetas = item.get("betas", betas)
                geps = item.get("eps", eps)
                gwd = item.get("weight_decay", weight_decay)
                validate(glr, gbetas, geps, gwd)
                for pi, (name, param) in enumerate(named(item["params"])):
                    add(name if name is not None else "group_{}_param_{}".format(gi, pi), param, glr, gbetas,
                        geps, gwd)
            else:
                for name, param in named((item,)):
                    add(name if name is not None else "param_{}".format(gi), param, lr, betas, eps,
                        weight_decay)
        super().__init__(groups, dict(lr=lr, beta1=betas[0], beta2=betas[1], eps=eps))
        if self._cap_period_by_shape_enabled():
            self._record_constructor_parameter_shapes()

    # ----------------------------------------------------------- reference hooks
    def _use_fused_automatic_vmean(self) -> bool:
        return self.fused and FUSE_AUTOMATIC_VMEAN_UPDATE

    def _use_fused_gefen_automatic_step(self) -> bool:
        return self.fused and FUSE_GEFEN_AUTOMATIC_STEP

    def _gefen_codebook_device(self) -> torch.device:
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is not None:
                    return p.grad.device
                return p.device
        raise ValueError("Expected at least one parameter when choosing the Gefen codebook device.")

    def _period_one_divisor_for_numel(self, numel: int) -> int:
        return largest_divisor_at_most(numel, 256)

    def _period_one_divisor_from_state(self, state, total_numel: int) -> int:
        d = state.get("period_one_divisor")
        if d is None:
            d = self._period_one_divisor_for_numel(total_numel)
            state["period_one_divisor"] = d
        elif not isinstance(d, int):
            raise TypeError("period_one_divisor must be an int, got {}".format(type(d).__name__))
        elif d <= 0:
            raise ValueError("period_one_divisor must be positive, got {}".format(d))
        elif total_numel % d != 0:
            raise ValueError("period_one_divisor {} must divide flattened tensor numel {}".format(d, total_numel))
        mag = state.get("m_magnitude")
        if torch.is_tensor(mag) and mag.shape != (total_numel // d, 1):
            raise ValueError("Expected m_magnitude shape {} for period_one_divisor {}, got {}".format(
                (total_numel // d, 1), d, tuple(mag.shape)))
        return d

    def _cap_period_by_shape_enabled(self) -> bool:
        return globals().get("CPBS", False)

    def _record_constructor_parameter_shapes(self) -> None:
        for group in self.param_groups:
            for p in group["params"]:
                self.state[p]["parameter_shape"] = tuple(p.shape)

    def _max_period_for_param(self, param: torch.Tensor) -> Optional[int]:
        if not self._cap_period_by_shape_enabled():
            return None
        shape = tuple(self.state.get(param, {}).get("parameter_shape", tuple(param.shape)))
        if len(shape) == 0:
            return 1
        return max(int(d) for d in shape)

    def _print_period_results_enabled(self) -> bool:
        ppr = globals().get("PPR", False)
        if not isinstance(ppr, bool):
            raise TypeError("PPR must be a bool, got {}".format(type(ppr).__name__))
        return ppr

    def _resolve_local_tensor(self, tensor: torch.Tensor, tensor_name: str) -> torch.Tensor:
        tensor = _local(tensor)
        if not isinstance(tensor, torch.Tensor):
            raise TypeError("Expected {} to resolve to a torch.Tensor, got {}.".format(tensor_name, type(tensor)))
        return tensor

    def _print_gefen_codebook(self, label: str, codebook: torch.Tensor) -> None:
        if self.verbose:
            print("{} ({} entries):".format(label, codebook.numel()))

    def _print_period(self, param_name: str, param: torch.Tensor, period: int) -> None:
        if self.verbose:
            print("Gefen shared-v:", param_name, "| shape=", tuple(param.shape), "| numel=", param.numel(),
                  "| automatic period=", period)

    # ----------------------------------------------------------- periods
    def _predict_periods(self, items) -> List[int]:
        """Periods of [(param, grad)] with one host sync (gefen.py:765-828)."""
        if items:
            _resolve_find_period_backend(items[0][1])
        ppr = self._print_period_results_enabled()
        scorer = PeriodScorer(mode=1)
        for p, grad in items:
            work = _local(grad)
            if work.device.type != "cuda":
                raise ValueError("gefen_amd runs on HIP devices; a gradient is on {}".format(work.device))
            try:
                flat = _flat_with_data(work)
            except RuntimeError as exc:
                # a lazily materialised (FSDP) gradient: add_(0) allocates it, then
                # the scores are taken again (gefen.py:789-810)
                msg = str(exc)
                if "data is not allocated yet" not in msg and "invalid python storage" not in msg:
                    raise
                work.add_(0)
                flat = _flat_with_data(work)
            scorer.add(flat, self._max_period_for_param(p), ppr)
        return scorer.finish()

    def _predict_period_from_grad_sq(self, param_name: str, param: torch.Tensor, grad: torch.Tensor) -> int:
        return self._predict_periods([(param, grad)])[0]

    def _iter_gefen_grad_periods(self, reuse_existing_periods: bool = False):
        """(name, flat grad, period, grad) per parameter with a gradient, periods
        predicted in one batch (gefen.py:882-924)."""
        entries = []
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                grad = _local(p.grad).detach()
                flat = grad.reshape(-1)
                if flat.numel() == 0:
                    continue
                entries.append((group, p, grad, flat))
        need = []
        for group, p, grad, flat in entries:
            st = self.state[p]
            if reuse_existing_periods:
                if "automatic_period" not in st:
                    raise ValueError(
                        "Expected automatic_period to exist for {} before refreshing Gefen codebook at optimizer "
                        "step {}".format(group["name"], self._gefen_global_step))
            elif flat.numel() == 1:
                st["automatic_period"] = 1
            else:
                need.append((p, grad))
        if need:
            for (p, _), period in zip(need, self._predict_periods(need)):
                self.state[p]["automatic_period"] = period
        for group, p, grad, flat in entries:
            period = self.state[p]["automatic_period"]
            if flat.numel() % period != 0:
                raise ValueError(
                    "Automatic partition period {} does not divide parameter {} with numel {} while learning "
                    "Gefen codebook".format(period, group["name"], flat.numel()))
            yield group["name"], flat, period, grad

    # ----------------------------------------------------------- codebook
    def _learn_gefen_exact_codebook(self, reuse_existing_periods: bool = False,
                                    compute_mse_logging: bool = True) -> Optional[torch.Tensor]:
        codebook = learn_gefen_exact_codebook_from_grad_periods(
            grad_periods=self._iter_gefen_grad_periods(reuse_existing_periods=reuse_existing_periods),
            codebook_device=self._gefen_codebook_device(), num_codebooks=256, force_endpoints=True,
            verbose=self.verbose, compute_mse_logging=compute_mse_logging, use_fused_histogram=True)
        if codebook is None:
            return None
        self._print_gefen_codebook("Gefen codebook", codebook)
        return codebook

    def _ensure_gefen_codebook(self, reuse_existing_periods: bool = False) -> None:
        mse = globals().get("COMPUTE_GEFEN_EXACT_MSE_LOGGING", False)
        codebook = self._learn_gefen_exact_codebook(reuse_existing_periods=reuse_existing_periods,
                                                    compute_mse_logging=mse)
        if codebook is not None:
            self._gefen_codebook = codebook

    def _has_restored_automatic_periods(self) -> bool:
        return any("automatic_period" in self.state.get(p, {}) for g in self.param_groups for p in g["params"])

    def _maybe_refresh_gefen_codebook(self) -> None:
        if self._gefen_codebook is not None:
            device = self._gefen_codebook_device()
            if self._gefen_codebook.device != device:
                self._gefen_codebook = self._gefen_codebook.to(device)
            return
        self._ensure_gefen_codebook(reuse_existing_periods=self._has_restored_automatic_periods())

    def _maybe_save_gefen_grad_histogram(self) -> None:
        if not hasattr(quantization_module, "LIST_STEPS_SAVE_HIST_GRAD"):
            return
        steps = quantization_module.LIST_STEPS_SAVE_HIST_GRAD
        if steps is None or self._gefen_global_step not in steps:
            return
        if not hasattr(quantization_module, "SAVE_CODEBOOK_PREFIX"):
            raise ValueError("LIST_STEPS_SAVE_HIST_GRAD requires SAVE_CODEBOOK_PREFIX to be defined and set.")
        prefix = quantization_module.SAVE_CODEBOOK_PREFIX
        if prefix is None:
            raise ValueError("LIST_STEPS_SAVE_HIST_GRAD requires SAVE_CODEBOOK_PREFIX to be set.")
        if self._gefen_codebook is None:
            raise ValueError("Expected Gefen codebook to be initialized before saving gradient histogram.")
        from gefen_amd.kernels.exact_histogram_fused import gefen_exact_histogram_cuda

        bins = self._gefen_codebook.numel() * 16
        lib = _lib.load()
        acc = None
        total = 0
        for _, flat, period, _ in self._iter_gefen_grad_periods(reuse_existing_periods=True):
            if acc is None:
                acc = torch.zeros(bins, dtype=torch.float32, device=flat.device)
            local = torch.zeros(bins, dtype=torch.int64, device=flat.device)
            gefen_exact_histogram_cuda(flat, period, local)
            _lib.check(lib.gefen_accumulate_counts(acc.data_ptr(), local.data_ptr(), bins,
                                                   torch.cuda.current_stream(flat.device).cuda_stream))
            total += flat.numel()
        if total == 0:
            raise ValueError("Cannot save Gefen gradient histogram because no gradients were available.")
        quantization_module.save_distribution_histogram_pt_from_counts(
            hist=acc.cpu(), prefix=prefix, suffix="grad_hist_step_{}".format(self._gefen_global_step),
            num_samples=total)

    def _codebook_tables(self) -> torch.Tensor:
        """Lookup tables of the current codebook, rebuilt when the codebook changes."""
        cb = self._gefen_codebook
        key = (id(cb), cb._version, cb.data_ptr(), cb.device)
        if self._tables is None or self._tables_key != key:
            lib = _lib.load()
            cbc = cb.detach().to(torch.float32).contiguous()
            tables = torch.empty(int(lib.gefen_codebook_tables_size()), dtype=torch.uint8, device=cb.device)
            with torch.cuda.device(cb.device):
                _lib.check(lib.gefen_prepare_codebook(cbc.data_ptr(), cbc.numel(), tables.data_ptr(),
                                                      torch.cuda.current_stream(cb.device).cuda_stream))
            self._tables = tables
            self._tables_key = key
            self._tables_src = cbc
        return self._tables

    # ----------------------------------------------------------- state
    def _init_gefen_state(self, state, grad_view: torch.Tensor) -> None:
        """gefen.py:1039-1062."""
        state["m_codebook_shape"] = tuple(grad_view.shape)
        state["m_codebook"] = torch.zeros_like(grad_view, dtype=torch.uint8, memory_format=torch.preserve_format)
        sdt = gefen_state_dtype_from_grad(grad_view)
        if grad_view.shape[1] == 1:
            d = self._period_one_divisor_for_numel(grad_view.numel())
            state["period_one_divisor"] = d
            rows = grad_view.numel() // d
        elif grad_view.shape[1] > 1:
            rows = grad_view.shape[0]
        else:
            raise ValueError("Expected grad_view second dimension to be positive, got {}".format(grad_view.shape[1]))
        state["m_magnitude"] = torch.zeros_like(grad_view[:rows, 0:1], dtype=sdt, memory_format=torch.preserve_format)

    def _maybe_save_grad_sq_and_exit(self, param_name: str, grad: torch.Tensor, automatic_period: int) -> None:
        name = globals().get("GRAD_SQ_PARAMETER_NAME_TO_SAVE")
        if name is None:
            return
        if not isinstance(name, str):
            raise TypeError("GRAD_SQ_PARAMETER_NAME_TO_SAVE must be a str, got {}".format(type(name).__name__))
        if name.lower() != param_name:
            return
        out = Path.cwd() / "{}_grad_sq.pt".format(_safe_filename(param_name))
        torch.save(grad.detach().float().square().reshape(-1).cpu(), out)
        print("Gefen automatic period for {} is {}".format(param_name, automatic_period), flush=True)
        print("Saved Gefen grad^2 tensor to {}".format(out.resolve()), flush=True)
        self._exit_after_grad_sq_save = True

    def _init_states(self, pending) -> None:
        """First touch of parameters (gefen.py:1232-1268): periods (batched), state tensors."""
        need = [(p, grad) for (group, p, local_p, grad) in pending
                if "automatic_period" not in self.state[p] and grad.numel() > 1]
        periods = self._predict_periods(need) if need else []
        for (p, _), period in zip(need, periods):
            self.state[p]["automatic_period"] = period
        for group, p, local_p, grad in pending:
            st = self.state[p]
            n = grad.numel()
            if "automatic_period" not in st:
                st["automatic_period"] = 1  # numel == 1
            period = st["automatic_period"]
            if n % period != 0:
                raise ValueError("Automatic partition period {} does not divide local shard of parameter {} with "
                                 "numel {}".format(period, group["name"], n))
            self._maybe_save_grad_sq_and_exit(group["name"], grad, period)
            st["step"] = 0
            view = automatic_partition_view(grad.reshape(-1), period)
            self._init_gefen_state(st, view)
            st["vmean"] = torch.zeros_like(view[:, 0:1], dtype=gefen_state_dtype_from_grad(view),
                                           memory_format=torch.preserve_format)
            self._print_period(group["name"], local_p, period)

    def _collect(self):
        """(group, param, local param, local grad) of every parameter with a gradient."""
        out = []
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                name = group["name"]
                local_p = self._resolve_local_tensor(p, "parameter {}".format(name))
                grad = self._resolve_local_tensor(p.grad, "gradient {}".format(name))
                if local_p.numel() != grad.numel():
                    raise ValueError("Local parameter shard numel {} does not match local gradient numel {} for {}."
                                     .format(local_p.numel(), grad.numel(), name))
                if grad.numel() == 0:
                    continue
                if grad.device.type != "cuda" or local_p.device.type != "cuda":
                    raise RuntimeError("gefen_amd runs on HIP devices; {} is on {}".format(name, grad.device))
                out.append((group, p, local_p, grad))
        return out

    def _step_all(self) -> None:
        """One fused kernel pass per tensor, batched per device (gefen.py:1208-1333).

        The task table is cached as a plan: while the same parameters carry
        gradients of the same layout and the state tensors are unchanged, a step
        only refreshes gradient addresses, step counts and hyperparameters.
        """
        plan = self._plan
        if plan is not None:
            tables = self._codebook_tables()
            if torch.cuda.current_device() == plan.dev_index:
                done = plan.step(self, tables, _stream_handle(plan.dev_index))
            else:
                with torch.cuda.device(plan.device):
                    done = plan.step(self, tables, _stream_handle(plan.dev_index))
            if done:
                return
        self._plan = None
        self._step_all_build()

    def _step_all_build(self) -> None:
        """_step_all from scratch: resolves every tensor, fills the task table and,
        when every tensor is a plain contiguous device tensor, caches the plan."""
        items = self._collect()
        if not items:
            return
        fresh = [it for it in items if "step" not in self.state[it[1]]]
        if fresh:
            self._init_states(fresh)
        if self._gefen_codebook is None:
            raise ValueError("Expected Gefen codebook to be initialized before fused update.")
        tables = self._codebook_tables()
        tasks = np.zeros(len(items), dtype=_lib.STEP_TASK)
        keep = []
        copy_back = []
        plain = True
        for i, (group, p, local_p, grad) in enumerate(items):
            st = self.state[p]
            period = st["automatic_period"]
            st["step"] += 1
            step = st["step"]
            lr_group = group["lr"]
            lr = float(lr_group.item()) if torch.is_tensor(lr_group) else float(lr_group)
            b1, b2 = group["beta1"], group["beta2"]
            plain = plain and local_p is p and grad is p.grad and grad.is_contiguous()
            flat_grad = grad.reshape(-1)
            if not flat_grad.is_contiguous():
                flat_grad = flat_grad.contiguous()
            if local_p.is_contiguous():
                fused_p = local_p
            elif hasattr(p, "to_local") and hasattr(p, "placements"):
                fused_p = local_p.contiguous()
                copy_back.append((local_p, fused_p))
            else:
                raise ValueError("Gefen fused update requires a contiguous parameter tensor for {}.".format(
                    group["name"]))
            if fused_p.dtype != flat_grad.dtype:
                raise ValueError("Expected grad_view dtype {} to match p dtype {}.".format(flat_grad.dtype,
                                                                                           fused_p.dtype))
            keep.append(flat_grad)
            wd = _kernel_weight_decay(lr_group, group["weight_decay"])
            if wd is None:
                # p.mul_(1 - lr * wd) as gefen.py:1280-1281 evaluates it for a 16-bit
                # tensor lr; the kernel then skips its own decay
                fused_p.mul_(1 - lr_group * group["weight_decay"])
                wd = 0.0
            t = tasks[i]
            t["p"] = fused_p.data_ptr()
            t["grad"] = flat_grad.data_ptr()
            t["m_codebook"] = st["m_codebook"].data_ptr()
            t["m_magnitude"] = st["m_magnitude"].data_ptr()
            t["vmean"] = st["vmean"].data_ptr()
            t["numel"] = flat_grad.numel()
            t["period"] = period
            t["period_one_divisor"] = (self._period_one_divisor_from_state(st, flat_grad.numel())
                                       if period == 1 else 0)
            t["param_dtype"] = _DTYPE_CODE[fused_p.dtype]
            t["state_dtype"] = _DTYPE_CODE[st["m_magnitude"].dtype]
            t["beta1"] = b1
            t["beta2"] = b2
            t["lr"] = lr
            t["eps"] = group["eps"]
            t["weight_decay"] = wd
            t["bias_correction_1"] = 1 - b1 ** step
            t["bias_correction_2"] = 1 - b2 ** step
        dev = items[0][3].device
        lib = _lib.load()
        with torch.cuda.device(dev):
            rc = lib.gefen_step_tasks(tasks.ctypes.data, len(items), tables.data_ptr(),
                                      torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(rc, "gefen_step_tasks")
        for local_p, fused_p in copy_back:
            local_p.copy_(fused_p)
        del keep
        if plain and all(it[3].device == dev for it in items):
            self._plan = _StepPlan(self, items, tasks, dev, tables)

    def _optimizer_state_memory_bytes(self) -> int:
        return sum(v.numel() * v.element_size() for s in self.state.values() for v in s.values() if torch.is_tensor(v))

    # ----------------------------------------------------------- checkpoint
    def state_dict(self):
        """Base state dict plus the global step and the codebook (gefen.py:1343-1349)."""
        sd = super().state_dict()
        sd["gefen_global_step"] = self._gefen_global_step
        sd["gefen_codebook"] = self._gefen_codebook
        return sd

    def load_state_dict(self, state_dict):
        """gefen.py:1351-1397: restores the codebook and keeps each saved state
        tensor's dtype where torch's loader would have cast it."""
        state_dict = dict(state_dict)
        gstep = state_dict.pop("gefen_global_step", 0)
        saved = state_dict.get("state", {}) or {}
        codebook = state_dict.pop("gefen_codebook", None)
        super().load_state_dict(state_dict)
        self._plan = None
        self._gefen_global_step = gstep
        if self._cap_period_by_shape_enabled():
            for group in self.param_groups:
                for param in group["params"]:
                    self.state[param].setdefault("parameter_shape", tuple(param.shape))
        self._gefen_codebook = codebook
        self._tables = None
        id_map = dict(zip(chain.from_iterable(g["params"] for g in state_dict["param_groups"]),
                          chain.from_iterable(g["params"] for g in self.param_groups)))
        for pid, pstate in saved.items():
            param = id_map.get(pid)
            if param is None:
                continue
            live = self.state.get(param)
            if live is None:
                continue
            for key, value in pstate.items():
                if not torch.is_tensor(value):
                    continue
                cur = live.get(key)
                if torch.is_tensor(cur) and cur.dtype == value.dtype:
                    continue
                device = cur.device if torch.is_tensor(cur) else param.device
                live[key] = value.to(device=device, dtype=value.dtype)

    @_step_entry
    def step(self, closure=None):
        """gefen.py:1399-1420 (the reference's step runs under torch.no_grad(); here
        the steady-state step through the cached plan records no autograd ops and
        skips entering it)."""
        if closure is None and self._plan is not None and self._cached_step():
            return None
        with torch.no_grad():
            self._maybe_refresh_gefen_codebook()
            self._maybe_save_gefen_grad_histogram()
            loss = None
            if closure is not None:
                with torch.enable_grad():
                    loss = closure()
            self._step_all()
            self._gefen_global_step += 1
            if self._exit_after_grad_sq_save:
                raise SystemExit(0)
            return loss

    def _cached_step(self) -> bool:
        """step() without a closure through the cached plan: taken when the codebook
        is in place on the gradients' device and no gradient-histogram save is due
        this step (the two checks at the top of step() then do nothing).  The kept
        launches write the tensors through their device addresses, so no autograd
        op is recorded.  False, with nothing changed, when the plan no longer
        applies; step() then runs in full."""
        cb = self._gefen_codebook
        if cb is None or cb.device != self._gefen_codebook_device():
            return False
        due = getattr(quantization_module, "LIST_STEPS_SAVE_HIST_GRAD", None)
        if due is not None and self._gefen_global_step in due:
            return False
        plan = self._plan
        tables = self._codebook_tables()
        if torch.cuda.current_device() == plan.dev_index:
            done = plan.step(self, tables, _stream_handle(plan.dev_index))
        else:
            with torch.cuda.device(plan.device):
                done = plan.step(self, tables, _stream_handle(plan.dev_index))
        if not done:
            self._plan = None
            return False
        self._gefen_global_step += 1
        if self._exit_after_grad_sq_save:
            raise SystemExit(0)
        return True

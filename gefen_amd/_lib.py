"""ctypes binding of libgefen_hip.so, the C ABI declared in include/gefen_hip.h.

The library is built in-tree by ``python -m gefen_amd.build``.  Loading fails
loudly when it is missing: there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libgefen_hip.so"

GEFEN_OK, GEFEN_EINVAL, GEFEN_ERUNTIME = 0, 1, 2
F32, F16, BF16 = 0, 1, 2

P = ctypes.c_void_p
I32 = ctypes.c_int
I64 = ctypes.c_int64
DBL = ctypes.c_double
SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/gefen_hip.h
SIGNATURES = {
    "gefen_last_error": (ctypes.c_char_p, []),
    "gefen_abi_version": (I32, []),
    "gefen_device_allocations": (I64, []),
    "gefen_struct_size": (SZ, [I32]),
    "gefen_codebook_tables_size": (SZ, []),
    "gefen_prepare_codebook": (I32, [P, I32, P, P]),
    "gefen_automatic_vmean_update": (I32, [P, I32, P, I32, I64, I64, DBL, P]),
    "gefen_automatic_fused_update": (I32, [P, P, I32, P, P, I32, P, P, I32, I32, I64, I64, DBL, DBL, P]),
    "gefen_automatic_fused_update_from_vmean": (
        I32, [P, P, I32, P, P, I32, P, I32, P, I32, I32, I64, I64, DBL, DBL, DBL, DBL, DBL, P]),
    "gefen_automatic_period1_update": (
        I32, [P, P, I32, P, P, I32, P, I32, P, I32, I64, I64, DBL, DBL, DBL, DBL, DBL, DBL, P]),
    "gefen_automatic_muon_momentum": (I32, [P, I32, P, P, I32, P, I32, P, I32, I64, I64, DBL, P]),
    "gefen_step_tasks": (I32, [P, I32, P, P]),
    "gefen_step_tasks_noalloc": (I32, [P, I32, P, P]),
    "gefen_step_plan_create": (I32, [P, I32, P, P]),
    "gefen_step_plan_run": (I32, [P, P, I32, P]),
    "gefen_step_plan_time_runs": (I32, [P, I32]),
    "gefen_step_plan_last_ms": (I32, [P, P]),
    "gefen_step_plan_destroy": (None, [P]),
    "gefen_muon_tasks": (I32, [P, I32, P, P]),
    "gefen_muon_tasks_sumsq": (I32, [P, I32, P, P, P]),
    "gefen_ns_prepare": (I32, [P, P, I32, I32, I32, DBL, P]),
    "gefen_ns_prepare_sumsq": (I32, [P, P, I32, I32, I32, DBL, P, P, P]),
    "gefen_ns_normalize_sumsq": (I32, [P, P, I32, I32, I32, DBL, P, P, I32, P]),
    "gefen_muon_apply_tasks": (I32, [P, I32, P]),
    "gefen_exact_histogram": (I32, [P, I32, I64, I64, P, I32, P]),
    "gefen_accumulate_counts": (I32, [P, P, I32, P]),
    "gefen_exact_dp_workspace_size": (SZ, [I32, I32]),
    "gefen_exact_dp": (I32, [P, I32, I32, I32, P, P, P]),
    "gefen_average_adjacent_log_block_mean_difference": (I32, [P, I32, I64, I64, I32, DBL, P, P]),
    "gefen_period_scores_workspace_size": (SZ, [I64, P, I32]),
    "gefen_period_scores": (I32, [P, I32, I64, P, I32, I32, DBL, P, P, P]),
    "gefen_average_within_block_variance": (I32, [P, I32, I64, I64, I32, P, P]),
    "gefen_average_within_block_coefficient_of_variation": (I32, [P, I32, I64, I64, I32, P, P]),
    "gefen_lloyd_accumulate": (I32, [P, I32, I64, I64, P, I32, P, P, P]),
    "gefen_lloyd_mse": (I32, [P, I32, I64, I64, P, P, I32, P, P, P]),
    "gefen_gemm_bf16": (I32, [P, I64, P, I64, I32, P, I64, P, I64, I32, I32, I32, DBL, DBL, P]),
    "gefen_gemm_bf16_nt_batched": (I32, [P, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, I32, I32,
                                         I32, I32, I32, DBL, DBL, I32, P]),
    "gefen_gram_bf16_batched": (I32, [P, I64, I64, P, I64, I64, I32, I32, I32, DBL, P]),
    "gefen_gemm_bf16_nt_batched_apply": (I32, [P, I64, I64, P, I64, I64, P, I64, I64, I32, I32, I32, I32, DBL, DBL,
                                               P, P]),
}

# numpy mirror of struct gefen_step_task / gefen_muon_task (natural C alignment)
STEP_TASK = np.dtype([
    ("p", np.uint64), ("grad", np.uint64), ("m_codebook", np.uint64), ("m_magnitude", np.uint64),
    ("vmean", np.uint64), ("numel", np.int64), ("period", np.int64), ("period_one_divisor", np.int64),
    ("param_dtype", np.int32), ("state_dtype", np.int32),
    ("beta1", np.float64), ("beta2", np.float64), ("lr", np.float64), ("eps", np.float64),
    ("weight_decay", np.float64), ("bias_correction_1", np.float64), ("bias_correction_2", np.float64),
])
MUON_TASK = np.dtype([
    ("grad", np.uint64), ("m_codebook", np.uint64), ("m_magnitude", np.uint64), ("out", np.uint64),
    ("numel", np.int64), ("block", np.int64), ("grad_dtype", np.int32), ("state_dtype", np.int32),
    ("momentum", np.float64), ("nesterov", np.int32), ("pad", np.int32),
])
MUON_APPLY_TASK = np.dtype([
    ("p", np.uint64), ("update", np.uint64), ("numel", np.int64), ("param_dtype", np.int32),
    ("transposed", np.int32), ("lr", np.float64), ("weight_decay", np.float64), ("adjusted_lr", np.float64),
])
assert STEP_TASK.itemsize == 128 and MUON_TASK.itemsize == 72 and MUON_APPLY_TASK.itemsize == 56

_LIB = None


class GefenError(RuntimeError):
    pass


def load():
    """Load libgefen_hip.so once; raise if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise ImportError(
            "gefen_amd: {} is missing; build it with `python -m gefen_amd.build` "
            "(hipcc, gfx950). There is no fallback implementation.".format(LIB_PATH))
    lib = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_LOCAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(rc: int, what: str = "") -> None:
    """Raise the Python exception the reference raises for this failure class."""
    if rc == GEFEN_OK:
        return
    msg = load().gefen_last_error().decode("utf-8", "replace")
    if rc == GEFEN_EINVAL:
        raise ValueError(msg)
    raise RuntimeError("{}{}".format(what + ": " if what else "", msg))

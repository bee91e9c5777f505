"""Partition-block scores (reference: kernels/period_variance.py:12-161).

The three reference entry points return a host float after a device sync, as
the reference does.  ``period_scores_cuda`` scores every divisor of one
gradient in one call (one sync for all divisors).
"""

from __future__ import annotations

from typing import Sequence

import numpy as np
import torch

from .gefen_hip import check, device_guard, dtype_code, load_extension, stream_of


def _check_values(values, period):
    if not isinstance(values, torch.Tensor):
        raise TypeError("Expected torch.Tensor, got {}".format(type(values).__name__))
    elif values.device.type != "cuda":
        raise ValueError("Expected a CUDA tensor, got device {}".format(values.device))
    elif values.numel() == 0:
        raise ValueError("Expected a non-empty tensor.")
    elif period <= 0:
        raise ValueError("Expected a positive period, got {}".format(period))
    elif values.numel() % period != 0:
        raise ValueError("Expected length {} to be divisible by period {}.".format(values.numel(), period))


def average_within_block_variance_cuda_kernel(values: torch.Tensor, period: int, *, input_is_squared: bool) -> float:
    _check_values(values, period)
    lib = load_extension()
    v = values.detach().reshape(-1).contiguous()
    out = torch.empty(1, dtype=torch.float64, device=v.device)
    with device_guard(v):
        rc = lib.gefen_average_within_block_variance(v.data_ptr(), dtype_code(v.dtype), v.numel(), int(period),
                                                     int(bool(input_is_squared)), out.data_ptr(), stream_of(v))
    check(rc, "average_within_block_variance_cuda")
    return float(out.item())


def average_within_block_coefficient_of_variation_cuda_kernel(values: torch.Tensor, period: int, *,
                                                               input_is_squared: bool) -> float:
    _check_values(values, period)
    lib = load_extension()
    v = values.detach().reshape(-1).contiguous()
    out = torch.empty(3, dtype=torch.float64, device=v.device)
    with device_guard(v):
        rc = lib.gefen_average_within_block_coefficient_of_variation(
            v.data_ptr(), dtype_code(v.dtype), v.numel(), int(period), int(bool(input_is_squared)),
            out.data_ptr(), stream_of(v))
    check(rc, "average_within_block_coefficient_of_variation_cuda")
    s, cnt, neg = out.tolist()
    # period_variance_kernel.cu:311-317
    if neg > 0.0:
        raise RuntimeError("Expected non-negative block means for coefficient of variation.")
    if cnt == 0.0:
        raise RuntimeError("Encountered only zero block means, cannot compute coefficient of variation.")
    return float(s / cnt)


def average_adjacent_log_block_mean_difference_cuda_kernel(values: torch.Tensor, period: int, *,
                                                           input_is_squared: bool, epsilon: float) -> float:
    _check_values(values, period)
    if epsilon <= 0.0:
        raise ValueError("Expected a positive epsilon, got {}".format(epsilon))
    elif values.numel() // period < 2:
        raise ValueError("Expected at least two blocks to compare adjacent block means.")
    lib = load_extension()
    v = values.detach().reshape(-1).contiguous()
    out = torch.empty(2, dtype=torch.float64, device=v.device)
    with device_guard(v):
        rc = lib.gefen_average_adjacent_log_block_mean_difference(
            v.data_ptr(), dtype_code(v.dtype), v.numel(), int(period), int(bool(input_is_squared)),
            float(epsilon), out.data_ptr(), stream_of(v))
    check(rc, "average_adjacent_log_block_mean_difference_cuda")
    score, invalid = out.tolist()
    if invalid > 0.0:  # period_variance_kernel.cu:392-394
        raise RuntimeError("Expected values plus epsilon to be positive before log transform.")
    return float(score)


def period_scores_launch(values: torch.Tensor, divisors: Sequence[int], mode: int, epsilon: float,
                         scores: torch.Tensor, workspace: torch.Tensor) -> None:
    """Enqueue the scores of all `divisors` (ascending) of one flat gradient into
    scores[:len(divisors)] (float64, device) and the invalid-input count into
    scores[len(divisors)]; no synchronisation."""
    lib = load_extension()
    v = values.detach().reshape(-1)
    if not v.is_contiguous():
        raise ValueError("Expected a contiguous tensor.")
    divs = np.ascontiguousarray(np.asarray(list(divisors), dtype=np.int64))
    with device_guard(v):
        rc = lib.gefen_period_scores(v.data_ptr(), dtype_code(v.dtype), v.numel(), divs.ctypes.data, divs.size,
                                     int(mode), float(epsilon), scores.data_ptr(), workspace.data_ptr(),
                                     stream_of(v))
    check(rc, "gefen_period_scores")


def period_scores_workspace_bytes(numel: int, divisors: Sequence[int]) -> int:
    divs = np.ascontiguousarray(np.asarray(list(divisors), dtype=np.int64))
    return int(load_extension().gefen_period_scores_workspace_size(int(numel), divs.ctypes.data, divs.size))

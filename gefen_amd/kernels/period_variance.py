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


def _flat(values: torch.Tensor) -> torch.Tensor:
    return values.detach().reshape(-1).contiguous()


def _average_within_block_variance_cuda_impl(values: torch.Tensor, period: int,
                                             input_is_squared: bool) -> torch.Tensor:
    """The extension function average_within_block_variance_cuda
    (period_variance_kernel.cu:177-243): float64 tensor [1] on the device,
    sqrt of the mean block variance."""
    lib = load_extension()
    v = _flat(values)
    out = torch.empty(1, dtype=torch.float64, device=v.device)
    with device_guard(v):
        rc = lib.gefen_average_within_block_variance(v.data_ptr(), dtype_code(v.dtype), v.numel(), int(period),
                                                     int(bool(input_is_squared)), out.data_ptr(), stream_of(v))
    check(rc, "average_within_block_variance_cuda")
    return out


def _average_within_block_coefficient_of_variation_cuda_impl(values: torch.Tensor, period: int,
                                                             input_is_squared: bool) -> torch.Tensor:
    """The extension function average_within_block_coefficient_of_variation_cuda
    (period_variance_kernel.cu:245-318): 0-d float64 tensor, the mean std/mean over
    blocks with a positive mean; raises RuntimeError as the reference does."""
    lib = load_extension()
    v = _flat(values)
    out = torch.empty(3, dtype=torch.float64, device=v.device)
    with device_guard(v):
        rc = lib.gefen_average_within_block_coefficient_of_variation(
            v.data_ptr(), dtype_code(v.dtype), v.numel(), int(period), int(bool(input_is_squared)),
            out.data_ptr(), stream_of(v))
    check(rc, "average_within_block_coefficient_of_variation_cuda")
    _, cnt, neg = out.tolist()
    # period_variance_kernel.cu:311-317
    if neg > 0.0:
        raise RuntimeError("Expected non-negative block means for coefficient of variation.")
    if cnt == 0.0:
        raise RuntimeError("Encountered only zero block means, cannot compute coefficient of variation.")
    return out[0].div(out[1])


def _average_adjacent_log_block_mean_difference_cuda_impl(values: torch.Tensor, period: int, input_is_squared: bool,
                                                          epsilon: float) -> torch.Tensor:
    """The extension function average_adjacent_log_block_mean_difference_cuda
    (period_variance_kernel.cu:320-396): 0-d float64 tensor."""
    lib = load_extension()
    v = _flat(values)
    out = torch.empty(2, dtype=torch.float64, device=v.device)
    with device_guard(v):
        rc = lib.gefen_average_adjacent_log_block_mean_difference(
            v.data_ptr(), dtype_code(v.dtype), v.numel(), int(period), int(bool(input_is_squared)),
            float(epsilon), out.data_ptr(), stream_of(v))
    check(rc, "average_adjacent_log_block_mean_difference_cuda")
    if out[1].item() > 0.0:  # period_variance_kernel.cu:392-394
        raise RuntimeError("Expected values plus epsilon to be positive before log transform.")
    return out[0].clone()


_OPAQUE_OP_AVAILABLE = False

# The opaque custom op of period_variance.py:49-72, registered under the same name.
if hasattr(torch.library, "custom_op"):

    @torch.library.custom_op("gefen::average_within_block_variance_cuda", mutates_args=())
    def _average_within_block_variance_cuda_opaque(values: torch.Tensor, period: int,
                                                   input_is_squared: bool) -> torch.Tensor:
        return _average_within_block_variance_cuda_impl(values, period, input_is_squared)

    @_average_within_block_variance_cuda_opaque.register_fake
    def _average_within_block_variance_cuda_opaque_fake(values: torch.Tensor, period: int,
                                                        input_is_squared: bool) -> torch.Tensor:
        del period, input_is_squared
        return values.new_empty(())

    _OPAQUE_OP_AVAILABLE = True


def average_within_block_variance_cuda_kernel(values: torch.Tensor, period: int, *, input_is_squared: bool) -> float:
    _check_values(values, period)
    return float(_average_within_block_variance_cuda_impl(values, period, input_is_squared).item())


def average_within_block_coefficient_of_variation_cuda_kernel(values: torch.Tensor, period: int, *,
                                                               input_is_squared: bool) -> float:
    _check_values(values, period)
    return float(_average_within_block_coefficient_of_variation_cuda_impl(values, period, input_is_squared).item())


def average_adjacent_log_block_mean_difference_cuda_kernel(values: torch.Tensor, period: int, *,
                                                           input_is_squared: bool, epsilon: float) -> float:
    _check_values(values, period)
    if epsilon <= 0.0:
        raise ValueError("Expected a positive epsilon, got {}".format(epsilon))
    elif values.numel() // period < 2:
        raise ValueError("Expected at least two blocks to compare adjacent block means.")
    return float(_average_adjacent_log_block_mean_difference_cuda_impl(values, period, input_is_squared,
                                                                       epsilon).item())


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

"""Block-normalised histogram entry point (reference: kernels/exact_histogram_fused.py:10-58)."""

from __future__ import annotations

import torch

from .gefen_hip import check, device_guard, dtype_code, load_extension, stream_of


def gefen_exact_histogram_cuda(grad_flat: torch.Tensor, period: int, bin_counts: torch.Tensor) -> None:
    """bin_counts += histogram of f32(g)/absmax(block) over [-1, 1] (gefen.py:350-366)."""
    tensors = {"grad_flat": grad_flat, "bin_counts": bin_counts}
    for name, tensor in tensors.items():
        if not isinstance(tensor, torch.Tensor):
            raise TypeError("Expected {} to be a torch.Tensor.".format(name))
        elif tensor.device.type != "cuda":
            raise ValueError("Expected {} to be on CUDA, got device {}.".format(name, tensor.device))
    if grad_flat.dim() != 1:
        raise ValueError("Expected grad_flat to be 1D, got dim={}".format(grad_flat.dim()))
    if bin_counts.dim() != 1:
        raise ValueError("Expected bin_counts to be 1D, got dim={}".format(bin_counts.dim()))
    if bin_counts.dtype != torch.int64:
        raise ValueError("Expected bin_counts to be int64, got {}".format(bin_counts.dtype))
    if period <= 0:
        raise ValueError("Expected period to be positive, got {}".format(period))
    if grad_flat.numel() % period != 0:
        raise ValueError("Expected grad_flat.numel()={} to be divisible by period={}.".format(
            grad_flat.numel(), period))
    if bin_counts.numel() <= 0 or bin_counts.numel() > 4096:
        raise ValueError("Expected histogram bins in [1, 4096], got {}".format(bin_counts.numel()))
    if not bin_counts.is_contiguous():
        raise ValueError("Expected grad_flat and bin_counts to be contiguous.")
    lib = load_extension()
    g = grad_flat.contiguous()
    with device_guard(g):
        rc = lib.gefen_exact_histogram(g.data_ptr(), dtype_code(g.dtype), g.numel(), int(period),
                                       bin_counts.data_ptr(), bin_counts.numel(), stream_of(g))
    check(rc, "gefen_exact_histogram_cuda")

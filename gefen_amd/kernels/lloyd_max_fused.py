"""Lloyd-Max accumulators (reference: kernels/lloyd_max_fused.py:10-143).

Exported like the reference's, which never calls them from the optimizer step.
"""

from __future__ import annotations

import torch

from .gefen_hip import check, device_guard, dtype_code, load_extension, stream_of


def _devices(tensors):
    for name, tensor in tensors.items():
        if not isinstance(tensor, torch.Tensor):
            raise TypeError("Expected {} to be a torch.Tensor.".format(name))
        elif tensor.device.type != "cuda":
            raise ValueError("Expected {} to be on CUDA, got device {}.".format(name, tensor.device))


def gefen_lloyd_accumulate_cuda(grad_flat, codebook, period: int, sums, counts) -> None:
    _devices({"grad_flat": grad_flat, "codebook": codebook, "sums": sums, "counts": counts})
    if grad_flat.dim() != 1:
        raise ValueError("Expected grad_flat to be 1D, got dim={}".format(grad_flat.dim()))
    elif codebook.dim() != 1:
        raise ValueError("Expected codebook to be 1D, got dim={}".format(codebook.dim()))
    elif sums.dim() != 1 or sums.numel() != codebook.numel():
        raise ValueError("Expected sums to be 1D with one entry per codebook value.")
    elif counts.dim() != 1 or counts.numel() != codebook.numel():
        raise ValueError("Expected counts to be 1D with one entry per codebook value.")
    elif codebook.dtype != torch.float32:
        raise ValueError("Expected codebook to be float32, got {}".format(codebook.dtype))
    elif sums.dtype != torch.float32:
        raise ValueError("Expected sums to be float32, got {}".format(sums.dtype))
    elif counts.dtype != torch.int64:
        raise ValueError("Expected counts to be int64, got {}".format(counts.dtype))
    elif period <= 0:
        raise ValueError("Expected period to be positive, got {}".format(period))
    elif grad_flat.numel() % period != 0:
        raise ValueError("Expected grad_flat.numel()={} to be divisible by period={}.".format(
            grad_flat.numel(), period))
    elif codebook.numel() > 256:
        raise ValueError("Expected codebook to have at most 256 entries, got {}".format(codebook.numel()))
    if not sums.is_contiguous() or not counts.is_contiguous():
        raise ValueError("Expected sums and counts to be contiguous.")
    lib = load_extension()
    g = grad_flat.contiguous()
    cb = codebook.contiguous()
    with device_guard(g):
        rc = lib.gefen_lloyd_accumulate(g.data_ptr(), dtype_code(g.dtype), g.numel(), int(period), cb.data_ptr(),
                                        cb.numel(), sums.data_ptr(), counts.data_ptr(), stream_of(g))
    check(rc, "gefen_lloyd_accumulate_cuda")


def gefen_lloyd_mse_cuda(grad_flat, old_codebook, new_codebook, period: int, mse_normalized_sum,
                         mse_original_sum) -> None:
    _devices({"grad_flat": grad_flat, "old_codebook": old_codebook, "new_codebook": new_codebook,
              "mse_normalized_sum": mse_normalized_sum, "mse_original_sum": mse_original_sum})
    if grad_flat.dim() != 1:
        raise ValueError("Expected grad_flat to be 1D, got dim={}".format(grad_flat.dim()))
    elif old_codebook.dim() != 1 or new_codebook.dim() != 1:
        raise ValueError("Expected old_codebook and new_codebook to be 1D.")
    elif old_codebook.numel() != new_codebook.numel():
        raise ValueError("Expected old_codebook and new_codebook to have the same number of entries.")
    elif mse_normalized_sum.numel() != 1 or mse_original_sum.numel() != 1:
        raise ValueError("Expected mse accumulators to be scalar tensors.")
    elif old_codebook.dtype != torch.float32 or new_codebook.dtype != torch.float32:
        raise ValueError("Expected codebooks to be float32.")
    elif mse_normalized_sum.dtype != torch.float32 or mse_original_sum.dtype != torch.float32:
        raise ValueError("Expected mse accumulators to be float32.")
    elif period <= 0:
        raise ValueError("Expected period to be positive, got {}".format(period))
    elif grad_flat.numel() % period != 0:
        raise ValueError("Expected grad_flat.numel()={} to be divisible by period={}.".format(
            grad_flat.numel(), period))
    elif old_codebook.numel() > 256:
        raise ValueError("Expected codebook to have at most 256 entries, got {}".format(old_codebook.numel()))
    lib = load_extension()
    g = grad_flat.contiguous()
    oc = old_codebook.contiguous()
    nc = new_codebook.contiguous()
    with device_guard(g):
        rc = lib.gefen_lloyd_mse(g.data_ptr(), dtype_code(g.dtype), g.numel(), int(period), oc.data_ptr(),
                                 nc.data_ptr(), oc.numel(), mse_normalized_sum.data_ptr(),
                                 mse_original_sum.data_ptr(), stream_of(g))
    check(rc, "gefen_lloyd_mse_cuda")

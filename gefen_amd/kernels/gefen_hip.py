"""Loader of the HIP extension (role of the reference's kernels/gefen_cuda.py:6-22).

``load_extension()`` returns the extension object: the eleven functions of the
reference's extension module (``gefen_cuda_binding.cpp:107-217``) under their
names, taking and returning torch tensors as the pybind11 functions do, plus
every C-ABI function of ``libgefen_hip.so`` (``gefen_*``, include/gefen_hip.h)
as a ctypes function.  The library is built ahead of time
(``python -m gefen_amd.build``), never JIT; a missing library raises.
"""

from __future__ import annotations

import torch

from gefen_amd import _lib

_DTYPE_CODE = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}

# binding name -> (wrapper module, function) that implements it
_BINDING = {
    "automatic_gefen_fused_update_cuda": ("automatic_gefen_fused", "automatic_gefen_fused_update_cuda"),
    "automatic_gefen_fused_update_from_vmean_cuda": ("automatic_gefen_fused",
                                                     "automatic_gefen_fused_update_from_vmean_cuda"),
    "automatic_gefen_period1_update_cuda": ("automatic_gefen_fused", "automatic_gefen_period1_update_cuda"),
    "automatic_gefen_muon_momentum_cuda": ("automatic_gefen_fused", "automatic_gefen_muon_momentum_cuda"),
    "automatic_vmean_update_cuda": ("automatic_vmean", "automatic_vmean_update_cuda"),
    "gefen_exact_histogram_cuda": ("exact_histogram_fused", "gefen_exact_histogram_cuda"),
    "average_within_block_variance_cuda": ("period_variance", "_average_within_block_variance_cuda_impl"),
    "average_within_block_coefficient_of_variation_cuda": (
        "period_variance", "_average_within_block_coefficient_of_variation_cuda_impl"),
    "average_adjacent_log_block_mean_difference_cuda": (
        "period_variance", "_average_adjacent_log_block_mean_difference_cuda_impl"),
    "gefen_lloyd_accumulate_cuda": ("lloyd_max_fused", "gefen_lloyd_accumulate_cuda"),
    "gefen_lloyd_mse_cuda": ("lloyd_max_fused", "gefen_lloyd_mse_cuda"),
}


class HipExtension:
    """The extension module of this build: binding names resolve to the tensor
    functions above, every other attribute to libgefen_hip.so's C ABI."""

    def __init__(self, lib):
        self._lib = lib

    def __getattr__(self, name):
        target = _BINDING.get(name)
        if target is not None:
            import importlib

            fn = getattr(importlib.import_module("gefen_amd.kernels." + target[0]), target[1])
            setattr(self, name, fn)
            return fn
        return getattr(self._lib, name)

    def __dir__(self):
        return sorted(set(_BINDING) | set(_lib.SIGNATURES))


_EXTENSION_MODULE = None


def load_extension() -> HipExtension:
    global _EXTENSION_MODULE
    if _EXTENSION_MODULE is None:
        _EXTENSION_MODULE = HipExtension(_lib.load())
    return _EXTENSION_MODULE


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError("unsupported dtype {}".format(dtype)) from None


def stream_of(t: torch.Tensor):
    """hipStream_t of torch's current stream on the tensor's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def device_guard(t: torch.Tensor):
    return torch.cuda.device(t.device)


def check(rc: int, what: str = "") -> None:
    _lib.check(rc, what)

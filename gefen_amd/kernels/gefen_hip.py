"""Loader of the HIP extension (role of the reference's kernels/gefen_cuda.py:6-22).

``load_extension()`` returns the ctypes handle of ``libgefen_hip.so``; the
library is built ahead of time (``python -m gefen_amd.build``), never JIT.
"""

from __future__ import annotations

import torch

from gefen_amd import _lib

_DTYPE_CODE = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


def load_extension():
    return _lib.load()


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

"""numpy <-> HIP tensor helpers for the GPU parity tests (storage convention:
f32 as float32, f16 / bf16 as uint16 bit patterns)."""

import numpy as np
import torch

TORCH = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
CODE = {"f32": 0, "f16": 1, "bf16": 2}


def to_dev(a: np.ndarray, dtype: str, device="cuda:0") -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if dtype == "f32":
        return torch.from_numpy(a.astype(np.float32, copy=False)).to(device)
    return torch.from_numpy(a.view(np.int16)).view(TORCH[dtype]).to(device)


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def stream():
    return torch.cuda.current_stream().cuda_stream


def ulps16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in units in the last place between 16-bit float bit patterns
    (bf16 or f16: sign-magnitude order)."""
    a = a.astype(np.int32)
    b = b.astype(np.int32)
    ka = np.where(a & 0x8000, 0x8000 - (a & 0x7FFF), 0x8000 + (a & 0x7FFF))
    kb = np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + (b & 0x7FFF))
    return np.abs(ka - kb)


def ulp_at16(bits: np.ndarray, dtype: str) -> np.ndarray:
    """The ulp (float64) at each 16-bit value of dtype 'bf16' or 'f16'."""
    if dtype == "bf16":
        v = np.abs((bits.astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64))
        e = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
        return np.ldexp(1.0, (e - 7).astype(np.int64))
    with np.errstate(over="ignore"):  # the spacing at the largest finite half is inf
        return np.abs(np.spacing(bits.view(np.float16))).astype(np.float64)

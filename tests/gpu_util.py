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

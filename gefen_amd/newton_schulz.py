"""Newton-Schulz orthogonalisation of GefenMuon (gefen_muon.py:16-51) on the device.

X = bf16(G) (transposed when rows > cols), X /= max(||X||, eps), then ns_steps
times:  A = X X^T;  B = b A + c A A;  X = a X + B X, every product rounded to
bf16 once after an fp32-accumulated GEMM.
"""

from __future__ import annotations

from typing import Tuple

import torch


def newton_schulz_bf16(grad: torch.Tensor, coeffs: Tuple[float, float, float], steps: int,
                       eps: float) -> torch.Tensor:
    a, b, c = coeffs
    x = grad.bfloat16()
    transposed = grad.size(0) > grad.size(1)
    if transposed:
        x = x.T
    x = x.contiguous()
    x.div_(x.norm().clamp(min=eps))
    for _ in range(steps):
        gram = x @ x.T.contiguous()
        upd = torch.addmm(gram, gram, gram, beta=b, alpha=c)
        x = torch.addmm(x, upd, x, beta=a)
    if transposed:
        x = x.T
    return x

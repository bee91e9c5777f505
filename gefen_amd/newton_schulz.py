"""Newton-Schulz orthogonalisation of GefenMuon (gefen_muon.py:16-51) on MFMA.

X = bf16(G) (transposed when rows > cols), X /= max(||X||, eps), then ns_steps
times:  A = X X^T;  B = b A + c A A;  X = a X + B X.  Each product is one
gefen_gemm_bf16 call (fp32 accumulation, one bf16 rounding of alpha*AB + beta*D).
"""

from __future__ import annotations

from typing import Tuple

import torch

from gefen_amd import _lib


def gemm(a: torch.Tensor, b: torch.Tensor, b_kcontig: bool, out: torch.Tensor, d: torch.Tensor = None,
         alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    m, k = a.shape
    n = b.shape[0] if b_kcontig else b.shape[1]
    lib = _lib.load()
    rc = lib.gefen_gemm_bf16(a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), int(b_kcontig), out.data_ptr(),
                             out.stride(0), d.data_ptr() if d is not None else None,
                             d.stride(0) if d is not None else 0, m, n, k, float(alpha), float(beta),
                             torch.cuda.current_stream(a.device).cuda_stream)
    _lib.check(rc, "gefen_gemm_bf16")
    return out


def newton_schulz_bf16(grad: torch.Tensor, coeffs: Tuple[float, float, float], steps: int,
                       eps: float) -> torch.Tensor:
    a, b, c = coeffs
    x = grad.bfloat16()
    transposed = grad.size(0) > grad.size(1)
    if transposed:
        x = x.T
    x = x.contiguous()
    x.div_(x.norm().clamp(min=eps))
    m, n = x.shape
    gram = torch.empty(m, m, dtype=torch.bfloat16, device=x.device)
    upd = torch.empty(m, m, dtype=torch.bfloat16, device=x.device)
    nxt = torch.empty_like(x)
    with torch.cuda.device(x.device):
        for _ in range(steps):
            gemm(x, x, True, gram)                                   # X X^T
            gemm(gram, gram, False, upd, d=gram, alpha=c, beta=b)    # b A + c A A
            gemm(upd, x, False, nxt, d=x, alpha=1.0, beta=a)         # a X + B X
            x, nxt = nxt, x
    if transposed:
        x = x.T
    return x

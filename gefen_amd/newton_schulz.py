"""Newton-Schulz orthogonalisation of GefenMuon (gefen_muon.py:16-51) on MFMA.

X = bf16(G) (transposed when rows > cols), X /= max(||X||, eps), then ns_steps
times:  A = X X^T;  B = b A + c A A;  X = a X + B X.  Each product rounds
alpha*AB + beta*D to bf16 once, as torch.addmm does.

newton_schulz_batched runs a stack of same-shaped matrices at once with the
large-tile batched GEMM (every product in A B^T form: X X^T, A A with A
symmetric, B X from X^T, which each step writes beside X); newton_schulz_bf16
is the one-matrix path for shapes the batched GEMM does not tile.
"""

from __future__ import annotations

from typing import Optional, Tuple

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


def batched_shape_ok(rows: int, cols: int) -> bool:
    """The batched GEMM tiles m = min(rows, cols) and n = max(rows, cols) by 256."""
    return rows > 0 and cols > 0 and rows % 256 == 0 and cols % 256 == 0


def gemm_nt_batched(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor, out_t: torch.Tensor = None,
                    d: torch.Tensor = None, alpha: float = 1.0, beta: float = 0.0, symmetric: bool = False,
                    d_t: torch.Tensor = None) -> None:
    """out[i] = alpha * a[i] @ b[i]^T + beta * D[i] (and out_t[i] = out[i]^T) for stacked bf16
    matrices; D is given as d, or as its transpose d_t (read four rows at a time)."""
    if d is not None and d_t is not None:
        raise ValueError("give D as d or as d_t, not both")
    transposed_d = d_t is not None
    if transposed_d:
        d = d_t
    g, m, k = a.shape
    n = b.shape[1]
    lib = _lib.load()

    def ptr(t):
        return t.data_ptr() if t is not None else None

    def ld(t):
        return t.stride(1) if t is not None else 0

    def bs(t):
        return t.stride(0) if t is not None else 0

    rc = lib.gefen_gemm_bf16_nt_batched(a.data_ptr(), a.stride(1), a.stride(0), b.data_ptr(), b.stride(1), b.stride(0),
                                        out.data_ptr(), out.stride(1), out.stride(0), ptr(out_t), ld(out_t), bs(out_t),
                                        ptr(d), ld(d), bs(d), 1 if transposed_d else 0, g, m, n, k, float(alpha),
                                        float(beta), 1 if symmetric else 0,
                                        torch.cuda.current_stream(a.device).cuda_stream)
    _lib.check(rc, "gefen_gemm_bf16_nt_batched")


def newton_schulz_batched(x: torch.Tensor, coeffs: Tuple[float, float, float], steps: int,
                          eps: float, work: Optional[dict] = None, sumsq: Optional[torch.Tensor] = None,
                          index: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Newton-Schulz of every matrix of a [G, rows, cols] bf16 stack, in place of
    x's values (x is normalised in place); returns the [G, rows, cols] result.

    work: a dict that keeps the intermediate buffers between calls with the same
    stack (allocated on first use); the result is then the same buffer on every
    call with the same number of steps.
    sumsq, index: the matrices' sums of squares, already gathered (float64 device
    tensor; matrix g's is sumsq[index[g]], int32 device index, or sumsq[g]), so
    the normalisation does not read the stack twice."""
    a, b, c = coeffs
    g, rows, cols = x.shape
    transposed = rows > cols
    if work is None:
        work = {}

    def buf(name, shape):
        t = work.get(name)
        if t is None or tuple(t.shape) != tuple(shape) or t.device != x.device:
            t = work[name] = torch.empty(shape, dtype=torch.bfloat16, device=x.device)
        return t

    # normalise each matrix, x /= max(||x||, eps) in bf16 (gefen_muon.py:37), and
    # write its transpose: X [G, m, n] with m <= n and X^T
    other = buf("other", (g, cols, rows))
    lib = _lib.load()
    with torch.cuda.device(x.device):
        stream = torch.cuda.current_stream(x.device).cuda_stream
        if sumsq is not None:
            _lib.check(lib.gefen_ns_prepare_sumsq(x.data_ptr(), other.data_ptr(), g, rows, cols, float(eps),
                                                  sumsq.data_ptr(), index.data_ptr() if index is not None else None,
                                                  stream), "gefen_ns_prepare_sumsq")
        else:
            _lib.check(lib.gefen_ns_prepare(x.data_ptr(), other.data_ptr(), g, rows, cols, float(eps), stream),
                       "gefen_ns_prepare")
    x, xt = (other, x) if transposed else (x, other)
    m, n = x.shape[1], x.shape[2]
    gram = buf("gram", (g, m, m))
    upd = buf("upd", (g, m, m))
    nx, nxt = buf("nx", (g, m, n)), buf("nxt", (g, n, m))
    with torch.cuda.device(x.device):
        for it in range(steps):
            gemm_nt_batched(x, x, gram, symmetric=True)                                # X X^T
            gemm_nt_batched(gram, gram, upd, d_t=gram, alpha=c, beta=b, symmetric=True)  # b A + c A A
            if it + 1 < steps:
                gemm_nt_batched(upd, xt, nx, out_t=nxt, d_t=xt, alpha=1.0, beta=a)       # a X + B X (and ^T)
                x, nx = nx, x
                xt, nxt = nxt, xt
            elif transposed:
                # last step, result wanted as X^T: a X^T + X^T B with B symmetric
                gemm_nt_batched(xt, upd, nxt, d_t=x, alpha=1.0, beta=a)
                xt = nxt
            else:
                gemm_nt_batched(upd, xt, nx, d_t=xt, alpha=1.0, beta=a)
                x = nx
    return xt if transposed else x

"""Newton-Schulz orthogonalisation of GefenMuon (gefen_muon.py:16-51) on MFMA.

X = bf16(G) (transposed when rows > cols), X /= max(||X||, eps), then ns_steps
times:  A = X X^T;  B = b A + c A A;  X = a X + B X.  Each product rounds
alpha*AB + beta*D to bf16 once, as torch.addmm does.

newton_schulz_batched runs a stack of same-shaped matrices at once with the
large-tile batched GEMM, keeping only X^T between iterations: X X^T comes from
X^T through transposing LDS reads (gefen_gram_bf16_batched), b A + c A A is an
A B^T product of the symmetric A, and B X = (X^T B)^T is written as X'^T (the
last iteration writes the orientation it returns).  newton_schulz_bf16 is the
one-matrix path for shapes the batched GEMM does not tile.
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
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


# The batched kernels address an operand through a buffer resource whose extent
# is a 32-bit byte count: the Gram product reads a whole X^T [n, m] through one
# (gefen_gram_bf16_batched rejects k * ldxt * 2 > 2^31 - 1), so a matrix of 2^30 or
# more bf16 elements takes the one-matrix path, which forms 64-bit addresses.
_BATCHED_MAX_BYTES = (1 << 31) - 1


def batched_shape_ok(rows: int, cols: int) -> bool:
    """The batched GEMM tiles m = min(rows, cols) and n = max(rows, cols) by 256,
    and reads one bf16 matrix through a buffer of less than 2^31 bytes."""
    return (rows > 0 and cols > 0 and rows % 256 == 0 and cols % 256 == 0
            and rows * cols * 2 <= _BATCHED_MAX_BYTES)


def gemm_nt_batched(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor, out_t: torch.Tensor = None,
                    d: torch.Tensor = None, alpha: float = 1.0, beta: float = 0.0, symmetric: bool = False,
                    d_t: torch.Tensor = None) -> None:
    """out[i] = alpha * a[i] @ b[i]^T + beta * D[i] (and out_t[i] = out[i]^T) for stacked bf16
    matrices; D is given as d, or as its transpose d_t (read four rows at a time); out may be
    None when out_t is given (only the transposed result is written)."""
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
                                        ptr(out), ld(out), bs(out), ptr(out_t), ld(out_t), bs(out_t),
                                        ptr(d), ld(d), bs(d), 1 if transposed_d else 0, g, m, n, k, float(alpha),
                                        float(beta), 1 if symmetric else 0,
                                        torch.cuda.current_stream(a.device).cuda_stream)
    _lib.check(rc, "gefen_gemm_bf16_nt_batched")


def gemm_nt_batched_apply(a: torch.Tensor, b: torch.Tensor, d_t: Optional[torch.Tensor], alpha: float, beta: float,
                          tasks) -> None:
    """U[i] = alpha * a[i] @ b[i]^T + beta * D[i] (D given as its transpose d_t),
    applied as GefenMuon's update of parameter tasks[i] (a MUON_APPLY_TASK array,
    one row per matrix; U[i] is the parameter's layout, or its transpose when
    tasks[i].transposed) instead of being stored."""
    g, m, k = a.shape
    n = b.shape[1]
    if len(tasks) != g:
        raise ValueError("one apply task per matrix")
    tasks = np.ascontiguousarray(tasks)
    lib = _lib.load()
    rc = lib.gefen_gemm_bf16_nt_batched_apply(a.data_ptr(), a.stride(1), a.stride(0), b.data_ptr(), b.stride(1),
                                              b.stride(0), d_t.data_ptr() if d_t is not None else None,
                                              d_t.stride(1) if d_t is not None else 0,
                                              d_t.stride(0) if d_t is not None else 0, g, m, n, k, float(alpha),
                                              float(beta), tasks.ctypes.data,
                                              torch.cuda.current_stream(a.device).cuda_stream)
    _lib.check(rc, "gefen_gemm_bf16_nt_batched_apply")


def gram_batched(xt: torch.Tensor, out: torch.Tensor) -> None:
    """out[i] = X[i] @ X[i]^T for the stacked X[i]^T = xt[i] ([k, m] bf16, row-major)."""
    g, k, m = xt.shape
    lib = _lib.load()
    rc = lib.gefen_gram_bf16_batched(xt.data_ptr(), xt.stride(1), xt.stride(0), out.data_ptr(), out.stride(1),
                                     out.stride(0), g, m, k, 1.0, torch.cuda.current_stream(xt.device).cuda_stream)
    _lib.check(rc, "gefen_gram_bf16_batched")


def newton_schulz_batched(x: torch.Tensor, coeffs: Tuple[float, float, float], steps: int,
                          eps: float, work: Optional[dict] = None, sumsq: Optional[torch.Tensor] = None,
                          index: Optional[torch.Tensor] = None, apply=None) -> Optional[torch.Tensor]:
    """Newton-Schulz of every matrix of a [G, rows, cols] bf16 stack; returns the
    [G, rows, cols] result.  x's values may be overwritten.

    work: a dict that keeps the intermediate buffers between calls with the same
    stack (allocated on first use); the result is then the same buffer on every
    call with the same number of steps.
    sumsq, index: the matrices' sums of squares, already gathered (float64 device
    tensor; matrix g's is sumsq[index[g]], int32 device index, or sumsq[g]), so
    the normalisation does not read the stack twice.
    apply: GefenMuon's update tasks of the stack's parameters (a MUON_APPLY_TASK
    array, one row per matrix, steps > 0): the last product is applied to them
    (gemm_nt_batched_apply) instead of returned, and the result is None."""
    a, b, c = coeffs
    if apply is not None and steps <= 0:
        raise ValueError("a fused update needs at least one Newton-Schulz step")
    g, rows, cols = x.shape
    transposed = rows > cols
    m, n = (cols, rows) if transposed else (rows, cols)  # X [m, n], m <= n
    if work is None:
        work = {}

    def buf(name, shape):
        t = work.get(name)
        if t is None or tuple(t.shape) != tuple(shape) or t.device != x.device:
            t = work[name] = torch.empty(shape, dtype=torch.bfloat16, device=x.device)
        return t

    # normalise each matrix, x /= max(||x||, eps) in bf16 (gefen_muon.py:37), as
    # X^T [G, n, m]: the stack itself for a transposed stack, its transpose else
    lib = _lib.load()
    with torch.cuda.device(x.device):
        stream = torch.cuda.current_stream(x.device).cuda_stream
        if sumsq is not None:
            xt = x if transposed else buf("xt", (g, n, m))
            _lib.check(lib.gefen_ns_normalize_sumsq(x.data_ptr(), None if transposed else xt.data_ptr(), g, rows, cols,
                                                    float(eps), sumsq.data_ptr(),
                                                    index.data_ptr() if index is not None else None,
                                                    0 if transposed else 1, stream), "gefen_ns_normalize_sumsq")
        else:
            other = buf("other", (g, cols, rows))
            _lib.check(lib.gefen_ns_prepare(x.data_ptr(), other.data_ptr(), g, rows, cols, float(eps), stream),
                       "gefen_ns_prepare")
            xt = x if transposed else other
    if steps == 0:
        if transposed:
            return xt
        out = buf("nx", (g, m, n))
        out.copy_(xt.transpose(1, 2))
        return out
    gram = buf("gram", (g, m, m))
    upd = buf("upd", (g, m, m))
    nxt = buf("t1", (g, n, m))  # X^T alternates between xt and this buffer
    with torch.cuda.device(x.device):
        for it in range(steps):
            gram_batched(xt, gram)                                                        # X X^T
            gemm_nt_batched(gram, gram, upd, d_t=gram, alpha=c, beta=b, symmetric=True)   # b A + c A A
            if it + 1 == steps and apply is not None:
                gemm_nt_batched_apply(upd, xt, xt, 1.0, a, apply)                        # p += adj * (a X + B X)
                return None
            if it + 1 < steps or transposed:
                gemm_nt_batched(upd, xt, None, out_t=nxt, d_t=xt, alpha=1.0, beta=a)      # (a X + B X)^T
                xt, nxt = nxt, xt
            else:
                nx = buf("nx", (g, m, n))
                gemm_nt_batched(upd, xt, nx, d_t=xt, alpha=1.0, beta=a)                   # a X + B X
                return nx
    return xt

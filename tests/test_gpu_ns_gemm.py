"""MFMA bf16 GEMM of the Newton-Schulz iteration against an fp32 PyTorch reference
of the same op (products in fp32 on the CPU, one bf16 rounding)."""

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref(a, b, b_kcontig, d, alpha, beta):
    af = a.float().cpu()
    bf = b.float().cpu()
    prod = af @ (bf.T if b_kcontig else bf)
    out = alpha * prod
    if beta != 0.0:
        out = out + beta * d.float().cpu()
    return out


@pytest.mark.parametrize("m,n,k,b_kcontig,alpha,beta", [
    (256, 256, 512, True, 1.0, 0.0),
    (128, 384, 128, False, 1.0, 3.4445),
    (200, 136, 72, True, 1.0, 0.0),       # ragged: not multiples of the tiles
    (96, 96, 96, False, 2.0315, -4.775),
    (1024, 1024, 2048, True, 1.0, 0.0),
    (64, 192, 64, False, 1.0, 3.4445),
])
def test_gemm_matches_fp32_reference(m, n, k, b_kcontig, alpha, beta):
    from gefen_amd.newton_schulz import gemm

    g = torch.Generator(device="cpu").manual_seed(m * 7 + n * 3 + k)
    a = torch.randn(m, k, generator=g).bfloat16().cuda()
    b = (torch.randn(n, k, generator=g) if b_kcontig else torch.randn(k, n, generator=g)).bfloat16().cuda()
    d = torch.randn(m, n, generator=g).bfloat16().cuda()
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda:0")
    gemm(a, b, b_kcontig, out, d=d if beta != 0.0 else None, alpha=alpha, beta=beta)
    ref = _ref(a, b, b_kcontig, d, alpha, beta)
    got = out.float().cpu()
    # fp32 accumulation in another order + one bf16 rounding: within 1 bf16 ulp of the
    # fp32 result plus the fp32 summation error bound (k * 2^-24 * sum |a||b|)
    bound = (a.float().abs().cpu() @ (b.float().abs().cpu().T if b_kcontig else b.float().abs().cpu())) * abs(alpha)
    tol = ref.abs() * 2.0 ** -8 + bound * k * 2.0 ** -24 + 1e-30
    assert bool(((got - ref).abs() <= tol).all()), float(((got - ref).abs() / tol).max())


def test_newton_schulz_matches_float64_restatement():
    from gefen_amd.newton_schulz import newton_schulz_bf16
    from oracle import oracle as orc

    g = torch.Generator(device="cpu").manual_seed(3)
    for shape in ((64, 96), (96, 64), (256, 128)):
        x = torch.randn(*shape, generator=g) * 1e-3
        got = newton_schulz_bf16(x.cuda(), (3.4445, -4.7750, 2.0315), 5, 1e-7).float().cpu().numpy()
        ref = orc.newton_schulz_bf16(x.numpy())
        # five bf16 rounds: agree to a few bf16 ulps of the O(1) singular directions
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel < 2e-2, (shape, rel)
        s = np.linalg.svd(got.astype(np.float64), compute_uv=False)
        assert s.max() < 1.3 and s.min() > 0.5, s  # quintic NS pushes singular values into ~[0.7, 1.2]


def _nt_batched(a, b, out, out_t=None, d=None, alpha=1.0, beta=0.0, symmetric=False, d_t=None):
    from gefen_amd.newton_schulz import gemm_nt_batched

    gemm_nt_batched(a, b, out, out_t=out_t, d=d, alpha=alpha, beta=beta, symmetric=symmetric, d_t=d_t)


@pytest.mark.parametrize("g,m,n,k,alpha,beta,sym,dt", [
    (3, 256, 512, 128, 1.0, 0.0, False, False),
    (2, 512, 256, 384, 1.7, -0.6, False, False),
    (2, 512, 768, 256, 1.0, 3.4445, False, True),
    (4, 512, 512, 768, 1.0, 0.0, True, False),
    (2, 768, 768, 768, 2.0315, -4.775, True, False),
    (2, 512, 512, 512, 2.0315, -4.775, True, True),
    (2, 768, 512, 128, 1.0, 0.75, False, True),          # two K steps, M > N, D given as D^T
    (2, 512, 768, 192, 1.0, -2.0, False, True),          # odd K step count
    (2, 512, 512, 1024, 2.0315, -4.775, True, True),
])
def test_batched_gemm_equals_one_matrix_gemm(g, m, n, k, alpha, beta, sym, dt):
    """The batched large-tile GEMM accumulates K in the same MFMA order as the
    one-matrix kernel: results are bit-identical, C^T is C transposed, and a
    symmetric product's mirrored tiles equal the computed ones."""
    from gefen_amd.newton_schulz import gemm

    gen = torch.Generator(device="cpu").manual_seed(g * 1000 + m + n + k)
    a = (torch.randn(g, m, k, generator=gen) * 0.05).bfloat16().cuda()
    if sym:
        b = a
        d = (a.float() @ a.float().transpose(1, 2)).bfloat16().contiguous()  # symmetric D
    else:
        b = (torch.randn(g, n, k, generator=gen) * 0.05).bfloat16().cuda()
        d = (torch.randn(g, m, n, generator=gen) * 0.05).bfloat16().cuda()
    out = torch.empty(g, m, n, dtype=torch.bfloat16, device="cuda:0")
    out_t = None if sym else torch.empty(g, n, m, dtype=torch.bfloat16, device="cuda:0")
    if dt and beta != 0.0:  # D passed as its transpose
        _nt_batched(a, b, out, out_t=out_t, d_t=d.transpose(1, 2).contiguous(), alpha=alpha, beta=beta,
                    symmetric=sym)
    else:
        _nt_batched(a, b, out, out_t=out_t, d=d if beta != 0.0 else None, alpha=alpha, beta=beta, symmetric=sym)
    ref = torch.empty_like(out)
    for i in range(g):
        gemm(a[i], b[i], True, ref[i], d=d[i] if beta != 0.0 else None, alpha=alpha, beta=beta)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    other = out if sym else out_t  # a symmetric product equals its transpose
    assert torch.equal(other.view(torch.int16), out.transpose(1, 2).contiguous().view(torch.int16))


@pytest.mark.parametrize("dt", [False, True])
def test_batched_gemm_without_transposed_output(dt):
    """C alone (no C^T, not symmetric), D row-major or given as D^T: bit-identical to
    the one-matrix kernel."""
    from gefen_amd.newton_schulz import gemm

    gen = torch.Generator(device="cpu").manual_seed(77 + dt)
    a = (torch.randn(3, 512, 256, generator=gen) * 0.05).bfloat16().cuda()
    b = (torch.randn(3, 768, 256, generator=gen) * 0.05).bfloat16().cuda()
    d = (torch.randn(3, 512, 768, generator=gen) * 0.05).bfloat16().cuda()
    out = torch.empty(3, 512, 768, dtype=torch.bfloat16, device="cuda:0")
    if dt:
        _nt_batched(a, b, out, d_t=d.transpose(1, 2).contiguous(), alpha=0.5, beta=-1.25)
    else:
        _nt_batched(a, b, out, d=d, alpha=0.5, beta=-1.25)
    ref = torch.empty_like(out)
    for i in range(3):
        gemm(a[i], b[i], True, ref[i], d=d[i], alpha=0.5, beta=-1.25)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_batched_gemm_rejects_untiled_shapes():
    from gefen_amd import _lib
    from gefen_amd.newton_schulz import gemm_nt_batched

    a = torch.zeros(2, 200, 64, dtype=torch.bfloat16, device="cuda:0")
    out = torch.empty(2, 200, 200, dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(ValueError):
        gemm_nt_batched(a, a, out, symmetric=True)
    b = torch.zeros(2, 256, 64, dtype=torch.bfloat16, device="cuda:0")
    out2 = torch.empty(2, 256, 512, dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(ValueError):  # symmetric needs a square product
        gemm_nt_batched(b, torch.zeros(2, 512, 64, dtype=torch.bfloat16, device="cuda:0"), out2, symmetric=True)
    sq = torch.empty(2, 256, 256, dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(ValueError):  # no separate transposed output for a symmetric product
        gemm_nt_batched(b, b, sq, out_t=torch.empty_like(sq), symmetric=True)
    assert _lib.GefenError is not None


@pytest.mark.parametrize("g,rows,cols", [(3, 256, 512), (2, 512, 256), (2, 256, 256)])
def test_batched_newton_schulz_matches_one_matrix_path(g, rows, cols):
    """Stacked Newton-Schulz equals the per-matrix path (same products, same
    rounding points) and the float64 restatement within the NS tolerance."""
    from gefen_amd.newton_schulz import newton_schulz_batched, newton_schulz_bf16
    from oracle import oracle as orc

    gen = torch.Generator(device="cpu").manual_seed(rows * 3 + cols)
    x = torch.randn(g, rows, cols, generator=gen) * 1e-3
    got = newton_schulz_batched(x.bfloat16().cuda(), (3.4445, -4.7750, 2.0315), 5, 1e-7)
    for i in range(g):
        one = newton_schulz_bf16(x[i].cuda(), (3.4445, -4.7750, 2.0315), 5, 1e-7)
        # the two paths differ only in how torch reduces the norm; when the bf16
        # norms agree the results are bit-identical
        d = (got[i].float() - one.float()).abs().max().item()
        assert d <= 2.0 ** -6, (i, d)
        ref = orc.newton_schulz_bf16(x[i].numpy())
        gi = got[i].float().cpu().numpy()
        rel = np.linalg.norm(gi - ref) / np.linalg.norm(ref)
        assert rel < 2e-2, (i, rel)


@pytest.mark.parametrize("g,m,k", [(3, 256, 512), (2, 512, 256), (2, 768, 1024), (1, 256, 64)])
def test_gram_from_transpose_equals_symmetric_product(g, m, k):
    """gefen_gram_bf16_batched(X^T) equals gefen_gemm_bf16_nt_batched(X, X,
    symmetric) bit for bit: the transposing LDS reads build the same MFMA
    operands in the same K order."""
    from gefen_amd.newton_schulz import gemm_nt_batched, gram_batched

    gen = torch.Generator(device="cpu").manual_seed(m + 7 * k + g)
    x = (torch.randn(g, m, k, generator=gen) * 0.05).bfloat16().cuda()
    xt = x.transpose(1, 2).contiguous()
    ref = torch.empty(g, m, m, dtype=torch.bfloat16, device="cuda:0")
    got = torch.empty_like(ref)
    gemm_nt_batched(x, x, ref, symmetric=True)
    gram_batched(xt, got)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def _newton_schulz_both_orientations(x, coeffs, steps, sumsq, index):
    """The scheme that kept X and X^T (normalisation writes both; B X writes both),
    composed from gefen_ns_prepare_sumsq and gefen_gemm_bf16_nt_batched."""
    from gefen_amd import _lib
    from gefen_amd.newton_schulz import gemm_nt_batched

    a, b, c = coeffs
    g, rows, cols = x.shape
    transposed = rows > cols
    other = torch.empty(g, cols, rows, dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    _lib.check(lib.gefen_ns_prepare_sumsq(x.data_ptr(), other.data_ptr(), g, rows, cols, 1e-7, sumsq.data_ptr(),
                                          index.data_ptr() if index is not None else None,
                                          torch.cuda.current_stream().cuda_stream))
    X, XT = (other, x) if transposed else (x, other)
    m, n = X.shape[1], X.shape[2]
    for _ in range(steps):
        gram = torch.empty(g, m, m, dtype=torch.bfloat16, device=x.device)
        upd = torch.empty_like(gram)
        gemm_nt_batched(X, X, gram, symmetric=True)
        gemm_nt_batched(gram, gram, upd, d_t=gram, alpha=c, beta=b, symmetric=True)
        nx = torch.empty(g, m, n, dtype=torch.bfloat16, device=x.device)
        nxt = torch.empty(g, n, m, dtype=torch.bfloat16, device=x.device)
        gemm_nt_batched(upd, XT, nx, out_t=nxt, d_t=XT, alpha=1.0, beta=a)
        X, XT = nx, nxt
    return XT if transposed else X


@pytest.mark.parametrize("g,rows,cols", [(3, 256, 512), (2, 512, 256), (2, 512, 768), (2, 768, 256)])
@pytest.mark.parametrize("steps", [0, 1, 2, 5])
def test_batched_newton_schulz_keeps_only_the_transpose_bit_exactly(g, rows, cols, steps):
    """newton_schulz_batched (X^T only between iterations, Gram product from X^T,
    normalisation in one orientation) equals the scheme that kept both
    orientations, bit for bit, for transposed and untransposed stacks and even
    and odd step counts."""
    from gefen_amd.newton_schulz import newton_schulz_batched

    gen = torch.Generator(device="cpu").manual_seed(rows * 5 + cols + steps)
    x0 = (torch.randn(g, rows, cols, generator=gen) * 1e-3).bfloat16().cuda()
    sumsq = torch.zeros(g * 128, dtype=torch.float64, device="cuda:0")
    sumsq.view(g, 8, 16)[:, 0, 0] = (x0.double() ** 2).sum(dim=(1, 2))
    index = torch.arange(g - 1, -1, -1, dtype=torch.int32, device="cuda:0")  # matrix i's sums are task g-1-i's
    sumsq_perm = torch.zeros_like(sumsq)
    sumsq_perm.view(g, 8, 16)[:, 0, 0] = sumsq.view(g, 8, 16)[:, 0, 0].flip(0)
    coeffs = (3.4445, -4.7750, 2.0315)
    ref = _newton_schulz_both_orientations(x0.clone(), coeffs, steps, sumsq, None)
    got = newton_schulz_batched(x0.clone(), coeffs, steps, 1e-7, sumsq=sumsq_perm, index=index)
    torch.cuda.synchronize()
    assert got.shape == ref.shape == x0.shape
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("dtype,transposed,wd,batch", [
    (torch.bfloat16, False, 0.1, 3),
    (torch.bfloat16, True, 0.0, 3),
    (torch.float32, False, 0.0, 2),
    (torch.float32, True, 0.1, 2),
    (torch.float16, True, 0.1, 2),
    (torch.bfloat16, True, 0.1, 70),   # two launches of at most 64 matrices
])
def test_fused_update_equals_product_then_apply(dtype, transposed, wd, batch):
    """gefen_gemm_bf16_nt_batched_apply (the last Newton-Schulz product applied as
    GefenMuon's update) equals storing the product with gefen_gemm_bf16_nt_batched
    and applying it with gefen_muon_apply_tasks, bit for bit, for every parameter
    dtype, both orientations and with / without weight decay."""
    import numpy as np
    from gefen_amd import _lib
    from gefen_amd.newton_schulz import gemm_nt_batched_apply

    m, n, k = (256, 512, 256) if batch <= 3 else (256, 256, 256)
    gen = torch.Generator(device="cpu").manual_seed(batch * 10 + int(transposed) + (wd > 0) * 100)
    a = (torch.randn(batch, m, k, generator=gen) * 0.05).bfloat16().cuda()
    b = (torch.randn(batch, n, k, generator=gen) * 0.05).bfloat16().cuda()
    d_t = (torch.randn(batch, n, m, generator=gen) * 0.05).bfloat16().cuda()
    shape = (n, m) if transposed else (m, n)
    p0 = (torch.randn(batch, *shape, generator=gen) * 0.02).to(dtype).cuda()
    p_fused, p_ref = p0.clone(), p0.clone()

    def tasks(params, update):
        t = np.zeros(batch, dtype=_lib.MUON_APPLY_TASK)
        for i in range(batch):
            t[i]["p"] = params[i].data_ptr()
            t[i]["update"] = update[i].data_ptr() if update is not None else 0
            t[i]["numel"] = params[i].numel()
            t[i]["param_dtype"] = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dtype]
            t[i]["transposed"] = 1 if transposed else 0
            t[i]["lr"] = 0.02
            t[i]["weight_decay"] = wd
            t[i]["adjusted_lr"] = 0.02 * 0.2 * math.sqrt(max(m, n))
        return t

    gemm_nt_batched_apply(a, b, d_t, 1.0, 3.4445, tasks(p_fused, None))
    if transposed:
        u = torch.empty(batch, n, m, dtype=torch.bfloat16, device="cuda:0")
        _nt_batched(a, b, None, out_t=u, d_t=d_t, alpha=1.0, beta=3.4445)
    else:
        u = torch.empty(batch, m, n, dtype=torch.bfloat16, device="cuda:0")
        _nt_batched(a, b, u, d_t=d_t, alpha=1.0, beta=3.4445)
    t = tasks(p_ref, u)
    _lib.check(_lib.load().gefen_muon_apply_tasks(t.ctypes.data, batch, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert not torch.equal(p_fused, p0)
    assert torch.equal(p_fused.view(torch.uint8), p_ref.view(torch.uint8))

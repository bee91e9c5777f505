"""Randomised shapes for the Newton-Schulz GEMMs.

The one-matrix kernel (gefen_gemm_bf16: C = alpha A op(B) + beta D, one bf16
rounding) over 40 random (m, n, k) from 1 to 700, both operand layouts, with
and without D: every element within one bf16 ulp of the float64 result plus the
float32 accumulation bound (k + 2) 2^-24 sum|terms| (half a bf16 ulp is at most
2^-8 of the value).  The batched tile kernel over random stacks of 256-multiple
shapes (symmetric or not, with D or D^T, with and without the transposed copy
of a non-symmetric product): bit-identical to the one-matrix kernel on every
matrix (both use the same MFMA K order)."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", [1, 2])
def test_random_one_matrix_gemm_shapes(seed):
    from gefen_amd.newton_schulz import gemm

    rng = np.random.default_rng(seed)
    g = torch.Generator(device="cpu").manual_seed(seed)
    worst = 0.0
    for case in range(40):
        m, n, k = (int(rng.integers(1, 701)) for _ in range(3))
        b_kcontig = bool(rng.integers(2))
        with_d = bool(rng.integers(2))
        alpha = float(rng.choice([1.0, 2.0315, -0.5]))
        beta = float(rng.choice([3.4445, -4.775, 1.0])) if with_d else 0.0
        a = torch.randn(m, k, generator=g).bfloat16()
        b = (torch.randn(n, k, generator=g) if b_kcontig else torch.randn(k, n, generator=g)).bfloat16()
        d = torch.randn(m, n, generator=g).bfloat16()
        out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda:0")
        gemm(a.cuda(), b.cuda(), b_kcontig, out, d=d.cuda() if with_d else None, alpha=alpha, beta=beta)
        af, bf, df = a.double(), b.double(), d.double()
        bm = bf.T if b_kcontig else bf
        exact = alpha * (af @ bm) + (beta * df if with_d else 0.0)
        terms = abs(alpha) * (af.abs() @ bm.abs()) + (abs(beta) * df.abs() if with_d else 0.0)
        got = out.cpu().double()
        tol = exact.abs() * 2.0 ** -8 + terms * (k + 2) * 2.0 ** -24 + 1e-37
        ratio = float(((got - exact).abs() / tol).max())
        worst = max(worst, ratio)
        assert ratio <= 1.0, (case, m, n, k, b_kcontig, with_d, ratio)
    print("seed", seed, "40 one-matrix GEMM shapes within the bound (worst {:.3f} of it)".format(worst), flush=True)


@pytest.mark.parametrize("seed", [3, 4])
def test_random_batched_gemm_equals_one_matrix_gemm(seed):
    from gefen_amd.newton_schulz import gemm, gemm_nt_batched

    rng = np.random.default_rng(seed)
    g = torch.Generator(device="cpu").manual_seed(seed)
    for case in range(8):
        batch = int(rng.integers(1, 5))
        m = 256 * int(rng.integers(1, 4))
        sym = bool(rng.random() < 0.4)
        n = m if sym else 256 * int(rng.integers(1, 4))
        k = 64 * int(rng.integers(1, 17))
        dmode = ["none", "d", "dt"][rng.integers(3)]
        want_t = not sym and bool(rng.integers(2))   # a symmetric product writes its mirror into C
        alpha, beta = float(rng.choice([1.0, 2.0315])), (float(rng.choice([3.4445, -4.775])) if dmode != "none" else 0.0)
        if sym:   # A A^T-type products: B = A (the kernel mirrors the upper tiles)
            a = torch.randn(batch, m, k, generator=g).bfloat16().cuda()
            b = a
        else:
            a = torch.randn(batch, m, k, generator=g).bfloat16().cuda()
            b = torch.randn(batch, n, k, generator=g).bfloat16().cuda()
        d = torch.randn(batch, m, n, generator=g).bfloat16().cuda()
        if sym:
            d = (d + d.transpose(1, 2)).contiguous()   # a symmetric D, as the Newton-Schulz products have
        out = torch.empty(batch, m, n, dtype=torch.bfloat16, device="cuda:0")
        out_t = torch.empty(batch, n, m, dtype=torch.bfloat16, device="cuda:0") if want_t else None
        kw = {}
        if dmode == "d":
            kw["d"] = d
        elif dmode == "dt":
            kw["d_t"] = d.transpose(1, 2).contiguous()
        gemm_nt_batched(a, b, out, out_t=out_t, alpha=alpha, beta=beta, symmetric=sym, **kw)
        torch.cuda.synchronize()
        for i in range(batch):
            one = torch.empty(m, n, dtype=torch.bfloat16, device="cuda:0")
            gemm(a[i], b[i], True, one, d=d[i] if dmode != "none" else None, alpha=alpha, beta=beta)
            torch.cuda.synchronize()
            tag = (case, batch, m, n, k, sym, dmode, want_t, i)
            assert torch.equal(out[i].view(torch.int16), one.view(torch.int16)), tag
            if want_t:
                assert torch.equal(out_t[i].view(torch.int16), one.T.contiguous().view(torch.int16)), tag
    print("seed", seed, "8 random stacks equal the one-matrix kernel bit for bit", flush=True)

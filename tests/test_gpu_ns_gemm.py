"""MFMA bf16 GEMM of the Newton-Schulz iteration against an fp32 PyTorch reference
of the same op (products in fp32 on the CPU, one bf16 rounding)."""

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

"""Randomised parity of the first Gefen step (period detection, gradient
histograms, exact DP codebook) with the CPU oracle.

Each case builds ~50 parameters of random sizes (rich divisor sets, primes,
tiny tensors), dtypes (bf16, f16, f32) and gradient structure (rows of a random
divisor length with their own scale, plain normal values, zero blocks) and
takes one Gefen step on the GPU.  Every tensor's automatic period must equal
oracle.find_period (gefen.py:765-828 on the CPU backend) and the learned
codebook must equal oracle.learn_codebook (gefen.py:305-419) bit for bit."""

import numpy as np
import pytest
import torch

import gpu_util as gu
from gefen_amd import synthetic as syn
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SIZES = [1, 2, 3, 7, 12, 31, 64, 97, 360, 768, 1000, 1021, 2304, 4096, 5040, 6144, 7919, 9216, 10080, 12288,
         20000, 27720, 32768, 45045, 55440, 65536, 98304, 110880, 131072, 196608, 262144]


def _case(rng, count):
    out = []
    for i in range(count):
        dt = ["bf16", "bf16", "f16", "f32"][rng.integers(4)]
        n = int(SIZES[rng.integers(len(SIZES))])
        divs = orc.divisors(n)
        kind = rng.integers(3)
        e_lo = int(rng.integers(-18, -8))
        e_hi = e_lo + int(rng.integers(1, 9))
        if kind == 0 and len(divs) > 2:
            cols = int(divs[rng.integers(1, len(divs))])   # rows of a random divisor length
            g = syn.row_scaled_normal(9000 + i, 1, n // cols, cols, e_lo, e_hi).reshape(-1)
        else:
            g = syn.row_scaled_normal(9000 + i, 1, 1, n, e_lo, e_hi).reshape(-1)
        if kind == 2 and n >= 8:
            g = g.copy()
            g[: n // 4] = 0.0                               # a zeroed quarter
        gb = syn.round_to(g, dt)
        out.append((dt, n, gb.view(np.uint16) if gb.dtype == np.float16 else gb))
    return out


@pytest.mark.parametrize("seed", [3, 31, 314])
def test_random_first_step_periods_and_codebook_match_oracle(seed):
    from gefen_amd.gefen import Gefen

    rng = np.random.default_rng(seed)
    case = _case(rng, 50)
    print("seed", seed, "tensors", len(case), "elements", sum(n for _, n, _ in case), flush=True)
    params = []
    for i, (dt, n, g) in enumerate(case):
        p = torch.nn.Parameter(torch.zeros(n, dtype=gu.TORCH[dt], device="cuda:0"))
        p.grad = gu.to_dev(g, dt)
        params.append(("t{}".format(i), p))
    opt = Gefen(params)
    opt.step()
    torch.cuda.synchronize()
    got = [opt.state[p]["automatic_period"] for _, p in params]
    want = [orc.find_period(g, dt) for dt, _, g in case]
    bad = [(i, case[i][0], case[i][1], a, b) for i, (a, b) in enumerate(zip(got, want)) if a != b]
    assert not bad, bad
    cb = opt._gefen_codebook.detach().cpu().numpy()
    ref = orc.learn_codebook([(g, dt, P) for (dt, _, g), P in zip(case, want)])
    np.testing.assert_array_equal(cb, ref)
    print("seed", seed, "periods", sorted(set(got)), "and the codebook match the oracle", flush=True)

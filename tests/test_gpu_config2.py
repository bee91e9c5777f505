"""BASELINE config 2 at full size: one fp32 tensor of 8192 x 8192 values 1e-3 *
Student-t(3).  Period scores and choice, the exact histogram, the exact-DP
codebook, the first Gefen step (indices, magnitudes, vmean, parameters) and the
Lloyd-Max counts against the C oracle on byte-identical inputs (the device
generator writes the tensor; the oracle reads a host copy of the same bytes)."""

import numpy as np
import pytest
import torch

import gpu_util as gu
from gefen_amd import synthetic as syn
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

N = 8192 * 8192


def test_config2_first_step_pipeline_at_full_size():
    from gefen_amd.gefen import Gefen
    from gefen_amd.kernels.exact_histogram_fused import gefen_exact_histogram_cuda
    from gefen_amd.kernels.lloyd_max_fused import gefen_lloyd_accumulate_cuda
    from gefen_amd.kernels.period_variance import period_scores_launch, period_scores_workspace_bytes
    from gefen_amd.partitioning import candidate_divisors
    from gefen_amd.quantization import exact_dp_from_counts

    print("config 2: 64M fp32 Student-t", flush=True)
    g = torch.empty(8192, 8192, dtype=torch.float32, device="cuda:0")
    syn.fill_device(g, 2026, 2, syn.KIND_STUDENT_T3, mult=1e-3)
    p = torch.empty(8192, 8192, dtype=torch.float32, device="cuda:0")
    syn.fill_device(p, 2026, 3, syn.KIND_NORMAL, mult=0.02)
    gh = g.cpu().numpy().reshape(-1)
    ph = p.cpu().numpy().reshape(-1)

    # period scores of every candidate divisor, and the choice
    divs = candidate_divisors(N)
    ws = torch.empty(period_scores_workspace_bytes(N, divs), dtype=torch.uint8, device="cuda:0")
    sc = torch.empty(len(divs) + 1, dtype=torch.float64, device="cuda:0")
    period_scores_launch(g.view(-1), divs, 1, 1e-12, sc, ws)
    ref_scores = orc.period_scores(gh, "f32", divs, mode=1)
    np.testing.assert_allclose(sc.cpu().numpy()[:-1], ref_scores, rtol=1e-11, atol=0)
    period = orc.finalize_period(list(zip(divs, ref_scores.tolist())), N)

    # exact histogram and the exact-DP codebook
    counts = torch.zeros(4096, dtype=torch.int64, device="cuda:0")
    gefen_exact_histogram_cuda(g.view(-1), period, counts)
    ref_counts = orc.histogram(gh, "f32", period)
    np.testing.assert_array_equal(counts.cpu().numpy(), ref_counts)
    cb = exact_dp_from_counts(counts.float(), 256, True).cpu().numpy()
    ref_cb = orc.exact_dp(ref_counts.astype(np.float32), 256, True)
    np.testing.assert_array_equal(cb, ref_cb)

    # the first Gefen step end to end (period detection and codebook learning included)
    p.requires_grad_(True)
    p.grad = g
    opt = Gefen([("w", p)])
    opt.step()
    st = opt.state[p]
    assert st["automatic_period"] == period
    np.testing.assert_array_equal(opt._gefen_codebook.cpu().numpy(), ref_cb)
    ost = orc.TensorState(N, period, "f32", "f32")
    pr = ph.copy()
    pod = orc.largest_divisor_at_most(N, 256) if period == 1 else 0
    rc = orc.lib().orc_gefen_step(0, 0, orc._ptr(pr), orc._ptr(gh), orc._ptr(ost.m_codebook),
                                  orc._ptr(ost.m_magnitude), orc._ptr(ost.vmean), N, period, pod, orc._ptr(ref_cb), 256,
                                  0.9, 0.999, 1e-3, 1e-8, 0.0, 1 - 0.9, 1 - 0.999, 16)
    assert rc == 0
    np.testing.assert_array_equal(gu.to_np(st["m_codebook"]).reshape(-1), ost.m_codebook)
    np.testing.assert_array_equal(gu.to_np(st["m_magnitude"]).reshape(-1), ost.m_magnitude)
    np.testing.assert_allclose(gu.to_np(st["vmean"]).reshape(-1), ost.vmean, rtol=4e-6, atol=0)
    np.testing.assert_allclose(gu.to_np(p).reshape(-1), pr, rtol=1e-5, atol=1e-7)

    # Lloyd-Max counts with the learned codebook: nearest codeword of each
    # block-normalised value (exact), sums to fp32 accumulation tolerance
    sums = torch.zeros(256, dtype=torch.float32, device="cuda:0")
    lcounts = torch.zeros(256, dtype=torch.int64, device="cuda:0")
    gefen_lloyd_accumulate_cuda(g.view(-1), torch.from_numpy(ref_cb).to("cuda:0"), period, sums, lcounts)
    rows = gh.reshape(-1, period)
    amax = np.abs(rows).max(axis=1, keepdims=True)
    x = np.where(amax > 0, rows / np.where(amax > 0, amax, 1), 0).astype(np.float32).reshape(-1)
    idx = orc.nearest(ref_cb, x)
    np.testing.assert_array_equal(lcounts.cpu().numpy(), np.bincount(idx, minlength=256))
    ref_sums = np.bincount(idx, weights=x.astype(np.float64), minlength=256)
    np.testing.assert_allclose(sums.cpu().numpy(), ref_sums, rtol=1e-3, atol=1e-1)
    assert int(lcounts.sum()) == N

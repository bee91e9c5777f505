"""First-step kernels on the GPU: histogram, exact DP, period scores, Lloyd-Max,
block variance, the GefenMuon momentum entry point and the device twin of the
synthetic generator."""

import numpy as np
import pytest
import torch

import gpu_util as gu
import traj_util as tu
from golden_util import load
from gefen_amd import synthetic as syn
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def test_device_generator_matches_numpy():
    for dt in ("f32", "bf16"):
        t = torch.empty(3 * 1000, dtype=gu.TORCH[dt], device="cuda:0")
        syn.fill_device(t, 5, 9, syn.KIND_ROW_SCALED, cols=1000, e_lo=-14, e_hi=-4)
        ref = syn.round_to(syn.row_scaled_normal(5, 9, 3, 1000, -14, -4), dt).reshape(-1)
        np.testing.assert_array_equal(gu.to_np(t), ref)
        syn.fill_device(t, 5, 10, syn.KIND_STUDENT_T3, mult=1e-3)
        ref = syn.round_to(syn.student_t3(syn.make_key(5, 10), t.numel()) * 1e-3, dt)
        np.testing.assert_array_equal(gu.to_np(t), ref)
        syn.fill_device(t, 5, 11, syn.KIND_NORMAL, mult=0.02)
        ref = syn.round_to(syn.normal(syn.make_key(5, 11), t.numel()) * 0.02, dt)
        np.testing.assert_array_equal(gu.to_np(t), ref)


@pytest.mark.parametrize("dt,n,period", [("f32", 64 * 1000, 1000), ("bf16", 96 * 768, 768), ("bf16", 4096, 1),
                                         ("f16", 300 * 7, 7), ("f32", 5 * 70000, 70000)])
def test_histogram_is_bit_exact(dt, n, period):
    from gefen_amd.kernels.exact_histogram_fused import gefen_exact_histogram_cuda

    g = syn.round_to(syn.row_scaled_normal(21, n, n // period, period, -14, -4), dt).reshape(-1)
    g = g.view(np.uint16) if g.dtype == np.float16 else g
    counts = torch.zeros(4096, dtype=torch.int64, device="cuda:0")
    gefen_exact_histogram_cuda(gu.to_dev(g, dt), period, counts)
    ref = orc.histogram(g, dt, period)
    np.testing.assert_array_equal(counts.cpu().numpy(), ref)
    assert int(counts.sum()) == n


def test_histogram_accumulates_and_handles_zero_blocks():
    from gefen_amd.kernels.exact_histogram_fused import gefen_exact_histogram_cuda

    g = np.zeros(64, np.float32)
    g[32:] = np.linspace(-1, 1, 32, dtype=np.float32)
    counts = torch.full((4096,), 5, dtype=torch.int64, device="cuda:0")
    gefen_exact_histogram_cuda(gu.to_dev(g, "f32"), 32, counts)
    ref = orc.histogram(g, "f32", 32, counts=np.full(4096, 5, np.int64))
    np.testing.assert_array_equal(counts.cpu().numpy(), ref)
    assert int(counts[2048]) == 5 + 32  # the all-zero block lands in the middle bin


def test_exact_dp_matches_reference_fixtures():
    from gefen_amd.quantization import exact_dp_from_counts

    data, meta = load("exact_dp")
    for case in meta:
        if case["kind"] != "exact_dp":
            continue
        name = case["name"]
        counts = torch.from_numpy(data[name + "/counts"]).to("cuda:0")
        cb = exact_dp_from_counts(counts, int(data[name + "/k"]), bool(data[name + "/force"]))
        np.testing.assert_array_equal(cb.cpu().numpy(), data[name + "/codebook"], err_msg=name)


def test_exact_dp_full_histogram_matches_oracle():
    """A dense 4096-bin histogram (about 3000 active bins, K = 256) against the C oracle."""
    from gefen_amd.quantization import exact_dp_from_counts

    g = syn.round_to(syn.student_t3(syn.make_key(4, 4), 1 << 20) * 1e-3, "f32")
    counts = orc.histogram(g, "f32", 1024).astype(np.float32)
    ref = orc.exact_dp(counts, 256, True)
    got = exact_dp_from_counts(torch.from_numpy(counts).to("cuda:0"), 256, True).cpu().numpy()
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("case", ["sparse_k256", "sparse_k16_free", "edges_k64", "few_bins_padded"])
def test_exact_dp_sparse_histograms_match_oracle(case):
    """Histograms whose active bins are scattered over the 4096 bins (runs of
    empty bins across the init kernel's per-thread bin ranges of 16, active
    first and last bins, fewer active bins than codebook entries), against the
    C oracle: the compaction keeps bin order and the prefix sums stay sequential."""
    from gefen_amd.quantization import exact_dp_from_counts

    rng = np.random.default_rng(17)
    counts = np.zeros(4096, np.float32)
    if case in ("sparse_k256", "sparse_k16_free"):
        active = rng.random(4096) < 0.3
        active[rng.integers(0, 4096 - 200):][:200] = False  # a long empty run
        counts[active] = rng.integers(1, 5000, int(active.sum())).astype(np.float32)
        k, force = (256, True) if case == "sparse_k256" else (16, False)
    elif case == "edges_k64":
        counts[[0, 15, 16, 17, 1000, 2047, 2048, 4080, 4095]] = [3, 1, 7, 2, 9, 4, 4, 5, 6]
        counts[np.arange(100, 4000, 37)] = rng.integers(1, 50, len(range(100, 4000, 37)))
        k, force = 64, True
    else:
        counts[[5, 300, 301, 3000]] = [2, 8, 1, 4]
        k, force = 16, True
    ref = orc.exact_dp(counts, k, force)
    got = exact_dp_from_counts(torch.from_numpy(counts).to("cuda:0"), k, force).cpu().numpy()
    np.testing.assert_array_equal(got, ref, err_msg=case)


def test_learned_codebook_pipeline_matches_reference():
    from gefen_amd.gefen import learn_gefen_exact_codebook_from_grad_periods

    data, meta = load("exact_dp")
    for case in meta:
        if case["kind"] != "pipeline":
            continue
        name = case["name"]
        gp = []
        for ti in range(case["ntensors"]):
            g = data["{}/grad{}".format(name, ti)]
            dt = "bf16" if g.dtype == np.uint16 else "f32"
            t = gu.to_dev(g.reshape(-1), dt)
            gp.append(("t{}".format(ti), t, int(data["{}/period{}".format(name, ti)]), t))
        cb = learn_gefen_exact_codebook_from_grad_periods(grad_periods=iter(gp), codebook_device=torch.device("cuda:0"),
                                                          num_codebooks=256, force_endpoints=True, verbose=False,
                                                          compute_mse_logging=False)
        np.testing.assert_array_equal(cb.cpu().numpy(), data[name + "/codebook"], err_msg=name)


def test_period_choice_matches_reference_fixtures():
    from gefen_amd.partitioning import PeriodScorer, candidate_divisors
    from gefen_amd.kernels.period_variance import period_scores_launch, period_scores_workspace_bytes

    data, meta = load("periods")
    scorer = PeriodScorer(mode=1)
    for case in meta:
        g = data[case["name"] + "/grad"]
        scorer.add(gu.to_dev(g.reshape(-1), case["dtype"]))
    got = scorer.finish()
    assert got == [c["period"] for c in meta]
    # raw scores against the reference's numpy scores
    for case in meta:
        g = data[case["name"] + "/grad"]
        divs = data[case["name"] + "/divisors"].tolist()
        if not divs:
            continue
        t = gu.to_dev(g.reshape(-1), case["dtype"])
        ws = torch.empty(period_scores_workspace_bytes(t.numel(), divs), dtype=torch.uint8, device="cuda:0")
        sc = torch.empty(len(divs) + 1, dtype=torch.float64, device="cuda:0")
        period_scores_launch(t, divs, 1, 1e-12, sc, ws)
        s = sc.cpu().numpy()
        np.testing.assert_allclose(s[:-1], data[case["name"] + "/scores"], rtol=1e-12, atol=0, err_msg=case["name"])
        assert s[-1] == 0


def test_period_scores_large_tensor_match_oracle():
    from gefen_amd.partitioning import candidate_divisors
    from gefen_amd.kernels.period_variance import period_scores_launch, period_scores_workspace_bytes

    n = 2048 * 1536
    t = torch.empty(n, dtype=torch.bfloat16, device="cuda:0")
    syn.fill_device(t, 8, 8, syn.KIND_ROW_SCALED, cols=1536, e_lo=-17, e_hi=-7)
    divs = candidate_divisors(n)
    ws = torch.empty(period_scores_workspace_bytes(n, divs), dtype=torch.uint8, device="cuda:0")
    sc = torch.empty(len(divs) + 1, dtype=torch.float64, device="cuda:0")
    period_scores_launch(t, divs, 1, 1e-12, sc, ws)
    ref = orc.period_scores(gu.to_np(t), "bf16", divs, mode=1)
    np.testing.assert_allclose(sc.cpu().numpy()[:-1], ref, rtol=1e-11, atol=0)


def test_adjacent_log_block_mean_difference_entry_point():
    from gefen_amd.kernels.period_variance import average_adjacent_log_block_mean_difference_cuda_kernel as f

    g = syn.round_to(syn.row_scaled_normal(2, 2, 40, 96, -14, -4), "f32").reshape(-1)
    a = np.abs(g)
    got = f(gu.to_dev(a, "f32"), 96, input_is_squared=True, epsilon=1e-12)
    ref = orc.period_scores(a, "f32", [96], mode=0)[0]
    assert abs(got - ref) <= 1e-12 * abs(ref)
    got = f(gu.to_dev(g, "f32"), 96, input_is_squared=False, epsilon=1e-12)
    ref = orc.period_scores(g, "f32", [96], mode=2)[0]
    assert abs(got - ref) <= 1e-12 * abs(ref)
    with pytest.raises(RuntimeError, match="positive before log"):
        f(gu.to_dev(-np.ones(8, np.float32), "f32"), 2, input_is_squared=True, epsilon=1e-12)


def test_block_variance_and_cov_entry_points():
    """Against the oracle's float64 restatement of the reference's CUDA scorers
    (period_variance_kernel.cu:13-106): the kernels sum each block in float32, so
    each block variance may differ by the float32 summation bound
    2 P 2^-24 (E[x^2] + 2 mean^2)."""
    from gefen_amd.kernels.period_variance import (average_within_block_coefficient_of_variation_cuda_kernel,
                                                   average_within_block_variance_cuda_kernel)

    for dt, rows, period in (("f32", 50, 64), ("bf16", 40, 300), ("f16", 30, 2048)):
        g = tu.bits(syn.round_to(syn.row_scaled_normal(3, rows, rows, period, -7, -2), dt).reshape(-1))
        t = gu.to_dev(g, dt)
        x = (orc.to_f32(g, dt) ** 2).astype(np.float64).reshape(rows, period)
        m, m2 = x.mean(1), (x * x).mean(1)
        var = np.maximum(m2 - m * m, 0)
        dvar = 2 * period * 2.0 ** -24 * (m2 + 2 * m * m)
        ref = orc.block_variance(g, dt, period, False, False)[0]
        got = average_within_block_variance_cuda_kernel(t, period, input_is_squared=False)
        assert abs(got - ref) <= dvar.mean() / (2 * ref) + 1e-15, (dt, got, ref)
        cov = orc.block_variance(g, dt, period, False, True)
        got = average_within_block_coefficient_of_variation_cuda_kernel(t, period, input_is_squared=False)
        # d(sqrt(var)/m) <= dvar / (2 sqrt(var) m) + sqrt(var) dm / m^2, dm <= P 2^-24 m
        dcov = (dvar / (2 * np.sqrt(np.maximum(var, 1e-300)) * m) + np.sqrt(var) * period * 2.0 ** -24 / m).mean()
        assert abs(got - cov[0] / cov[1]) <= dcov, (dt, got, cov)
    with pytest.raises(RuntimeError, match="non-negative block means"):
        average_within_block_coefficient_of_variation_cuda_kernel(gu.to_dev(-np.ones(8, np.float32), "f32"), 4,
                                                                  input_is_squared=True)


@pytest.mark.parametrize("case", ["plain", "nonfinite", "beyond_last"])
def test_lloyd_accumulate_and_mse(case):
    """gefen_lloyd_accumulate / gefen_lloyd_mse against the oracle's restatement of
    the reference's CUDA semantics (lloyd_max_fused_kernel.cu:17-195): counts
    bit-exact, float32 sums within the summation bound n_k 2^-24 sum|x|_k.
    "nonfinite": NaN elements (the block absmax skips them, the element counts at
    index 0) and an inf element; "beyond_last": a codebook ending below the
    largest normalised value with a repeated last entry."""
    from gefen_amd.kernels.lloyd_max_fused import gefen_lloyd_accumulate_cuda, gefen_lloyd_mse_cuda

    data, _ = load("exact_dp")
    cb = data["hist_k256_forced/codebook"]
    period, rows = 128, 30
    g = syn.round_to(syn.row_scaled_normal(6, 6, rows, period, -14, -4), "f32").reshape(-1).copy()
    if case == "nonfinite":
        g[3 * period + 5] = np.nan
        g[3 * period + 70] = np.nan
        g[8 * period + 1] = np.inf
        g[12 * period:13 * period] = 0.0
    if case == "beyond_last":
        cb = np.concatenate([cb[:200], cb[199:200]]).astype(np.float32)  # ends at cb[199] < 1, repeated
    sums = torch.zeros(cb.size, dtype=torch.float32, device="cuda:0")
    counts = torch.zeros(cb.size, dtype=torch.int64, device="cuda:0")
    cbd = torch.from_numpy(cb).to("cuda:0")
    gefen_lloyd_accumulate_cuda(gu.to_dev(g, "f32"), cbd, period, sums, counts)
    ref_sums, ref_counts = orc.lloyd_accumulate(g, "f32", period, cb)
    np.testing.assert_array_equal(counts.cpu().numpy(), ref_counts)
    got = sums.cpu().numpy().astype(np.float64)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref_sums))
    ok = ~np.isnan(ref_sums)
    # |x| <= 1, so sum|x|_k <= n_k: float32 summation in any order stays within n_k^2 2^-24
    bound = ref_counts[ok].astype(np.float64) ** 2 * 2.0 ** -24
    assert np.all(np.abs(got[ok] - ref_sums[ok]) <= bound)
    new = (cb * np.float32(0.97)).astype(np.float32)
    mn = torch.zeros(1, dtype=torch.float32, device="cuda:0")
    mo = torch.zeros(1, dtype=torch.float32, device="cuda:0")
    gefen_lloyd_mse_cuda(gu.to_dev(g, "f32"), cbd, torch.from_numpy(new).to("cuda:0"), period, mn, mo)
    rn, ro = orc.lloyd_mse(g, "f32", period, cb, new)
    if case == "nonfinite":
        assert np.isnan(mn.item()) and np.isnan(ro) and np.isnan(rn) and np.isnan(mo.item())
    else:
        n = g.size
        assert abs(mn.item() - rn) <= n * 2.0 ** -24 * rn
        assert abs(mo.item() - ro) <= n * 2.0 ** -24 * ro


@pytest.mark.parametrize("dt,period", [("bf16", 64), ("f32", 32), ("bf16", 5000)])
def test_muon_momentum_entry_point_is_bit_exact(dt, period):
    from gefen_amd.kernels.automatic_gefen_fused import automatic_gefen_muon_momentum_cuda

    data, _ = load("exact_dp")
    cb = data["hist_k256_forced/codebook"]
    rows = 12
    n = rows * period
    st = orc.TensorState(n, period, dt, dt)
    idx = torch.zeros(rows, period, dtype=torch.uint8, device="cuda:0")
    mag = torch.zeros(rows, 1, dtype=gu.TORCH[dt], device="cuda:0")
    for step in range(1, 4):
        g = syn.round_to(syn.row_scaled_normal(9, step, rows, period, -12, -8), dt).reshape(-1)
        out = torch.empty(rows, period, dtype=gu.TORCH[dt], device="cuda:0")
        automatic_gefen_muon_momentum_cuda(gu.to_dev(g, dt).reshape(rows, period), idx, mag,
                                           torch.from_numpy(cb).to("cuda:0"), out, False, 0.95)
        ref = orc.muon_momentum(g, dt, st, cb, 0.95, False)
        np.testing.assert_array_equal(gu.to_np(idx).reshape(-1), st.m_codebook)
        np.testing.assert_array_equal(gu.to_np(mag).reshape(-1), st.m_magnitude)
        np.testing.assert_array_equal(gu.to_np(out).reshape(-1), ref)


def test_single_tensor_entry_points_match_oracle():
    """vmean + from_vmean (P > 1) and period1 entry points vs the oracle's step."""
    from gefen_amd.kernels.automatic_gefen_fused import (automatic_gefen_fused_update_from_vmean_cuda,
                                                         automatic_gefen_period1_update_cuda)
    from gefen_amd.kernels.automatic_vmean import automatic_vmean_update_cuda

    data, _ = load("exact_dp")
    cb = data["hist_k256_forced/codebook"]
    cbd = torch.from_numpy(cb).to("cuda:0")
    # P > 1
    R, P = 16, 384
    p = syn.round_to(syn.normal(syn.make_key(1, 2), R * P) * 0.02, "f32")
    g = syn.round_to(syn.row_scaled_normal(1, 3, R, P, -14, -4), "f32").reshape(-1)
    pd, gd = gu.to_dev(p, "f32"), gu.to_dev(g, "f32").reshape(R, P)
    idx = torch.zeros(R, P, dtype=torch.uint8, device="cuda:0")
    mag = torch.zeros(R, 1, device="cuda:0")
    v = torch.zeros(R, 1, device="cuda:0")
    automatic_vmean_update_cuda(v, gd, 0.999)
    automatic_gefen_fused_update_from_vmean_cuda(pd, gd, idx, mag, v, cbd, False, 0.9, 1e-3, 0.1, 1 - 0.999, 1e-8)
    st = orc.TensorState(R * P, P, "f32", "f32")
    orc.lib().orc_gefen_step(0, 0, orc._ptr(p), orc._ptr(g), orc._ptr(st.m_codebook), orc._ptr(st.m_magnitude),
                             orc._ptr(st.vmean), R * P, P, 0, orc._ptr(cb), 256, 0.9, 0.999, 1e-3, 1e-8, 0.0, 0.1,
                             1 - 0.999, 1)
    np.testing.assert_array_equal(gu.to_np(idx).reshape(-1), st.m_codebook)
    np.testing.assert_array_equal(gu.to_np(mag).reshape(-1), st.m_magnitude)
    np.testing.assert_allclose(gu.to_np(v).reshape(-1), st.vmean, rtol=4e-6)
    np.testing.assert_allclose(gu.to_np(pd), p, rtol=1e-5, atol=1e-7)
    # P = 1
    n = 2000
    p = syn.round_to(syn.normal(syn.make_key(1, 4), n) * 0.02, "bf16")
    g = syn.round_to(syn.row_scaled_normal(1, 5, 1, n, -14, -4), "bf16").reshape(-1)
    pod = orc.largest_divisor_at_most(n, 256)
    pd, gd = gu.to_dev(p, "bf16"), gu.to_dev(g, "bf16")
    idx = torch.zeros(n, 1, dtype=torch.uint8, device="cuda:0")
    mag = torch.zeros(n // pod, 1, dtype=torch.bfloat16, device="cuda:0")
    v = torch.zeros(n, 1, dtype=torch.bfloat16, device="cuda:0")
    automatic_gefen_period1_update_cuda(pd, gd, idx, mag, v, cbd, pod, 0.9, 0.999, 1e-3, 0.1, 1 - 0.999, 1e-8)
    st = orc.TensorState(n, 1, "bf16", "bf16")
    orc.lib().orc_gefen_step(2, 2, orc._ptr(p), orc._ptr(g), orc._ptr(st.m_codebook), orc._ptr(st.m_magnitude),
                             orc._ptr(st.vmean), n, 1, pod, orc._ptr(cb), 256, 0.9, 0.999, 1e-3, 1e-8, 0.0, 0.1,
                             1 - 0.999, 1)
    np.testing.assert_array_equal(gu.to_np(idx).reshape(-1), st.m_codebook)
    np.testing.assert_array_equal(gu.to_np(mag).reshape(-1), st.m_magnitude)
    np.testing.assert_array_equal(gu.to_np(v).reshape(-1), st.vmean)
    np.testing.assert_array_equal(gu.to_np(pd), p)

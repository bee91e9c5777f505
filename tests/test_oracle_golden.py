"""Pin the CPU oracle to the reference's own CPU path (golden fixtures).

The fixtures in tests/golden/ were written by tests/golden/make_golden.py from
the reference package (ndvbd/Gefen 1.2.3) in the survey container.
"""

import numpy as np
import pytest

from golden_util import load
import traj_util as tu
from oracle import oracle as orc


# ------------------------------------------------------------------ periods
def test_period_scores_and_choice_match_reference():
    data, meta = load("periods")
    for case in meta:
        name, dtype = case["name"], case["dtype"]
        g = data[name + "/grad"]
        divs = data[name + "/divisors"].tolist()
        ref_scores = data[name + "/scores"]
        if divs:
            sc = orc.period_scores(g, dtype, divs, mode=1)
            np.testing.assert_allclose(sc, ref_scores, rtol=1e-13, atol=0, err_msg=name)
        assert orc.find_period(g, dtype) == int(data[name + "/period"]), name


def test_period_fixture_checksums_are_stable():
    # the generator used to build the inputs must still produce the same bytes
    from gefen_amd import synthetic as syn
    import make_golden as mg
    data, meta = load("periods")
    for i, case in enumerate(mg.PERIOD_CASES):
        name, rows, cols, dtype, mode, e_lo, e_hi = case
        g = mg.period_case_grad(1234, i, rows, cols, dtype, mode, e_lo, e_hi)
        np.testing.assert_array_equal(g, data[name + "/grad"], err_msg=name)
        assert syn.checksum(g) == meta[i]["checksum"]


# ------------------------------------------------------------------ exact DP
def test_exact_dp_matches_reference_histograms():
    data, meta = load("exact_dp")
    for case in meta:
        if case["kind"] != "exact_dp":
            continue
        name = case["name"]
        cb = orc.exact_dp(data[name + "/counts"], int(data[name + "/k"]), bool(data[name + "/force"]))
        np.testing.assert_array_equal(cb, data[name + "/codebook"], err_msg=name)


def test_first_step_pipeline_matches_reference():
    data, meta = load("exact_dp")
    for case in meta:
        if case["kind"] != "pipeline":
            continue
        name = case["name"]
        gp = []
        for ti in range(case["ntensors"]):
            g = data["{}/grad{}".format(name, ti)]
            dtype = "bf16" if g.dtype == np.uint16 else "f32"
            gp.append((g, dtype, int(data["{}/period{}".format(name, ti)])))
        cb = orc.learn_codebook(gp)
        np.testing.assert_array_equal(cb, data[name + "/codebook"], err_msg=name)


# ------------------------------------------------------------------ trajectories
def _check_snapshot(name, dtype, got, ref, step):
    if dtype == "f32":
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-7, err_msg="{} step {}".format(name, step))
    else:
        d = tu.ulp_distance_bf16(got, ref)
        assert d.max() <= 1, "{} step {}: max ulp distance {}".format(name, step, d.max())


@pytest.mark.parametrize("name", [n for n in tu.TRAJ_NAMES if not n.startswith("muon")])
def test_gefen_trajectory_matches_reference(name):
    data, meta, params, skip = tu.build(name)
    arrs = [dict(prm, p=prm["p0"].reshape(-1).copy()) for prm in params]
    cb = None if meta["kind"] == "gefen_learn" else data["codebook_in"]
    opt = orc.GefenOracle(arrs, codebook=cb, nthreads=1)
    for step in range(1, meta["steps"] + 1):
        opt.step(tu.grads_for(meta, params, step, skip))
        if step == 1:
            assert [opt.periods[i] for i in range(len(params))] == data["periods"].tolist()
            np.testing.assert_array_equal(opt.codebook, data["codebook_out"])
        if step in (1, 2, 20):
            for i, prm in enumerate(arrs):
                st = opt.state[i]
                key = "s{}/m_codebook/step{}".format(i, step)
                np.testing.assert_array_equal(st.m_codebook, tu.bits(data[key]).reshape(-1), err_msg=key)
                key = "s{}/m_magnitude/step{}".format(i, step)
                np.testing.assert_array_equal(st.m_magnitude, tu.bits(data[key]).reshape(-1), err_msg=key)
                key = "s{}/vmean/step{}".format(i, step)
                sdt = prm.get("sdtype", prm["dtype"])
                vref = orc.to_f32(tu.bits(data[key]).reshape(-1), sdt)
                vgot = orc.to_f32(st.vmean, sdt)
                if sdt == "f32":
                    np.testing.assert_allclose(vgot, vref, rtol=2e-6, atol=0, err_msg=key)
                else:
                    assert tu.ulp_distance_bf16(st.vmean, tu.bits(data[key]).reshape(-1)).max() <= 1, key
        if step in (1, 2, 5, 10, 20):
            for i, prm in enumerate(arrs):
                ref = tu.bits(data["p{}/step{}".format(i, step)]).reshape(-1)
                _check_snapshot("{}/p{}".format(name, i), prm["dtype"], prm["p"], ref, step)


@pytest.mark.parametrize("name", ["muon_bf16", "muon_f32"])
def test_gefen_muon_trajectory_matches_reference(name):
    data, meta, params, skip = tu.build(name)
    arrs = [dict(prm, p=prm["p0"].reshape(-1).copy()) for prm in params]
    kw = meta["kwargs"]
    opt = orc.GefenMuonOracle(arrs, codebook=data["codebook_in"], momentum=0.95,
                              nesterov=kw.get("nesterov", True))
    for step in range(1, meta["steps"] + 1):
        opt.step(tu.grads_for(meta, params, step, skip))
        if step == 1:
            assert [opt.periods[i] for i in range(len(params))] == data["periods"].tolist()
        if step in (1, 2, 20):
            # the quantised momentum never sees the parameters: bit-exact at every step
            for i in range(len(params)):
                st = opt.state[i]
                key = "s{}/m_codebook/step{}".format(i, step)
                if key not in data:
                    continue
                np.testing.assert_array_equal(st.m_codebook, tu.bits(data[key]).reshape(-1), err_msg=key)
                key = "s{}/m_magnitude/step{}".format(i, step)
                np.testing.assert_array_equal(st.m_magnitude, tu.bits(data[key]).reshape(-1), err_msg=key)
        if step in (1, 2, 5, 10, 20):
            for i, prm in enumerate(arrs):
                dt = prm["dtype"]
                p0 = orc.to_f32(prm["p0"].reshape(-1), dt)
                ours = orc.to_f32(prm["p"], dt) - p0
                ref = orc.to_f32(tu.bits(data["p{}/step{}".format(i, step)]).reshape(-1), dt) - p0
                # Newton-Schulz is five bf16 GEMM rounds whose fp32 accumulation order on the
                # reference's CPU BLAS is unpublished; the accumulated update agrees to
                # a few percent (bf16 parameters) / a few tenths of a percent (fp32).
                tol = 0.05 if dt != "f32" else 0.01
                rel = np.linalg.norm(ours - ref) / max(np.linalg.norm(ref), 1e-30)
                assert rel <= tol, "{} p{} step {}: relative update error {:.3g}".format(name, i, step, rel)


# ------------------------------------------------------------------ kernel-level entry points
def test_packed_nibble_layout():
    """automatic_gefen_fused_kernel.cu:14-57: element i's index is the low nibble of byte
    i/2 for even i and the high nibble for odd i; a store keeps the low four bits of the
    index and leaves the other nibble of its byte as it was."""
    packed = np.array([0xFF, 0xAB], np.uint8)
    orc.pack_nibbles(np.array([1, 2, 19], np.uint8), packed)
    assert packed.tolist() == [0x21, 0xA3]
    assert orc.unpack_nibbles(packed, 3).tolist() == [1, 2, 3]
    assert orc.unpack_nibbles(np.array([0x5A, 0x0F], np.uint8), 4).tolist() == [0xA, 0x5, 0xF, 0x0]
    rng = np.random.default_rng(3)
    for n in (1, 2, 7, 64, 1001):
        idx = rng.integers(0, 256, n, dtype=np.uint8)
        packed = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
        tail = packed[-1] >> 4
        orc.pack_nibbles(idx, packed)
        np.testing.assert_array_equal(orc.unpack_nibbles(packed, n), idx & 15)
        if n % 2:
            assert packed[-1] >> 4 == tail


@pytest.mark.parametrize("dt,sdt,period", [("f32", "f32", 96), ("bf16", "bf16", 33), ("bf16", "f32", 7),
                                           ("f16", "f16", 256)])
def test_given_vmean_and_given_stepsize_updates_equal_the_step(dt, sdt, period):
    """The given-vmean update after the vmean EMA, and the given-stepsize update with the
    stepsize of gefen.py:1326-1327 computed here in numpy float32, both equal one step of
    the (trajectory-pinned) oracle step, bit for bit, through three steps."""
    from gefen_amd import synthetic as syn

    data, _ = load("exact_dp")
    cb = np.ascontiguousarray(data["hist_k256_forced/codebook"], dtype=np.float32)
    rows = 6
    n = rows * period
    b1, b2, lr, eps = 0.9, 0.999, 1e-3, 1e-8
    p0 = syn.round_to(syn.normal(syn.make_key(2, 1), n) * 0.02, dt)
    st = {k: orc.TensorState(n, period, dt, sdt) for k in "abc"}
    p = {k: p0.copy() for k in "abc"}
    vb = st["b"].vmean
    for step in (1, 2, 3):
        g = syn.round_to(syn.row_scaled_normal(4, step, rows, period, -14, -4), dt).reshape(-1)
        bc1, bc2 = 1 - b1 ** step, 1 - b2 ** step
        a = st["a"]
        rc = orc.lib().orc_gefen_step(orc.DT[dt], orc.DT[sdt], orc._ptr(p["a"]), orc._ptr(g),
                                      orc._ptr(a.m_codebook), orc._ptr(a.m_magnitude), orc._ptr(a.vmean), n,
                                      period, 0, orc._ptr(cb), cb.size, b1, b2, lr, eps, 0.0, bc1, bc2, 1)
        assert rc == 0
        orc.lib().orc_vmean_update(orc.DT[sdt], orc._ptr(vb), orc.DT[dt], orc._ptr(g), rows, period, b2)
        orc.gefen_update_given(dt, sdt, p["b"], g, st["b"].m_codebook, st["b"].m_magnitude, period, cb, b1, lr,
                               vmean=vb, bc1=bc1, bc2=bc2, eps=eps)
        v = orc.to_f32(vb, sdt)
        h = np.sqrt(v) / np.float32(np.sqrt(bc2)) + np.float32(eps)
        ss = ((np.float32(1.0) / h) * np.float32(1.0 / bc1)).astype(np.float32)
        orc.gefen_update_given(dt, sdt, p["c"], g, st["c"].m_codebook, st["c"].m_magnitude, period, cb, b1, lr,
                               stepsize=ss)
        np.testing.assert_array_equal(vb, a.vmean)
        for o in "bc":
            np.testing.assert_array_equal(st[o].m_codebook, a.m_codebook)
            np.testing.assert_array_equal(st[o].m_magnitude, a.m_magnitude)
            np.testing.assert_array_equal(p[o], p["a"])
        assert int(a.m_codebook.astype(np.int64).sum()) > 0


# ------------------------------------------------------------------ Lloyd-Max / block variance (CUDA semantics)
def _lloyd_brute(g, period, cb):
    """Independent restatement of lloyd_max_fused_kernel.cu:17-107 for a sorted
    codebook with distinct entries: the nearest codeword with ties to the lower
    index, NaN to index 0; the block absmax ignores NaN."""
    x = g.reshape(-1, period).astype(np.float32)
    absmax = np.nanmax(np.abs(x), axis=1, keepdims=True)
    absmax = np.where(np.isnan(absmax), 0, absmax).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        xn = np.where(absmax > 0, x / absmax, np.float32(0)).astype(np.float32).reshape(-1)
    d = np.abs(xn[:, None].astype(np.float64) - cb[None, :].astype(np.float64))
    idx = np.argmin(np.where(np.isnan(d), np.inf, d), axis=1)
    idx[np.isnan(xn)] = 0
    return xn, idx


def test_lloyd_oracle_matches_brute_force():
    from gefen_amd import synthetic as syn

    data, _ = load("exact_dp")
    for cb in (data["hist_k256_forced/codebook"], data["hist_k16_free/codebook"]):
        assert np.all(np.diff(cb) > 0)
        g = syn.round_to(syn.row_scaled_normal(7, 1, 24, 96, -12, -3), "f32").reshape(-1).copy()
        g[5 * 96 + 7] = np.nan            # a NaN element: skipped by the absmax, counted at index 0
        g[9 * 96:10 * 96] = 0.0           # a zero block: every x is 0
        g[11 * 96 + 3] = np.inf           # an inf element: absmax inf, x = 0 or NaN
        xn, idx = _lloyd_brute(g, 96, cb)
        sums, counts = orc.lloyd_accumulate(g, "f32", 96, cb)
        np.testing.assert_array_equal(counts, np.bincount(idx, minlength=cb.size))
        ref = np.bincount(idx, weights=xn.astype(np.float64), minlength=cb.size)
        np.testing.assert_array_equal(np.isnan(sums), np.isnan(ref))
        ok = ~np.isnan(ref)
        np.testing.assert_allclose(sums[ok], ref[ok], rtol=1e-12, atol=1e-12)
        new = (cb * np.float32(0.99)).astype(np.float32)
        mn, mo = orc.lloyd_mse(g, "f32", 96, cb, new)
        assert np.isnan(mn) and np.isnan(mo)   # the NaN element's error is NaN
        g2 = g.copy()
        g2[np.isnan(g2) | np.isinf(g2)] = 0.5
        xn, idx = _lloyd_brute(g2, 96, cb)
        amax = np.repeat(np.abs(g2.reshape(-1, 96)).max(1), 96).astype(np.float32)
        err = (xn - new[idx]).astype(np.float32)
        mn, mo = orc.lloyd_mse(g2, "f32", 96, cb, new)
        # each squared error is a float32 product (lines 173-176); sums in double
        assert abs(mn - float((err * err).astype(np.float64).sum())) <= 1e-12 * max(mn, 1e-30)
        oe = (err * amax).astype(np.float32)
        assert abs(mo - float((oe * oe).astype(np.float64).sum())) <= 1e-12 * max(mo, 1e-30)


def test_lloyd_oracle_index_beyond_the_last_codeword():
    """x above the last codeword: the reference compares the last two entries, so
    a duplicated last codeword takes the lower index (lloyd_max_fused_kernel.cu:33-47)."""
    cb = np.array([-0.5, 0.0, 0.25, 0.25], np.float32)
    g = np.array([1.0, 0.5, -1.0, 0.0], np.float32)   # absmax 1: x = 1, 0.5, -1, 0
    _, counts = orc.lloyd_accumulate(g, "f32", 4, cb)
    assert counts.tolist() == [1, 1, 2, 0]


def test_block_variance_oracle_matches_closed_form():
    from gefen_amd import synthetic as syn

    g = syn.round_to(syn.row_scaled_normal(3, 3, 50, 64, -7, -2), "f32").reshape(-1)
    x = (g.astype(np.float32) ** 2).astype(np.float64).reshape(50, 64)
    var = np.maximum((x * x).mean(1) - x.mean(1) ** 2, 0)
    out = orc.block_variance(g, "f32", 64, False, False)
    np.testing.assert_allclose(out[0], np.sqrt(var.mean()), rtol=1e-12)
    out = orc.block_variance(g, "f32", 64, False, True)
    np.testing.assert_allclose(out[0], (np.sqrt(var) / x.mean(1)).sum(), rtol=1e-12)
    assert out[1] == 50 and out[2] == 0
    out = orc.block_variance(-np.ones(8, np.float32), "f32", 4, True, True)
    assert out[2] == 2 and out[1] == 0


def test_full_size_period_fixture_k_proj():
    """The oracle on a full-size config tensor (Llama-3-8B k_proj, 4.2M bf16
    elements, regenerated from its seed) against the reference's scores; the two
    larger tensors of periods_full.npz are checked on the GPU box, where their
    inputs come from the device generator."""
    from gefen_amd import synthetic as syn
    import make_golden as mg

    data, meta = load("periods_full")
    case = next(c for c in mg.PERIOD_FULL_CASES if c[0] == "llama8b_k_proj_bf16")
    m = next(x for x in meta if x["name"] == case[0])
    g = mg.period_full_grad(case)
    assert syn.checksum(g) == m["checksum"]
    divs = data[case[0] + "/divisors"].tolist()
    np.testing.assert_allclose(orc.period_scores(g, "bf16", divs, mode=1), data[case[0] + "/scores"], rtol=1e-13,
                               atol=0)
    assert orc.find_period(g, "bf16") == m["period"]

"""Pin the oracle's GefenMuon arithmetic to the reference's own outputs.

Fixtures (written from the reference by tests/golden/make_golden.py):
* ``ns_products.npz``: every bf16 product of the five Newton-Schulz iterations
  of ``_zeropower_via_newtonschulz`` (gefen_muon.py:16-51) on seeded inputs:
  X_0 (normalised), then per iteration A = X X^T, B = addmm(A, A, A, beta=b,
  alpha=c), X' = addmm(X, B, X, beta=a), and the function's result;
* ``muon_steps_*.npz``: along the GefenMuon trajectories, each step's
  Newton-Schulz input (the Nesterov blend, gefen_muon.py:302-316), its result,
  and every parameter before and after the update (gefen_muon.py:318-329).

Each product is fed the reference's own bf16 operands, so it is checked on its
own, free of what earlier iterations did.  torch-CPU accumulates the products
in float32; the oracle forms them exactly and rounds once, so the two agree on
all but a few elements in 10^4, and every element lies within one bf16 ulp plus
the float32 accumulation bound 2(K+1) 2^-24 sum|terms|.  A mistake in a rounding
point (a rounding before instead of after the addmm, an alpha not applied in
float32) breaks the exact-match fraction and the bound on the elements where
the terms cancel.
"""

import numpy as np
import pytest

from golden_util import load
import traj_util as tu
from oracle import oracle as orc

NS = ("ns_256x512", "ns_512x256", "ns_128x384")
A, B, C = 3.4445, -4.7750, 2.0315


def check_product(got_bits, ref_bits, bound, what, min_exact=0.999):
    """Every element within 1 bf16 ulp + the accumulation bound; the exact-match
    fraction at least min_exact.  Returns (exact fraction, max ulps)."""
    got = orc.to_f32(got_bits, "bf16").astype(np.float64)
    ref = orc.to_f32(ref_bits, "bf16").astype(np.float64)
    tol = np.maximum(orc.ulp_bf16(ref_bits), orc.ulp_bf16(got_bits)) + bound
    excess = np.abs(got - ref) / tol
    ulps = tu.ulp_distance_bf16(got_bits, ref_bits)
    exact = float((ulps == 0).mean())
    assert excess.max() <= 1.0, "{}: |got - ref| exceeds the bound by {:.3g}x".format(what, excess.max())
    assert exact >= min_exact, "{}: only {:.5f} of the elements are exact".format(what, exact)
    return exact, int(ulps.max())


@pytest.mark.parametrize("name", NS)
def test_oracle_newton_schulz_products_match_reference(name):
    d, _ = load("ns_products")
    x0 = orc.ns_normalize(d[name + "/g"])
    np.testing.assert_array_equal(x0, d[name + "/x0"], err_msg=name + " normalisation")
    for k in range(1, 6):
        x, a, b, xn = (d["{}/{}".format(name, key)] for key in ("x{}".format(k - 1), "a{}".format(k),
                                                                  "b{}".format(k), "x{}".format(k)))
        check_product(orc.ns_gram(x), a, orc.ns_term_bound("gram", x), "{} A{}".format(name, k))
        check_product(orc.ns_poly(a, B, C), b, orc.ns_term_bound("poly", a, b=B, c=C), "{} B{}".format(name, k))
        check_product(orc.ns_update(b, x, A), xn, orc.ns_term_bound("update", b, x, a=A), "{} X{}".format(name, k))


def test_newton_schulz_product_checks_catch_a_misplaced_rounding():
    """The check above fails an oracle that rounds A A to bf16 before adding b A
    (a plausible misreading of addmm)."""
    d, _ = load("ns_products")
    name = "ns_256x512"
    a = d[name + "/a3"]
    af = orc.to_f32(a, "bf16").astype(np.float64)
    aa = orc.to_f32(orc.from_f32((af @ af).astype(np.float32), "bf16"), "bf16").astype(np.float64)
    wrong = orc.from_f32((B * af + C * aa).astype(np.float32), "bf16")
    with pytest.raises(AssertionError):
        check_product(wrong, d[name + "/b3"], orc.ns_term_bound("poly", a, b=B, c=C), "misplaced rounding")


@pytest.mark.parametrize("name", NS)
def test_oracle_newton_schulz_end_to_end(name):
    """The whole function from the raw input: five iterations amplify the rare
    last-bit differences of single products (near-zero singular values grow by up
    to a^5 ~ 490), so the result agrees in norm, not bit for bit."""
    d, _ = load("ns_products")
    g = orc.to_f32(d[name + "/g"], "bf16")
    got = orc.newton_schulz_bf16(g)
    ref = orc.to_f32(d[name + "/out"], "bf16")
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= 0.02, "{}: relative error {:.3g}".format(name, rel)


def test_ns_fixture_inputs_regenerate():
    from gefen_amd import synthetic as syn
    import make_golden as mg
    d, meta = load("ns_products")
    for case, m in zip(mg.NS_CASES, meta):
        name, rows, cols, stream = case
        g = syn.round_to(syn.normal(syn.make_key(m["seed"], stream), rows * cols) * 1e-3, "bf16")
        np.testing.assert_array_equal(g.reshape(rows, cols), d[name + "/g"])
        assert syn.checksum(g) == m["checksum_g"]


@pytest.mark.parametrize("name", ["muon_bf16", "muon_f32"])
def test_oracle_muon_blend_and_update_match_reference_steps(name):
    """Along the reference trajectory: the oracle's quantised momentum with the
    Nesterov blend equals the reference's Newton-Schulz input bit for bit; the
    oracle's parameter update applied to the reference's Newton-Schulz result
    equals the reference's parameter bit for bit; and the oracle's Newton-Schulz
    of the reference's input is within 2% (norm) of the reference's result."""
    steps_data, steps_meta = load("muon_steps_" + name)
    data, meta, params, skip = tu.build(name)
    arrs = [dict(prm, p=prm["p0"].reshape(-1).copy()) for prm in params]
    kw = meta["kwargs"]
    opt = orc.GefenMuonOracle(arrs, codebook=data["codebook_in"], momentum=0.95, nesterov=kw.get("nesterov", True))
    for step in range(1, max(steps_meta["steps"]) + 1):
        opt.step(tu.grads_for(meta, params, step, skip))
        if step not in steps_meta["steps"]:
            continue
        for i, prm in enumerate(arrs):
            key = "p{}/step{}/".format(i, step)
            dt, shape = prm["dtype"], prm["shape"]
            ns_in = tu.bits(steps_data[key + "ns_in"]).reshape(-1)
            np.testing.assert_array_equal(opt.last_blend[i], ns_in, err_msg=key + "blend")
            ns_out = tu.bits(steps_data[key + "ns_out"])
            p = tu.bits(steps_data[key + "before"]).reshape(-1).copy()
            orc.muon_apply(p, ns_out, dt, shape, prm["lr"], prm["weight_decay"],
                           orc.adjust_lr(prm["lr"], None, shape))
            np.testing.assert_array_equal(p, tu.bits(steps_data[key + "after"]).reshape(-1), err_msg=key + "apply")
            u = orc.newton_schulz_bf16(orc.to_f32(ns_in, dt).reshape(shape))
            ref = orc.to_f32(ns_out, "bf16").reshape(shape)
            rel = np.linalg.norm(u - ref) / np.linalg.norm(ref)
            assert rel <= 0.02, "{}: Newton-Schulz relative error {:.3g}".format(key, rel)


@pytest.mark.parametrize("name", ["muon_bf16", "muon_f32"])
def test_muon_step_fixture_agrees_with_trajectory_fixture(name):
    """Two fixtures written by separate replays of the reference: the parameters
    after the captured steps are the trajectory's snapshots."""
    steps_data, steps_meta = load("muon_steps_" + name)
    data, meta, params, skip = tu.build(name)
    for step in steps_meta["steps"]:
        for i in range(len(params)):
            np.testing.assert_array_equal(tu.bits(steps_data["p{}/step{}/after".format(i, step)]).reshape(-1),
                                          tu.bits(data["p{}/step{}".format(i, step)]).reshape(-1))

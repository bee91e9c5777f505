"""GefenMuon on the GPU against the reference's own Newton-Schulz products and
GefenMuon steps (fixtures ns_products.npz, muon_steps_*.npz written from the
reference by tests/golden/make_golden.py).

Every GPU product is fed the reference's bf16 operands of that product, through
the C ABI (gefen_gemm_bf16_nt_batched, gefen_gemm_bf16, gefen_ns_prepare,
gefen_muon_apply_tasks).  The bar for a product is the one the oracle meets
(tests/test_oracle_newton_schulz.py): every element within one bf16 ulp plus the
float32 accumulation bound 2(K+1) 2^-24 sum|terms|, and at least 99.9% of the
elements bit-exact.  The Nesterov blend and the parameter update are bit-exact.
"""

import numpy as np
import pytest
import torch

from golden_util import load
import gpu_util as gu
import traj_util as tu
from oracle import oracle as orc
from test_oracle_newton_schulz import A, B, C, check_product

pytestmark = pytest.mark.gpu

NS_BATCHED = ("ns_256x512", "ns_512x256")
NS_ALL = ("ns_256x512", "ns_512x256", "ns_128x384")


def dev(bits):
    return gu.to_dev(np.ascontiguousarray(bits), "bf16")


def host(t):
    return gu.to_np(t)


@pytest.mark.parametrize("name", NS_BATCHED)
def test_batched_gemm_products_match_reference(name):
    from gefen_amd.newton_schulz import gemm_nt_batched

    print("ns products (batched)", name, flush=True)
    d, _ = load("ns_products")
    report = []
    for k in range(1, 6):
        x, a, b, xn = (d["{}/{}".format(name, key)] for key in ("x{}".format(k - 1), "a{}".format(k),
                                                                  "b{}".format(k), "x{}".format(k)))
        m, n = x.shape
        xd, ad, bd = dev(x)[None], dev(a)[None], dev(b)[None]
        xtd = dev(np.ascontiguousarray(x.T))[None]
        gram = torch.empty(1, m, m, dtype=torch.bfloat16, device="cuda:0")
        gemm_nt_batched(xd, xd, gram, symmetric=True)                                   # X X^T
        upd = torch.empty(1, m, m, dtype=torch.bfloat16, device="cuda:0")
        gemm_nt_batched(ad, ad, upd, d_t=ad, alpha=C, beta=B, symmetric=True)             # b A + c A A
        nx = torch.empty(1, m, n, dtype=torch.bfloat16, device="cuda:0")
        nxt = torch.empty(1, n, m, dtype=torch.bfloat16, device="cuda:0")
        gemm_nt_batched(bd, xtd, nx, out_t=nxt, d_t=xtd, alpha=1.0, beta=A)               # a X + B X
        report.append(check_product(host(gram[0]), a, orc.ns_term_bound("gram", x), "{} A{}".format(name, k)))
        report.append(check_product(host(upd[0]), b, orc.ns_term_bound("poly", a, b=B, c=C), "{} B{}".format(name, k)))
        got_x = host(nx[0])
        report.append(check_product(got_x, xn, orc.ns_term_bound("update", b, x, a=A), "{} X{}".format(name, k)))
        np.testing.assert_array_equal(host(nxt[0]), np.ascontiguousarray(got_x.T))
    print(name, "exact fraction / max ulp per product:", report, flush=True)


@pytest.mark.parametrize("name", NS_ALL)
def test_single_matrix_gemm_products_match_reference(name):
    from gefen_amd.newton_schulz import gemm

    print("ns products (single)", name, flush=True)
    d, _ = load("ns_products")
    for k in range(1, 6):
        x, a, b, xn = (d["{}/{}".format(name, key)] for key in ("x{}".format(k - 1), "a{}".format(k),
                                                                  "b{}".format(k), "x{}".format(k)))
        m, n = x.shape
        xd, ad, bd = dev(x), dev(a), dev(b)
        gram = torch.empty(m, m, dtype=torch.bfloat16, device="cuda:0")
        gemm(xd, xd, True, gram)
        upd = torch.empty(m, m, dtype=torch.bfloat16, device="cuda:0")
        gemm(ad, ad, False, upd, d=ad, alpha=C, beta=B)
        nx = torch.empty(m, n, dtype=torch.bfloat16, device="cuda:0")
        gemm(bd, xd, False, nx, d=xd, alpha=1.0, beta=A)
        check_product(host(gram), a, orc.ns_term_bound("gram", x), "{} A{}".format(name, k))
        check_product(host(upd), b, orc.ns_term_bound("poly", a, b=B, c=C), "{} B{}".format(name, k))
        check_product(host(nx), xn, orc.ns_term_bound("update", b, x, a=A), "{} X{}".format(name, k))


@pytest.mark.parametrize("name", NS_BATCHED)
def test_ns_prepare_matches_reference_normalisation(name):
    """gefen_ns_prepare: x / max(bf16(||x||), bf16(eps)) in bf16 and the transpose;
    the float32 norm is a reduction in another order, so the bf16 norm (and then
    every quotient) can differ by its last bit only when the float32 norm lies at
    a bf16 rounding boundary: within 1 ulp, and bit-exact here."""
    from gefen_amd import _lib

    d, _ = load("ns_products")
    g = d[name + "/g"]
    rows, cols = g.shape
    x = dev(g)[None].clone()
    xt = torch.empty(1, cols, rows, dtype=torch.bfloat16, device="cuda:0")
    lib = _lib.load()
    _lib.check(lib.gefen_ns_prepare(x.data_ptr(), xt.data_ptr(), 1, rows, cols, 1e-7, gu.stream()))
    got = host(x[0]) if rows <= cols else host(xt[0])
    ulps = tu.ulp_distance_bf16(got, d[name + "/x0"])
    assert ulps.max() <= 1
    assert (ulps == 0).mean() >= 0.999, (ulps == 0).mean()
    np.testing.assert_array_equal(host(xt[0]), np.ascontiguousarray(host(x[0]).T))


@pytest.mark.parametrize("name", NS_ALL)
def test_newton_schulz_end_to_end_matches_reference(name):
    """From the raw input through five iterations: the rare last-bit product
    differences are amplified by the iteration (small singular values grow by up
    to a^5), so the results agree in norm (the oracle's own error against the
    reference is 0.5-0.7% here)."""
    from gefen_amd.newton_schulz import batched_shape_ok, newton_schulz_batched, newton_schulz_bf16

    d, _ = load("ns_products")
    g = d[name + "/g"]
    ref = orc.to_f32(d[name + "/out"], "bf16").astype(np.float64)
    outs = [newton_schulz_bf16(dev(g), (A, B, C), 5, 1e-7)]
    if batched_shape_ok(*g.shape):
        outs.append(newton_schulz_batched(dev(g)[None].clone(), (A, B, C), 5, 1e-7)[0])
    for out in outs:
        got = orc.to_f32(host(out), "bf16").astype(np.float64)
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel <= 0.02, (name, rel)


@pytest.mark.parametrize("name", ["muon_bf16", "muon_f32"])
def test_muon_steps_match_reference_blend_update_and_newton_schulz(name, monkeypatch):
    """GefenMuon on the GPU along the reference trajectory: at the captured steps
    the Nesterov blend (the Newton-Schulz input) is bit-exact; the parameter
    update of gefen_muon_apply_tasks applied to the reference's own parameter and
    Newton-Schulz result is bit-exact; the GPU Newton-Schulz of the reference's
    input is within 2% (norm) of the reference's result."""
    from gefen_amd import _lib
    from gefen_amd import gefen_muon as gm
    from gefen_amd.newton_schulz import newton_schulz_bf16

    print("muon steps", name, flush=True)
    steps_data, steps_meta = load("muon_steps_" + name)
    data, meta, params, skip = tu.build(name)
    dtype = meta["dtype"]
    tensors = [gu.to_dev(prm["p0"], dtype).reshape(prm["shape"]).requires_grad_(True) for prm in params]
    opt = gm.GefenMuon([(prm["name"], t) for prm, t in zip(params, tensors)], **meta["kwargs"])
    opt._gefen_codebook = torch.from_numpy(data["codebook_in"]).to("cuda:0")
    seen = []
    real_ns = gm._zeropower_via_newtonschulz

    def spy(grad, coeffs, ns_steps, eps):
        seen.append(grad.detach().clone())
        return real_ns(grad, coeffs, ns_steps, eps)

    monkeypatch.setattr(gm, "_zeropower_via_newtonschulz", spy)
    lib = _lib.load()
    for step in range(1, max(steps_meta["steps"]) + 1):
        for t, g, prm in zip(tensors, tu.grads_for(meta, params, step, skip), params):
            t.grad = gu.to_dev(g.reshape(-1), dtype).reshape(prm["shape"])
        seen.clear()
        opt.step()
        assert len(seen) == len(params)  # these shapes take the one-matrix Newton-Schulz path
        if step not in steps_meta["steps"]:
            continue
        for i, prm in enumerate(params):
            key = "p{}/step{}/".format(i, step)
            ns_in = tu.bits(steps_data[key + "ns_in"])
            np.testing.assert_array_equal(gu.to_np(seen[i]).reshape(-1), ns_in.reshape(-1), err_msg=key + "blend")
            ns_out = tu.bits(steps_data[key + "ns_out"])
            p = gu.to_dev(tu.bits(steps_data[key + "before"]).reshape(-1), dtype)
            u = dev(ns_out.reshape(-1))
            task = np.zeros(1, dtype=_lib.MUON_APPLY_TASK)
            task[0]["p"], task[0]["update"], task[0]["numel"] = p.data_ptr(), u.data_ptr(), p.numel()
            task[0]["param_dtype"] = gu.CODE[dtype]
            task[0]["transposed"] = 1 if prm["shape"][0] > prm["shape"][1] else 0
            task[0]["lr"], task[0]["weight_decay"] = prm["lr"], prm["weight_decay"]
            task[0]["adjusted_lr"] = orc.adjust_lr(prm["lr"], None, prm["shape"])
            _lib.check(lib.gefen_muon_apply_tasks(task.ctypes.data, 1, gu.stream()))
            np.testing.assert_array_equal(gu.to_np(p), tu.bits(steps_data[key + "after"]).reshape(-1),
                                          err_msg=key + "apply")
            got = newton_schulz_bf16(gu.to_dev(ns_in.reshape(-1), dtype).reshape(prm["shape"]), (A, B, C), 5, 1e-7)
            got = orc.to_f32(gu.to_np(got), "bf16").reshape(prm["shape"]).astype(np.float64)
            ref = orc.to_f32(ns_out, "bf16").reshape(prm["shape"]).astype(np.float64)
            rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
            assert rel <= 0.02, (key, rel)


def test_momentum_sums_of_squares_feed_the_same_normalisation():
    """gefen_muon_tasks_sumsq leaves each task's sum of squares of the outputs it
    wrote (float32 sums per lane and wave, added in float64: within 1e-5 of a
    float64 sum of the same values; the norm is rounded to bf16 from it), and
    gefen_ns_prepare_sumsq with those sums normalises and transposes the stack
    bit-identically to gefen_ns_prepare, which computes the norms itself."""
    from gefen_amd import _lib
    from gefen_amd import synthetic as syn

    lib = _lib.load()
    data, _ = load("exact_dp")
    cb = torch.from_numpy(data["hist_k256_forced/codebook"]).to("cuda:0")
    tables = torch.empty(int(lib.gefen_codebook_tables_size()), dtype=torch.uint8, device="cuda:0")
    _lib.check(lib.gefen_prepare_codebook(cb.data_ptr(), cb.numel(), tables.data_ptr(), gu.stream()))
    G, rows, cols = 5, 256, 512
    stack = torch.empty(G, rows, cols, dtype=torch.bfloat16, device="cuda:0")
    grads = [torch.empty(rows * cols, dtype=torch.bfloat16, device="cuda:0") for _ in range(G)]
    states = []
    tasks = np.zeros(G, dtype=_lib.MUON_TASK)
    for i, g in enumerate(grads):
        syn.fill_device(g, 77, i, syn.KIND_ROW_SCALED, cols=cols, e_lo=-12, e_hi=-8)
        block = (512, 256, 128, 1024, 2048)[i]  # magnitude blocks of several lengths
        idx = torch.zeros(rows * cols, dtype=torch.uint8, device="cuda:0")
        mag = torch.zeros(rows * cols // block, dtype=torch.bfloat16, device="cuda:0")
        states.append((idx, mag))
        t = tasks[i]
        t["grad"], t["m_codebook"], t["m_magnitude"] = g.data_ptr(), idx.data_ptr(), mag.data_ptr()
        t["out"], t["numel"], t["block"] = stack[i].data_ptr(), rows * cols, block
        t["grad_dtype"] = t["state_dtype"] = gu.CODE["bf16"]
        t["momentum"], t["nesterov"] = 0.95, 1
    sumsq = torch.empty(G * 128, dtype=torch.float64, device="cuda:0")  # GEFEN_SUMSQ_STRIDE per task
    for _ in range(2):  # twice: the sums restart from zero on every call
        _lib.check(lib.gefen_muon_tasks_sumsq(tasks.ctypes.data, G, tables.data_ptr(), sumsq.data_ptr(),
                                              gu.stream()))
    ref = (stack.double() ** 2).sum(dim=(1, 2))
    assert torch.allclose(sumsq.view(G, 8, 16)[:, :, 0].sum(1), ref, rtol=1e-5, atol=0), (sumsq, ref)
    x1, x2 = stack.clone(), stack.clone()
    t1 = torch.empty(G, cols, rows, dtype=torch.bfloat16, device="cuda:0")
    t2 = torch.empty_like(t1)
    order = torch.tensor([4, 3, 2, 1, 0], dtype=torch.int32, device="cuda:0")
    x2 = x2.flip(0).contiguous()  # matrix g of x2 is task 4 - g: found through the index
    _lib.check(lib.gefen_ns_prepare(x1.data_ptr(), t1.data_ptr(), G, rows, cols, 1e-7, gu.stream()))
    _lib.check(lib.gefen_ns_prepare_sumsq(x2.data_ptr(), t2.data_ptr(), G, rows, cols, 1e-7, sumsq.data_ptr(),
                                          order.data_ptr(), gu.stream()))
    assert torch.equal(x1.view(torch.int16), x2.flip(0).view(torch.int16))
    assert torch.equal(t1.view(torch.int16), t2.flip(0).view(torch.int16))

"""BASELINE config 5 at its full size against the oracle: GefenMuon on the
Qwen3-1.7B-shaped set (196 bf16 matrices, 28 layers of q 2048x2048, k/v
1024x2048, o 2048x2048, gate/up 6144x2048, down 2048x6144), built as bench.py
builds it and stepped by the optimizer as a whole (stacked Newton-Schulz, cached
plan, the last product applying the parameter update in its epilogue).

* every matrix's automatic period equals oracle.find_period, and the learned
  codebook equals oracle.learn_codebook, bit for bit;
* the quantised momentum state (codebook indices and magnitudes) of one matrix
  of each of the four shapes equals oracle.muon_momentum, bit for bit, over
  three steps with a new gradient each (the oracle running on its own: the
  state depends only on the gradients);
* the Newton-Schulz products of the last iteration of the third step, for one
  matrix per stack, taken from the GPU's own stacked buffers: A = X X^T (K =
  2048 or 6144), B = b A + c A A and a X + B X (K = 1024 or 2048) against
  oracle.ns_gram / ns_poly / ns_update of the same operands, each element within
  one bf16 ulp plus the float32 accumulation bound 2(K+1) 2^-24 sum|terms| and
  at least 99.9% of the elements bit-exact (the bar the oracle meets against the
  reference's own products, tests/test_oracle_newton_schulz.py);
* the parameter after that step, updated by the fused epilogue, equals
  oracle.muon_apply on the parameter before the step and the GPU's a X + B X
  (the same product, stored by the plain GEMM), bit for bit.
Reference: gefen_muon.py:16-51 (Newton-Schulz), 132-171 and 216-329 (step).
"""

import numpy as np
import pytest
import torch

import gpu_util as gu
from oracle import oracle as orc
from test_oracle_newton_schulz import A, B, C, check_product

pytestmark = pytest.mark.gpu

STEPS = 3


def _host(t):
    return gu.to_np(t).reshape(-1)


def test_qwen3_muon_full_config_matches_oracle():
    import bench
    from gefen_amd.gefen_muon import GefenMuon
    from gefen_amd.newton_schulz import gemm_nt_batched

    cfg = bench.CONFIGS["muon"]
    dev = torch.device("cuda:0")
    params = bench.build_problem(cfg, dev)
    print("Qwen3 problem built:", len(params), "matrices", flush=True)
    grads = [_host(p.grad) for _, p in params]
    opt = GefenMuon(params)
    opt.step()
    torch.cuda.synchronize()
    periods = [opt.state[p]["automatic_period"] for _, p in params]
    ref_periods = [orc.find_period(g, "bf16") for g in grads]
    bad = [(params[i][0], a, b) for i, (a, b) in enumerate(zip(periods, ref_periods)) if a != b]
    assert not bad, bad
    ref_cb = orc.learn_codebook([(g, "bf16", P) for g, P in zip(grads, ref_periods)])
    np.testing.assert_array_equal(opt._gefen_codebook.detach().cpu().numpy(), ref_cb)
    print("periods and codebook match the oracle; periods", sorted(set(periods)), flush=True)
    # one matrix of each shape: q (2048x2048), k (1024x2048), gate (6144x2048), down (2048x6144)
    sample = [0, 1, 4, 6]
    assert [tuple(params[i][1].shape) for i in sample] == [(2048, 2048), (1024, 2048), (6144, 2048), (2048, 6144)]
    g0 = opt.param_groups[0]
    mom, nest = g0["momentum"], g0["nesterov"]
    states = [orc.TensorState(params[i][1].numel(), ref_periods[i], "bf16", "bf16") for i in sample]
    ref_g = [grads[i] for i in sample]
    del grads
    before = None
    for step in range(1, STEPS + 1):
        if step > 1:
            before = [_host(params[i][1]).copy() for i in sample]
            for i, (_, p) in enumerate(params):
                bench.fill_grad(cfg, p.grad, i, step)
            opt.step()
            torch.cuda.synchronize()
            ref_g = [_host(params[i][1].grad) for i in sample]
        for k, i in enumerate(sample):
            orc.muon_momentum(ref_g[k], "bf16", states[k], ref_cb, mom, nest)
            st = opt.state[params[i][1]]
            tag = "{} step {}".format(params[i][0], step)
            np.testing.assert_array_equal(_host(st["m_codebook"]), states[k].m_codebook, err_msg=tag + " indices")
            np.testing.assert_array_equal(_host(st["m_magnitude"]), states[k].m_magnitude,
                                          err_msg=tag + " magnitudes")
        print("step", step, "momentum state of", [params[i][0] for i in sample], "bit-exact", flush=True)
    # the third step ran through the cached plan with the fused update: the last
    # iteration's operands are still in the stacks' buffers
    plan = opt._plan
    assert plan is not None and all(plan.fuse)
    coeffs = tuple(g0["ns_coefficients"])
    assert coeffs == (A, B, C) and g0["ns_steps"] == 5
    checked = set()
    for (key, idx, buf, work, _), fuse in zip(plan.stacks, plan.fuse):
        i = next(j for j in sample if j in idx)
        slot = idx.index(i)
        rows, cols = key[0], key[1]
        transposed = rows > cols
        m, n = min(rows, cols), max(rows, cols)
        # five iterations leave X^T of the last one in the stack's first X^T buffer
        # (the stack itself for a transposed stack), A and B in the work buffers
        xt = (buf if transposed else work["xt"])[slot:slot + 1]
        x = np.ascontiguousarray(gu.to_np(xt[0]).T)           # X [m, n]
        a_got = gu.to_np(work["gram"][slot])
        b_got = gu.to_np(work["upd"][slot])
        u = torch.empty(1, m, n, dtype=torch.bfloat16, device=dev)
        gemm_nt_batched(work["upd"][slot:slot + 1], xt, u, d_t=xt, alpha=1.0, beta=A)   # a X + B X
        u_got = gu.to_np(u[0])
        name = "{} ({}x{}, K = {} / {})".format(params[i][0], rows, cols, n, m)
        rep = [check_product(a_got, orc.ns_gram(x), orc.ns_term_bound("gram", x), name + " A = X X^T"),
               check_product(b_got, orc.ns_poly(a_got, B, C), orc.ns_term_bound("poly", a_got, b=B, c=C),
                             name + " B = bA + cAA"),
               check_product(u_got, orc.ns_update(b_got, x, A), orc.ns_term_bound("update", b_got, x, a=A),
                             name + " aX + BX")]
        print(name, "exact fraction / max ulp per product:", rep, flush=True)
        # the fused epilogue's update against the oracle's, applied to the GPU's product
        k = sample.index(i)
        p_ref = before[k].copy()
        shape = tuple(params[i][1].shape)
        u_param = np.ascontiguousarray(u_got.T) if transposed else u_got
        orc.muon_apply(p_ref, u_param.reshape(-1), "bf16", shape, g0["lr"], g0["weight_decay"],
                       orc.adjust_lr(g0["lr"], g0["adjust_lr_fn"], shape))
        np.testing.assert_array_equal(_host(params[i][1]), p_ref, err_msg=name + " fused update")
        checked.add((rows, cols))
    assert checked == {(2048, 2048), (1024, 2048), (6144, 2048), (2048, 6144)}, checked

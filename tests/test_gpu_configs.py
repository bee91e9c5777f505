"""The BASELINE configurations at their full sizes against the oracle.

Each configuration is built as bench.py builds it (device generator, seed 2026)
and stepped by the optimizer as a whole (batched launches, side stream, cached
plan).  Checked against the CPU oracle on the same bytes (the gradients are
copied from the device):
* every tensor's automatic period equals oracle.find_period;
* the learned codebook equals oracle.learn_codebook, bit for bit;
* sampled tensors (the embedding, the last tensor, a block-row matrix, a
  period-one matrix where the configuration has one, a norm or bias) over the
  configuration's stated number of steps (GPT-2 and Llama-1.5B 20, Llama-8B 10),
  a new gradient each step, with the oracle running on its own (never
  resynchronised from the GPU): codebook indices and magnitudes bit-exact at
  every step (the momentum state depends only on the gradients).  GPT-2 (fp32):
  vmean within rtol 2^-16 and parameters within rtol 1e-5 / atol 1e-7 after 20
  steps; GPT-2 also step by step over three steps with the oracle started from
  the GPU's state each step.
* bf16 configs: a block mean of g^2 summed in another order (the oracle sums in
  double, the reference and the GPU in float32, each in its own order) can round
  to the neighbouring bf16 vmean; from then on that row's stepsize differs by at
  most ~2^-8 relative and its parameters drift apart by a small fraction of the
  update.  Every other row (every period-one tensor: vmean is element-wise
  there) must stay bit-exact.  Rows whose vmean has differed at some step are
  tracked: their vmean within 2 ulps, their parameters within
  2^-7 * (sum of the oracle's per-step |update|) + (steps) * ulp.  The count and
  fraction of those rows and of the elements beyond one ulp are printed and
  bounded: at most 1e-2 of a tensor's rows (a float32 sum of 2048 squares is
  within ~2^-21 relative of the exact one, so a row's bf16 vmean flips with
  probability ~2^-12 / k at step k, ~1e-3 over 20 steps) and 1e-3 of the
  sampled elements.
"""

import numpy as np
import pytest
import torch

import gpu_util as gu
import traj_util as tu
from golden_util import load
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

STEPS = 3


def _host(t):
    return gu.to_np(t).reshape(-1)


def _initial(cfg, params, i):
    """The initial value of parameter i, regenerated as bench.build_problem made it."""
    from gefen_amd import synthetic as syn

    t = torch.empty_like(params[i][1].detach())
    syn.fill_device(t, 2026, 1_000_000 + i, syn.KIND_NORMAL, mult=0.02)
    return _host(t)


def _sample(params, opt):
    """Indices of: the first tensor (embedding), the last, a block-row matrix, a
    period-one matrix (if any), a 1-D tensor (norm or bias)."""
    periods = [opt.state[p]["automatic_period"] for _, p in params]
    dims = [p.dim() for _, p in params]
    pick = [0, len(params) - 1]
    for want in ("rows", "one", "vector"):
        for i, (P, d) in enumerate(zip(periods, dims)):
            if i in pick:
                continue
            if (want == "rows" and d == 2 and P > 1) or (want == "one" and d == 2 and P == 1) or \
                    (want == "vector" and d == 1):
                pick.append(i)
                break
    return sorted(pick)


def _compare(params, opt, ref, sample, dt, what, before):
    """before: each sampled tensor's oracle parameters before this step."""
    for k, i in enumerate(sample):
        name, p = params[i]
        st = opt.state[p]
        rs = ref.state[k]
        tag = "{} {} step {}".format(what, name, rs.step)
        np.testing.assert_array_equal(_host(st["m_codebook"]), rs.m_codebook, err_msg=tag + " indices")
        np.testing.assert_array_equal(_host(st["m_magnitude"]), rs.m_magnitude, err_msg=tag + " magnitudes")
        got_p, ref_p = _host(p), ref.params[k]["p"]
        got_v, ref_v = _host(st["vmean"]), rs.vmean
        if dt == "f32":
            np.testing.assert_allclose(got_v, ref_v, rtol=2.0 ** -18, atol=0, err_msg=tag + " vmean")
            np.testing.assert_allclose(got_p, ref_p, rtol=1e-5, atol=1e-7, err_msg=tag + " params")
            continue
        dv = tu.ulp_distance_bf16(got_v, ref_v)
        assert dv.max() <= 1, tag + " vmean"
        d = tu.ulp_distance_bf16(got_p, ref_p)
        far = np.nonzero(d > 1)[0]
        if far.size:
            # only where the row's vmean rounded the other way, within 2^-7 of the update
            rows = far // (p.numel() // got_v.size)
            assert np.all(dv[rows] == 1), (tag, far[:8])
            upd = np.abs(orc.to_f32(ref_p[far], "bf16").astype(np.float64) -
                         orc.to_f32(before[k][far], "bf16").astype(np.float64))
            diff = np.abs(orc.to_f32(got_p[far], "bf16").astype(np.float64) -
                          orc.to_f32(ref_p[far], "bf16").astype(np.float64))
            assert np.all(diff <= 2.0 ** -7 * upd + orc.ulp_bf16(ref_p[far])), (tag, far[:8])
        print(tag, "params: {} exact, {} of {} beyond one ulp (vmean rounding)".format(
            int((d == 0).sum()), far.size, d.size), flush=True)


def _run(config):
    import bench
    from gefen_amd.gefen import Gefen

    print("config", config, flush=True)
    cfg = bench.CONFIGS[config]
    dt = "f32" if cfg["dtype"] == torch.float32 else "bf16"
    dev = torch.device("cuda:0")
    params = bench.build_problem(cfg, dev)
    grads = [_host(p.grad) for _, p in params]
    opt = Gefen(params)
    opt.step()
    torch.cuda.synchronize()
    print("first step done; oracle periods and codebook", flush=True)
    periods = [opt.state[p]["automatic_period"] for _, p in params]
    ref_periods = [1 if g.size == 1 else orc.find_period(g, dt) for g in grads]
    bad = [(params[i][0], a, b) for i, (a, b) in enumerate(zip(periods, ref_periods)) if a != b]
    assert not bad, bad
    cb = opt._gefen_codebook.detach().cpu().numpy()
    ref_cb = orc.learn_codebook([(g, dt, P) for g, P in zip(grads, ref_periods)])
    np.testing.assert_array_equal(cb, ref_cb)
    sample = _sample(params, opt)
    kinds = {("one" if periods[i] == 1 else "rows") if params[i][1].dim() == 2 else "vector" for i in sample}
    assert {"rows", "vector"} <= kinds, sample
    arrs = [{"p": _initial(cfg, params, i), "dtype": dt, "shape": tuple(params[i][1].shape), "lr": 1e-3,
             "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 0.0} for i in sample]
    del grads
    ref = orc.GefenOracle(arrs, codebook=ref_cb)
    ref.periods = [ref_periods[i] for i in sample]
    # the first step of the sampled tensors from their initial values and gradients
    before = [a["p"].copy() for a in arrs]
    ref.step([_host(params[i][1].grad) for i in sample])
    _compare(params, opt, ref, sample, dt, config, before)
    for step in range(2, STEPS + 1):
        # the oracle takes the step from the GPU's parameters and state
        for k, i in enumerate(sample):
            p = params[i][1]
            st, rs = opt.state[p], ref.state[k]
            ref.params[k]["p"] = _host(p).copy()
            rs.m_codebook, rs.m_magnitude, rs.vmean = (_host(st["m_codebook"]).copy(),
                                                       _host(st["m_magnitude"]).copy(), _host(st["vmean"]).copy())
            assert rs.step == st["step"]
        for i, (_, p) in enumerate(params):
            bench.fill_grad(cfg, p.grad, i, step)
        opt.step()
        torch.cuda.synchronize()
        before = [a["p"].copy() for a in arrs]
        ref.step([_host(params[i][1].grad) for i in sample])
        _compare(params, opt, ref, sample, dt, config, before)
    print("sampled tensors", [(params[i][0], periods[i]) for i in sample], flush=True)


def test_gpt2_124m_fp32_full_config_matches_oracle():
    _run("gpt2")


def test_gpt2_124m_fp32_twenty_free_running_steps_match_oracle():
    """The GPT-2 124M fp32 configuration over 20 steps (a new gradient each step)
    with the oracle running on its own for the sampled tensors, never resynchronised
    from the GPU: the momentum state depends only on the gradients, so codebook
    indices and magnitudes stay bit-exact at every step, and the parameters meet
    the north star's bound after 20 steps (rtol 1e-5, atol 1e-7; the float32
    block mean of g^2 is summed in another order, within rtol 2^-18 per step)."""
    import bench
    from gefen_amd.gefen import Gefen

    cfg = bench.CONFIGS["gpt2"]
    dev = torch.device("cuda:0")
    params = bench.build_problem(cfg, dev)
    opt = Gefen(params)
    opt.step()
    torch.cuda.synchronize()
    sample = _sample(params, opt)
    grads = [_host(p.grad) for _, p in params]
    ref_cb = orc.learn_codebook([(g, "f32", opt.state[p]["automatic_period"]) for g, (_, p) in zip(grads, params)])
    np.testing.assert_array_equal(opt._gefen_codebook.detach().cpu().numpy(), ref_cb)
    arrs = [{"p": _initial(cfg, params, i), "dtype": "f32", "shape": tuple(params[i][1].shape), "lr": 1e-3,
             "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 0.0} for i in sample]
    ref = orc.GefenOracle(arrs, codebook=ref_cb)
    ref.step([grads[i] for i in sample])  # the oracle predicts its own periods
    del grads
    assert ref.periods == [opt.state[params[i][1]]["automatic_period"] for i in sample]
    for step in range(2, 21):
        for i, (_, p) in enumerate(params):
            bench.fill_grad(cfg, p.grad, i, step)
        opt.step()
        torch.cuda.synchronize()
        ref.step([_host(params[i][1].grad) for i in sample])
        for k, i in enumerate(sample):
            st = opt.state[params[i][1]]
            tag = "gpt2 {} step {}".format(params[i][0], step)
            np.testing.assert_array_equal(_host(st["m_codebook"]), ref.state[k].m_codebook, err_msg=tag)
            np.testing.assert_array_equal(_host(st["m_magnitude"]), ref.state[k].m_magnitude, err_msg=tag)
    for k, i in enumerate(sample):
        name, p = params[i]
        np.testing.assert_allclose(_host(p), ref.params[k]["p"], rtol=1e-5, atol=1e-7, err_msg=name + " params")
        np.testing.assert_allclose(_host(opt.state[p]["vmean"]), ref.state[k].vmean, rtol=2.0 ** -16, atol=0,
                                   err_msg=name + " vmean")
        err = np.abs(_host(p).astype(np.float64) - ref.params[k]["p"])
        print("gpt2", name, "period", ref.periods[k], "20 steps: indices and magnitudes exact; params max |diff|",
              float(err.max()), "= {:.3f} of the tolerance".format(
                  float(np.max(err / (1e-7 + 1e-5 * np.abs(ref.params[k]["p"]))))), flush=True)


def _free_running_bf16(config, steps):
    """config (bf16) at full size: periods and codebook against the oracle after the
    first step, then `steps` steps with the oracle running on its own for the
    sampled tensors (see the module docstring for the bars)."""
    import bench
    from gefen_amd.gefen import Gefen

    print("config", config, "free running for", steps, "steps", flush=True)
    cfg = bench.CONFIGS[config]
    dev = torch.device("cuda:0")
    params = bench.build_problem(cfg, dev)
    grads = [_host(p.grad) for _, p in params]
    opt = Gefen(params)
    opt.step()
    torch.cuda.synchronize()
    periods = [opt.state[p]["automatic_period"] for _, p in params]
    ref_periods = [1 if g.size == 1 else orc.find_period(g, "bf16") for g in grads]
    bad = [(params[i][0], a, b) for i, (a, b) in enumerate(zip(periods, ref_periods)) if a != b]
    assert not bad, bad
    ref_cb = orc.learn_codebook([(g, "bf16", P) for g, P in zip(grads, ref_periods)])
    np.testing.assert_array_equal(opt._gefen_codebook.detach().cpu().numpy(), ref_cb)
    print("periods and codebook match the oracle", flush=True)
    # the embedding, a block-row and a period-one matrix, a norm (the lm_head has the
    # embedding's shape and period: left out to keep the run within two minutes)
    sample = [i for i in _sample(params, opt) if i != len(params) - 1]
    kinds = {("one" if periods[i] == 1 else "rows") if params[i][1].dim() == 2 else "vector" for i in sample}
    assert {"rows", "one", "vector"} <= kinds, sample
    arrs = [{"p": _initial(cfg, params, i), "dtype": "bf16", "shape": tuple(params[i][1].shape), "lr": 1e-3,
             "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 0.0} for i in sample]
    ref = orc.GefenOracle(arrs, codebook=ref_cb)
    ref.periods = [ref_periods[i] for i in sample]
    ref_g = [grads[i] for i in sample]
    del grads
    flagged = [None] * len(sample)  # per sampled tensor: rows whose vmean has differed
    cum = [np.zeros(params[i][1].numel(), dtype=np.float32) for i in sample]  # the oracle's |update| sums there
    beyond_total = elems_total = 0
    for step in range(1, steps + 1):
        if step > 1:
            for i, (_, p) in enumerate(params):
                bench.fill_grad(cfg, p.grad, i, step)
            opt.step()
            torch.cuda.synchronize()
            ref_g = [_host(params[i][1].grad) for i in sample]
        before = [a["p"].copy() for a in arrs]
        ref.step(ref_g)
        for k, i in enumerate(sample):
            name, p = params[i]
            st, rs = opt.state[p], ref.state[k]
            tag = "{} {} step {}".format(config, name, step)
            assert rs.step == st["step"] == step, tag
            np.testing.assert_array_equal(_host(st["m_codebook"]), rs.m_codebook, err_msg=tag + " indices")
            np.testing.assert_array_equal(_host(st["m_magnitude"]), rs.m_magnitude, err_msg=tag + " magnitudes")
            got_v = _host(st["vmean"])
            dv = tu.ulp_distance_bf16(got_v, rs.vmean)
            assert dv.max() <= 2, tag + " vmean"
            flag = flagged[k] = (dv > 0) if flagged[k] is None else (flagged[k] | (dv > 0))
            ref_p = ref.params[k]["p"]
            per_row = ref_p.size // got_v.size
            # |update| of this step summed over the steps, in the flagged rows (elsewhere unused)
            frows = np.nonzero(flag)[0]
            if frows.size:
                fe = (frows[:, None] * per_row + np.arange(per_row)[None, :]).reshape(-1)
                cum[k][fe] += np.abs(orc.to_f32(ref_p[fe], "bf16") - orc.to_f32(before[k][fe], "bf16"))
            got_p = _host(p)
            off = np.nonzero(got_p != ref_p)[0]
            # outside the flagged rows: bit-exact
            outside = off[~flag[off // per_row]]
            assert outside.size == 0, (tag, outside[:8])
            d = tu.ulp_distance_bf16(got_p[off], ref_p[off])
            diff = np.abs(orc.to_f32(got_p[off], "bf16").astype(np.float64) -
                          orc.to_f32(ref_p[off], "bf16").astype(np.float64))
            bound = 2.0 ** -7 * cum[k][off].astype(np.float64) + step * orc.ulp_bf16(ref_p[off])
            assert np.all(diff <= bound), (tag, off[diff > bound][:8])
            if step == steps:
                nflag = int(frows.size)
                beyond = int((d > 1).sum())
                beyond_total += beyond
                elems_total += ref_p.size
                print("{}: period {}, {} of {} rows with a vmean that differed at some step, {} of {} elements "
                      "differ ({} beyond one ulp)".format(tag, periods[i], nflag, flag.size, off.size, ref_p.size,
                                                           beyond), flush=True)
                assert nflag <= max(1, 1e-2 * flag.size), tag
    print("{} after {} steps: {} of {} sampled elements beyond one bf16 ulp ({:.2e})".format(
        config, steps, beyond_total, elems_total, beyond_total / elems_total), flush=True)
    assert beyond_total <= 1e-3 * elems_total


def test_llama_1_5b_bf16_twenty_free_running_steps_match_oracle():
    _free_running_bf16("llama1.5b", 20)


def test_llama_8b_bf16_ten_free_running_steps_match_oracle():
    _free_running_bf16("llama8b", 10)


def test_full_size_period_scores_match_reference():
    """Every divisor's score and the chosen period of full-size config tensors
    (GPT-2 wte, 8B k_proj and down_proj), from the device scorer and from the
    oracle, against the reference's own (tests/golden/periods_full.npz)."""
    import bench
    from gefen_amd import synthetic as syn
    from gefen_amd.kernels.period_variance import period_scores_launch, period_scores_workspace_bytes
    from gefen_amd.partitioning import PeriodScorer

    data, meta = load("periods_full")
    for case in meta:
        cfg = bench.CONFIGS[case["config"]]
        g = torch.empty(tuple(case["shape"]), dtype=cfg["dtype"], device="cuda:0")
        bench.fill_grad(cfg, g, case["index"], 0)
        host = _host(g)
        assert syn.checksum(host) == case["checksum"], case["name"]
        divs = data[case["name"] + "/divisors"].tolist()
        ref_scores = data[case["name"] + "/scores"]
        dt = case["dtype"]
        np.testing.assert_allclose(orc.period_scores(host, dt, divs, mode=1), ref_scores, rtol=1e-13, atol=0,
                                   err_msg=case["name"] + " oracle")
        assert orc.find_period(host, dt) == case["period"], case["name"]
        flat = g.reshape(-1)
        ws = torch.empty(period_scores_workspace_bytes(flat.numel(), divs), dtype=torch.uint8, device="cuda:0")
        sc = torch.empty(len(divs) + 1, dtype=torch.float64, device="cuda:0")
        period_scores_launch(flat, divs, 1, 1e-12, sc, ws)
        got = sc.cpu().numpy()
        assert got[-1] == 0  # no invalid log input
        # float64 block sums in another order than numpy's pairwise sums: each block
        # mean within (log2 n + 1) 2^-53 max|log(x + 1e-12)|, max|log| <= 28 here
        bound = 2 * (np.log2(flat.numel()) + 2) * 2.0 ** -53 * 28.0
        assert np.all(np.abs(got[:-1] - ref_scores) <= bound), (case["name"], np.abs(got[:-1] - ref_scores).max())
        scorer = PeriodScorer(mode=1)
        scorer.add(flat, None, False)
        assert scorer.finish() == [case["period"]], case["name"]
        print(case["name"], "period", case["period"], flush=True)

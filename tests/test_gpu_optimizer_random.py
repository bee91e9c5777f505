"""Randomised optimizer-level parity: Gefen on the GPU against oracle.GefenOracle
(gefen.py:1399-1420 on the CPU path) over 8 steps of ~24 parameters of random
shapes and dtypes in three param groups, with the events a training loop
produces between steps:

* step 3: a group's lr changed (a scheduler writing group["lr"]);
* step 4: one parameter without a gradient (skipped; its state does not advance);
* step 5: its gradient back, and another group's weight decay turned on;
* step 6: a parameter's gradient replaced by a new tensor (set_to_none, then
  backward), so its address changes;
* step 7: a group's lr given as a 0-d float64 tensor.

The optimizer's cached step plan must take the new hyperparameters and gradient
addresses (steps 2, 3 and 6-8 run through it) and give way to the full step
where a parameter loses or regains its gradient (steps 4 and 5); both paths must
give the oracle's results.  Indices and magnitudes bit-exact at every step;
period-one vmean and parameters bit-exact;
block vmean of 16-bit state within one ulp, float32 within 2^-18 relative;
float32 parameters within rtol 1e-5 / atol 1e-7; 16-bit parameters within one
ulp except in rows whose vmean rounded the other way at some step (then within
2^-7 of the summed update plus one ulp per step)."""

import numpy as np
import pytest
import torch

import gpu_util as gu
from gefen_amd import synthetic as syn
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

STEPS = 8
SHAPES = [(64, 96), (128, 768), (768,), (2304,), (48, 1000), (1024, 12), (7, 13), (3072, 8), (1,), (256, 256),
          (96, 96), (2048, 4), (5, 4096), (500,), (33, 64), (640, 48)]


def _grad(seed, i, step, shape, dt):
    n = int(np.prod(shape))
    rows = shape[0] if len(shape) == 2 else 1
    g = syn.round_to(syn.row_scaled_normal(seed * 100 + i, step, rows, n // rows, -14, -5), dt).reshape(-1)
    return g.view(np.uint16) if g.dtype == np.float16 else g


@pytest.mark.parametrize("seed", [1, 2])
def test_random_training_loop_matches_oracle(seed):
    from gefen_amd.gefen import Gefen

    rng = np.random.default_rng(seed)
    specs = []
    for i in range(24):
        shape = SHAPES[rng.integers(len(SHAPES))]
        dt = ["bf16", "bf16", "f32", "f16"][rng.integers(4)]
        specs.append((shape, dt, int(rng.integers(3))))
    hyper = [{"lr": 2e-3, "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 0.0},
             {"lr": 1e-3, "betas": (0.85, 0.99), "eps": 1e-6, "weight_decay": 0.0},
             {"lr": 5e-4, "betas": (0.9, 0.95), "eps": 1e-8, "weight_decay": 0.1}]
    params, arrs = [], []
    for i, (shape, dt, grp) in enumerate(specs):
        p0 = syn.round_to(syn.normal(syn.make_key(seed, 500 + i), int(np.prod(shape))) * 0.02, dt)
        p0 = p0.view(np.uint16) if p0.dtype == np.float16 else p0
        t = gu.to_dev(p0, dt).reshape(shape)
        params.append(torch.nn.Parameter(t))
        h = hyper[grp]
        arrs.append({"p": p0.copy(), "dtype": dt, "shape": shape, "lr": h["lr"], "beta1": h["betas"][0],
                     "beta2": h["betas"][1], "eps": h["eps"], "weight_decay": h["weight_decay"]})
    groups = [{"params": [("p{}".format(i), params[i]) for i in range(len(specs)) if specs[i][2] == k], **hyper[k]}
              for k in range(3)]
    groups = [g for g in groups if g["params"]]
    opt = Gefen(groups)
    ref = orc.GefenOracle(arrs)
    skip = 5 % len(params)
    moved = [np.zeros(a["p"].size) for a in arrs]
    flags = [None] * len(arrs)
    for step in range(1, STEPS + 1):
        gi = {id(p): k for k, g in enumerate(opt.param_groups) for p in g["params"]}
        if step == 3:  # a scheduler halves group 0's lr
            opt.param_groups[0]["lr"] *= 0.5
        if step == 5:  # weight decay turned on for the second group
            opt.param_groups[min(1, len(opt.param_groups) - 1)]["weight_decay"] = 0.05
        if step == 7:  # lr as a 0-d float64 tensor
            opt.param_groups[-1]["lr"] = torch.tensor(float(opt.param_groups[-1]["lr"]), dtype=torch.float64)
        grads = []
        for i, (shape, dt, _) in enumerate(specs):
            g = _grad(seed, i, step, shape, dt)
            if step == 4 and i == skip:
                params[i].grad = None
                grads.append(None)
                continue
            gd = gu.to_dev(g, dt).reshape(shape)
            if params[i].grad is None or step == 6 and i == (skip + 1) % len(params):
                params[i].grad = gd.clone()       # a new gradient tensor (new address)
            else:
                params[i].grad.copy_(gd)
            grads.append(g)
        plan = opt._plan
        opt.step()
        kept = plan is not None and opt._plan is plan
        # the kept plan takes new hyperparameters and gradient addresses; a parameter
        # that loses or regains its gradient needs a new one
        assert kept == (step not in (1, 4, 5)), (step, kept)
        for i, p in enumerate(params):            # the oracle reads the groups' current settings
            grp = opt.param_groups[gi[id(p)]]
            arrs[i]["lr"] = float(grp["lr"])
            arrs[i]["weight_decay"] = float(grp["weight_decay"])
        before = [a["p"].copy() for a in arrs]
        ref.step(grads)
        torch.cuda.synchronize()
        beyond = 0
        for i, p in enumerate(params):
            dt = arrs[i]["dtype"]
            tag = "param {} {} {} step {}".format(i, dt, specs[i][0], step)
            with np.errstate(invalid="ignore"):
                moved[i] += np.abs(orc.to_f32(arrs[i]["p"], dt).astype(np.float64) -
                                   orc.to_f32(before[i], dt).astype(np.float64))
            rs = ref.state[i]
            st = opt.state[p]
            if rs is None:
                assert "m_codebook" not in st, tag
                continue
            assert st["step"] == rs.step, tag
            assert st["automatic_period"] == rs.period, tag
            np.testing.assert_array_equal(gu.to_np(st["m_codebook"]).reshape(-1), rs.m_codebook, err_msg=tag + " idx")
            np.testing.assert_array_equal(gu.to_np(st["m_magnitude"]).reshape(-1), rs.m_magnitude,
                                          err_msg=tag + " mag")
            gv = gu.to_np(st["vmean"]).reshape(-1)
            gp = gu.to_np(p.detach()).reshape(-1)
            if rs.period == 1:
                np.testing.assert_array_equal(gv, rs.vmean, err_msg=tag + " vmean")
                np.testing.assert_array_equal(gp, arrs[i]["p"], err_msg=tag + " params")
                continue
            if dt == "f32":
                np.testing.assert_allclose(gv, rs.vmean, rtol=2.0 ** -18, atol=0, err_msg=tag + " vmean")
                np.testing.assert_allclose(gp, arrs[i]["p"], rtol=1e-5, atol=1e-7, err_msg=tag + " params")
                continue
            dv = gu.ulps16(gv, rs.vmean)
            assert dv.max() <= 1, tag + " vmean"
            flags[i] = (dv == 1) if flags[i] is None else (flags[i] | (dv == 1))
            dp = gu.ulps16(gp, arrs[i]["p"])
            far = np.nonzero(dp > 1)[0]
            if far.size:
                assert np.all(flags[i][far // rs.period]), (tag, far[:8])
                diff = np.abs(orc.to_f32(gp[far], dt).astype(np.float64) -
                              orc.to_f32(arrs[i]["p"][far], dt).astype(np.float64))
                assert np.all(diff <= 2.0 ** -7 * moved[i][far] + rs.step * gu.ulp_at16(arrs[i]["p"][far], dt)), \
                    (tag, far[:8])
                beyond += far.size
        print("seed", seed, "step", step, "cached plan" if kept else "full step",
              "all", len(params), "parameters match the oracle;", beyond, "16-bit elements beyond one ulp",
              flush=True)

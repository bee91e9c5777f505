"""The cached step plans against the full step, bit for bit, under random
changes between steps.

Two optimizers start from the same parameters: one steps through its cached
plan wherever the plan still applies (_StepPlan for Gefen, _MuonPlan for
GefenMuon), the other takes the full step every time (its plan is dropped
before each step).  Between steps a seeded generator changes hyperparameters of
random groups (lr as a number or a 0-d float64 or float32 tensor; weight decay
on and off; Gefen's betas and eps; GefenMuon's momentum, Nesterov flag and
adjust_lr_fn), drops a gradient, brings it back, or replaces a gradient tensor.  After every step both optimizers' parameters and states
must be identical.  The full step itself is checked against the oracle by the
trajectory and randomised optimizer tests, so this pins the plans' refresh
logic to it."""

import numpy as np
import pytest
import torch

import gpu_util as gu
from gefen_amd import synthetic as syn

pytestmark = pytest.mark.gpu

STEPS = 10


def _grad(seed, i, step, shape, dt):
    n = int(np.prod(shape))
    rows = shape[0] if len(shape) == 2 else 1
    g = syn.round_to(syn.row_scaled_normal(seed * 100 + i, step, rows, n // rows, -14, -5), dt).reshape(-1)
    return gu.to_dev(g.view(np.uint16) if g.dtype == np.float16 else g, dt).reshape(shape)


def _pair(opt_cls, seed, shapes, dtypes, **kw):
    a, b = [], []
    for i, (shape, dt) in enumerate(zip(shapes, dtypes)):
        p0 = syn.round_to(syn.normal(syn.make_key(seed, 900 + i), int(np.prod(shape))) * 0.02, dt)
        t = gu.to_dev(p0.view(np.uint16) if p0.dtype == np.float16 else p0, dt).reshape(shape)
        a.append(torch.nn.Parameter(t.clone()))
        b.append(torch.nn.Parameter(t.clone()))
    return (a, opt_cls([("w{}".format(i), p) for i, p in enumerate(a)], **kw),
            b, opt_cls([("w{}".format(i), p) for i, p in enumerate(b)], **kw))


def _same(pa, oa, pb, ob, tag):
    for i, (x, y) in enumerate(zip(pa, pb)):
        assert torch.equal(x.detach().view(torch.uint8), y.detach().view(torch.uint8)), (tag, "param", i)
        sa, sb = oa.state[x], ob.state[y]
        assert sorted(sa) == sorted(sb), (tag, i)
        for k, v in sa.items():
            if torch.is_tensor(v):
                assert torch.equal(v.view(torch.uint8), sb[k].view(torch.uint8)), (tag, "state", i, k)
            else:
                assert v == sb[k], (tag, "state", i, k)


def _events(rng, opts, params, step, kind):
    """The same random change applied to both optimizers' groups / gradients."""
    ev = rng.integers(8)
    gi = int(rng.integers(len(opts[0].param_groups)))
    for opt in opts:
        g = opt.param_groups[gi]
        if ev == 0:
            g["lr"] = float(g["lr"]) * 0.7
        elif ev == 1:
            g["lr"] = torch.tensor(float(g["lr"]), dtype=torch.float64)
        elif ev == 2:
            g["weight_decay"] = 0.0 if g["weight_decay"] > 0 else 0.05
        elif ev == 3:
            g["lr"] = torch.tensor(float(g["lr"]), dtype=torch.float32)
        elif ev == 4 and kind == "gefen":
            g["beta1"], g["beta2"] = 0.85, 0.995
        elif ev == 4:
            g["momentum"] = 0.9
        elif ev == 5 and kind == "gefen":
            g["eps"] = 1e-6
        elif ev == 5:
            g["nesterov"] = not g["nesterov"]
        elif ev == 6 and kind == "muon":
            g["adjust_lr_fn"] = "match_rms_adamw" if g["adjust_lr_fn"] is None else None
    return ev, gi


def _run(kind, seed, shapes, dtypes, opt_cls, **kw):
    rng = np.random.default_rng(seed)
    pa, oa, pb, ob = _pair(opt_cls, seed, shapes, dtypes, **kw)
    dropped = None
    cached = 0
    for step in range(1, STEPS + 1):
        if step > 1:
            ev, gi = _events(rng, (oa, ob), (pa, pb), step, kind)
        else:
            ev, gi = -1, -1
        for i, (shape, dt) in enumerate(zip(shapes, dtypes)):
            g = _grad(seed, i, step, shape, dt)
            for ps in (pa, pb):
                if ev == 7 and i == gi and dropped is None:
                    ps[i].grad = None                  # dropped for this step
                elif ps[i].grad is None or (ev == 6 and kind == "gefen" and i == gi):
                    ps[i].grad = g.clone()             # a new gradient tensor
                else:
                    ps[i].grad.copy_(g)
        dropped = gi if ev == 7 and dropped is None else None
        plan = oa._plan
        oa.step()
        cached += int(plan is not None and oa._plan is plan)
        ob._plan = None
        ob.step()
        torch.cuda.synchronize()
        _same(pa, oa, pb, ob, (kind, seed, step, ev, gi))
    print(kind, "seed", seed, STEPS, "steps identical;", cached, "through the cached plan", flush=True)
    assert cached >= STEPS // 3


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_gefen_cached_plan_equals_full_steps(seed):
    from gefen_amd.gefen import Gefen

    shapes = [(64, 96), (768,), (128, 768), (48, 1000), (7, 13), (1,), (256, 256), (5, 4096), (2304,), (33, 64)]
    dtypes = ["bf16", "f32", "bf16", "f16", "bf16", "f32", "bf16", "bf16", "f16", "f32"]
    _run("gefen", seed, shapes, dtypes, Gefen, lr=2e-3, weight_decay=0.01)


@pytest.mark.parametrize("seed", [4, 5])
def test_gefen_muon_cached_plan_equals_full_steps(seed):
    from gefen_amd.gefen_muon import GefenMuon

    # stacks of the batched Newton-Schulz path and two matrices off it (one-matrix path)
    shapes = [(256, 512), (512, 256), (256, 512), (256, 256), (96, 200), (768, 256), (300, 64)]
    dtypes = ["bf16", "bf16", "bf16", "f32", "bf16", "bf16", "f32"]
    _run("muon", seed, shapes, dtypes, GefenMuon, lr=2e-3, weight_decay=0.01)

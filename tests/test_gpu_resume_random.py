"""Checkpoint and resume inside this build: an optimizer saved after a random
number of steps (state_dict, through torch.save / torch.load) and loaded into a
fresh optimizer over copies of the parameters continues exactly as the
uninterrupted run, bit for bit, for Gefen and GefenMuon (the uninterrupted run
steps through its cached plan; the resumed one starts without a plan).  Also a
load_state_dict into the running optimizer itself, which must drop its plan."""

import io

import numpy as np
import pytest
import torch

import gpu_util as gu
from gefen_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _grad(seed, i, step, shape, dt):
    n = int(np.prod(shape))
    rows = shape[0] if len(shape) == 2 else 1
    g = syn.round_to(syn.row_scaled_normal(seed * 100 + i, step, rows, n // rows, -14, -5), dt).reshape(-1)
    return gu.to_dev(g.view(np.uint16) if g.dtype == np.float16 else g, dt).reshape(shape)


def _params(seed, shapes, dtypes):
    out = []
    for i, (shape, dt) in enumerate(zip(shapes, dtypes)):
        p0 = syn.round_to(syn.normal(syn.make_key(seed, 700 + i), int(np.prod(shape))) * 0.02, dt)
        out.append(torch.nn.Parameter(gu.to_dev(p0.view(np.uint16) if p0.dtype == np.float16 else p0,
                                                dt).reshape(shape)))
    return out


def _equal(pa, pb, oa, ob, tag):
    for i, (x, y) in enumerate(zip(pa, pb)):
        assert torch.equal(x.detach().view(torch.uint8), y.detach().view(torch.uint8)), (tag, i)
        for k, v in oa.state[x].items():
            w = ob.state[y][k]
            if torch.is_tensor(v):
                assert torch.equal(v.view(torch.uint8), w.view(torch.uint8)), (tag, i, k)
            else:
                assert v == w, (tag, i, k)


def _run(kind, seed, shapes, dtypes, make):
    rng = np.random.default_rng(seed)
    steps = 8
    cut = int(rng.integers(1, steps - 1))
    pa = _params(seed, shapes, dtypes)
    oa = make(pa)
    pb = oa_b = None
    for step in range(1, steps + 1):
        for i, (shape, dt) in enumerate(zip(shapes, dtypes)):
            g = _grad(seed, i, step, shape, dt)
            pa[i].grad = g.clone()
            if pb is not None:
                pb[i].grad = g.clone()
        oa.step()
        if pb is not None:
            oa_b.step()
            torch.cuda.synchronize()
            _equal(pa, pb, oa, oa_b, (kind, seed, "resumed", step))
        if step == cut:
            buf = io.BytesIO()
            torch.save(oa.state_dict(), buf)
            buf.seek(0)
            pb = [torch.nn.Parameter(p.detach().clone()) for p in pa]
            oa_b = make(pb)
            oa_b.load_state_dict(torch.load(buf, weights_only=True))
            assert oa_b._plan is None
            _equal(pa, pb, oa, oa_b, (kind, seed, "loaded", step))
    # loading into the running optimizer drops its plan and changes nothing else
    sd = oa.state_dict()
    oa.load_state_dict(sd)
    assert oa._plan is None
    for i, (shape, dt) in enumerate(zip(shapes, dtypes)):
        g = _grad(seed, i, steps + 1, shape, dt)
        pa[i].grad = g.clone()
        pb[i].grad = g.clone()
    oa.step()
    oa_b.step()
    torch.cuda.synchronize()
    _equal(pa, pb, oa, oa_b, (kind, seed, "reloaded"))
    print(kind, "seed", seed, "saved after step", cut, "and resumed: identical through step", steps + 1, flush=True)


@pytest.mark.parametrize("seed", [1, 2])
def test_gefen_resume_equals_uninterrupted_run(seed):
    from gefen_amd.gefen import Gefen

    shapes = [(64, 96), (768,), (128, 768), (7, 13), (1,), (256, 256), (2304,)]
    dtypes = ["bf16", "f32", "bf16", "f16", "f32", "bf16", "f16"]
    _run("gefen", seed, shapes, dtypes,
         lambda ps: Gefen([("w{}".format(i), p) for i, p in enumerate(ps)], lr=2e-3, weight_decay=0.01))


@pytest.mark.parametrize("seed", [3])
def test_gefen_muon_resume_equals_uninterrupted_run(seed):
    from gefen_amd.gefen_muon import GefenMuon

    shapes = [(256, 512), (512, 256), (256, 256), (96, 200)]
    dtypes = ["bf16", "bf16", "f32", "bf16"]
    _run("muon", seed, shapes, dtypes,
         lambda ps: GefenMuon([("w{}".format(i), p) for i, p in enumerate(ps)], lr=2e-3, weight_decay=0.01))

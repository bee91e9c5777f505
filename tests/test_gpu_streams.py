"""Two optimizers stepping on two streams at once equal the same optimizers
stepped one after the other on the default stream, bit for bit.

Both optimizers hold period-one bf16 and f16 tensors (their stepsize tables
live in the device's shared table pool) with different betas and eps, so each
step rebuilds the pool's tables; the pool orders a call on one stream after the
last call on the other.  Gradients are written on each optimizer's stream right
before its step, and nothing synchronises between the steps of the two streams."""

import numpy as np
import pytest
import torch

import gpu_util as gu
from gefen_amd import synthetic as syn

pytestmark = pytest.mark.gpu

STEPS = 6
SHAPES = [(256, 64), (4096,), (96, 128), (512, 40), (64, 96)]
DTYPES = ["bf16", "f16", "bf16", "f16", "f32"]


def _make(seed, betas, eps):
    from gefen_amd.gefen import Gefen

    ps = []
    for i, (shape, dt) in enumerate(zip(SHAPES, DTYPES)):
        t = torch.empty(shape, dtype=gu.TORCH[dt], device="cuda:0")
        syn.fill_device(t, seed, 500 + i, syn.KIND_NORMAL, mult=0.02)
        ps.append(torch.nn.Parameter(t))
    return ps, Gefen([("w{}".format(i), p) for i, p in enumerate(ps)], lr=2e-3, betas=betas, eps=eps,
                     weight_decay=0.01)


def _grads(ps, seed, step):
    for i, p in enumerate(ps):
        if p.grad is None:
            p.grad = torch.empty_like(p)
        # one scale per tensor: no row structure, so the periods come out as one
        syn.fill_device(p.grad, seed, step * 1000 + i, syn.KIND_ROW_SCALED, cols=p.numel(), e_lo=-8, e_hi=-8)


def _state(ps, opt):
    out = []
    for p in ps:
        out.append(p.detach().clone())
        for k in ("m_codebook", "m_magnitude", "vmean"):
            out.append(opt.state[p][k].clone())
    return out


def test_two_optimizers_on_two_streams_equal_sequential_steps():
    settings = [((0.9, 0.999), 1e-8, 11), ((0.85, 0.99), 1e-6, 12)]
    # sequential on the default stream
    seq = [_make(seed, betas, eps) for betas, eps, seed in settings]
    for step in range(1, STEPS + 1):
        for (ps, opt), (_, _, seed) in zip(seq, settings):
            _grads(ps, seed, step)
            opt.step()
            torch.cuda.synchronize()
    periods = [[opt.state[p]["automatic_period"] for p in ps] for ps, opt in seq]
    assert all(1 in pp for pp in periods), periods
    # the same two optimizers on two streams, interleaved without synchronisation
    par = [_make(seed, betas, eps) for betas, eps, seed in settings]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for step in range(1, STEPS + 1):
        for (ps, opt), (_, _, seed), s in zip(par, settings, streams):
            with torch.cuda.stream(s):
                _grads(ps, seed, step)
                opt.step()
    torch.cuda.synchronize()
    for k, ((pa, oa), (pb, ob)) in enumerate(zip(seq, par)):
        for i, (x, y) in enumerate(zip(_state(pa, oa), _state(pb, ob))):
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), (k, i)
    print("periods", periods, "; two streams equal the sequential run", flush=True)

"""Local-shard handling of the reference (gefen.py:163-168, 692-706, 789-810),
on one GPU with tensor subclasses standing in for torch's distributed types:

* a DTensor-like parameter and gradient (``to_local()``, ``placements``,
  ``device_mesh``, ``from_local``): the step runs on the local tensors;
* an AsyncCollectiveTensor-like gradient (``wait()``);
* a gradient whose storage is "not allocated yet" until written (FSDP's lazily
  materialised gradients): the period scoring catches the error, materialises it
  with add_(0) and scores again.

The plain-tensor run is checked against the CPU oracle (GefenOracle /
GefenMuonOracle on the same inputs: periods, learned codebook, codebook indices
and magnitudes bit-exact; fp32 parameters within rtol 1e-5 / atol 1e-7, bf16
within one ulp outside rows whose vmean rounded the other way; GefenMuon
parameters within 5% of the update norm, the bound its Newton-Schulz products
allow, tests/test_gpu_optimizer.py), and every wrapped case must give the same
parameters and state as the plain run, bit for bit."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


class LocalShard(torch.Tensor):
    """DTensor stand-in whose local shard is the whole tensor."""
    placements = ("Shard(dim=0)",)
    device_mesh = "mesh(1 rank)"

    @staticmethod
    def __new__(cls, data, requires_grad=False):
        return torch.Tensor._make_subclass(cls, data, requires_grad)

    def to_local(self):
        return self.as_subclass(torch.Tensor)

    @classmethod
    def from_local(cls, local, device_mesh, placements):
        return cls(local)


class Pending(torch.Tensor):
    """AsyncCollectiveTensor stand-in: wait() gives the finished tensor."""

    @staticmethod
    def __new__(cls, data):
        return torch.Tensor._make_subclass(cls, data, False)

    def wait(self):
        return self.as_subclass(torch.Tensor)


def make_lazy_class():
    class Lazy(torch.Tensor):
        """A gradient whose data is 'not allocated yet' until an in-place write."""
        allocated = False
        touched_before_allocation = 0

        @staticmethod
        def __new__(cls, data):
            return torch.Tensor._make_subclass(cls, data, False)

        def data_ptr(self):
            if not type(self).allocated:
                type(self).touched_before_allocation += 1
                raise RuntimeError("The tensor has a non-zero number of elements, but its data is not allocated yet.")
            return super().data_ptr()

        def add_(self, other, *args, **kwargs):
            type(self).allocated = True
            return super().add_(other, *args, **kwargs)

    return Lazy


SHAPES = [(64, 96), (200,), (128, 48)]


def _inputs(dtype, step):
    g = torch.Generator().manual_seed(100 + step)
    return [(torch.randn(s, generator=g) * 1e-3).to(dtype).cuda() for s in SHAPES]


def _params(dtype):
    g = torch.Generator().manual_seed(7)
    return [(torch.randn(s, generator=g) * 0.02).to(dtype).cuda() for s in SHAPES]


def _run(opt_cls, dtype, wrap_param, wrap_grad, steps=3, **kw):
    raw = _params(dtype)
    params = [wrap_param(t).requires_grad_(True) for t in raw]
    opt = opt_cls([("t{}".format(i), p) for i, p in enumerate(params)], **kw)
    for step in range(steps):
        for p, g in zip(params, _inputs(dtype, step)):
            p.grad = wrap_grad(g)
        opt.step()
    torch.cuda.synchronize()
    return params, opt


def _oracle_check(params, opt, dtype, steps=3, muon=False):
    """The plain-tensor run (params, opt) against the CPU oracle on the same inputs."""
    import gpu_util as gu
    import traj_util as tu
    from oracle import oracle as orc

    dt = "bf16" if dtype == torch.bfloat16 else "f32"
    p0 = [gu.to_np(t).reshape(-1) for t in _params(dtype)]
    g0 = opt.param_groups[0]
    if muon:
        arrs = [{"p": p.copy(), "dtype": dt, "shape": s, "lr": g0["lr"], "beta1": g0["momentum"], "beta2": 0.0,
                 "eps": g0["eps"], "weight_decay": g0["weight_decay"]} for p, s in zip(p0, SHAPES)]
        ref = orc.GefenMuonOracle(arrs, momentum=g0["momentum"], nesterov=g0["nesterov"],
                                  ns_coefficients=tuple(g0["ns_coefficients"]), ns_steps=g0["ns_steps"],
                                  eps=g0["eps"], adjust_lr_fn=g0["adjust_lr_fn"])
    else:
        arrs = [{"p": p.copy(), "dtype": dt, "shape": s, "lr": g0["lr"], "beta1": g0["beta1"], "beta2": g0["beta2"],
                 "eps": g0["eps"], "weight_decay": g0["weight_decay"]} for p, s in zip(p0, SHAPES)]
        ref = orc.GefenOracle(arrs)
    for step in range(steps):
        ref.step([gu.to_np(g).reshape(-1) for g in _inputs(dtype, step)])
    np.testing.assert_array_equal(opt._gefen_codebook.detach().cpu().numpy(), ref.codebook)
    for i, (prm, t) in enumerate(zip(arrs, params)):
        st = opt.state[t]
        assert st["automatic_period"] == ref.periods[i], i
        np.testing.assert_array_equal(gu.to_np(st["m_codebook"]).reshape(-1), ref.state[i].m_codebook)
        np.testing.assert_array_equal(gu.to_np(st["m_magnitude"]).reshape(-1), ref.state[i].m_magnitude)
        got = gu.to_np(t.to_local() if hasattr(t, "to_local") else t).reshape(-1)
        if muon:
            ours = orc.to_f32(got, dt).astype(np.float64) - orc.to_f32(p0[i], dt)
            theirs = orc.to_f32(prm["p"], dt).astype(np.float64) - orc.to_f32(p0[i], dt)
            rel = np.linalg.norm(ours - theirs) / max(np.linalg.norm(theirs), 1e-30)
            print("local shard oracle: muon p{} relative update error {:.3g}".format(i, rel), flush=True)
            assert rel <= 0.05, (i, rel)
        elif dt == "f32":
            np.testing.assert_allclose(got, prm["p"], rtol=1e-5, atol=1e-7)
        else:
            d = tu.ulp_distance_bf16(got, prm["p"])
            far = np.nonzero(d > 1)[0]
            if far.size:  # only in rows whose bf16 vmean rounded the other way
                vm = gu.to_np(st["vmean"]).reshape(-1)
                dv = tu.ulp_distance_bf16(vm, ref.state[i].vmean)
                assert np.all(dv[far // (got.size // vm.size)] > 0), (i, far[:8])
            print("local shard oracle: p{} period {}: {} of {} elements exact, {} beyond one ulp".format(
                i, ref.periods[i], int((d == 0).sum()), d.size, far.size), flush=True)


def _same(a_params, a_opt, b_params, b_opt):
    for pa, pb in zip(a_params, b_params):
        la = pa.to_local() if hasattr(pa, "to_local") else pa
        lb = pb.to_local() if hasattr(pb, "to_local") else pb
        assert torch.equal(la.detach().view(torch.int16 if la.dtype != torch.float32 else torch.int32),
                           lb.detach().view(torch.int16 if lb.dtype != torch.float32 else torch.int32))
        sa, sb = a_opt.state[pa], b_opt.state[pb]
        assert sa["automatic_period"] == sb["automatic_period"] and sa["step"] == sb["step"]
        for k in ("m_codebook", "m_magnitude", "vmean"):
            if k in sa:
                assert torch.equal(sa[k], sb[k]), k


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dtensor_like_parameters_and_gradients(dtype):
    from gefen_amd.gefen import Gefen

    base = _run(Gefen, dtype, lambda t: t, lambda g: g)
    _oracle_check(*base, dtype)
    shard = _run(Gefen, dtype, lambda t: LocalShard(t), lambda g: LocalShard(g))
    assert all(type(p) is LocalShard for p in shard[0])
    _same(*base, *shard)
    _oracle_check(*shard, dtype)


def test_waitable_gradients():
    from gefen_amd.gefen import Gefen

    base = _run(Gefen, torch.bfloat16, lambda t: t, lambda g: g)
    _oracle_check(*base, torch.bfloat16)
    waited = _run(Gefen, torch.bfloat16, lambda t: t, lambda g: Pending(g))
    _same(*base, *waited)


def test_lazily_materialised_gradient_is_added_zero_and_rescored():
    from gefen_amd.gefen import Gefen

    Lazy = make_lazy_class()
    base = _run(Gefen, torch.bfloat16, lambda t: t, lambda g: g, steps=1)
    _oracle_check(*base, torch.bfloat16, steps=1)
    lazy = _run(Gefen, torch.bfloat16, lambda t: t, lambda g: Lazy(g), steps=1)
    assert Lazy.allocated and Lazy.touched_before_allocation == 1
    _same(*base, *lazy)


def test_gefen_muon_with_dtensor_like_parameters():
    from gefen_amd.gefen_muon import GefenMuon

    global SHAPES
    saved = SHAPES
    SHAPES = [(64, 96), (128, 48)]  # GefenMuon: 2-D parameters only
    try:
        base = _run(GefenMuon, torch.bfloat16, lambda t: t, lambda g: g)
        _oracle_check(*base, torch.bfloat16, muon=True)
        shard = _run(GefenMuon, torch.bfloat16, lambda t: LocalShard(t), lambda g: LocalShard(g))
        _same(*base, *shard)
    finally:
        SHAPES = saved


def test_dequantised_momentum_keeps_the_dtensor_type():
    """gefen_dequantize_unpacked_indices (gefen.py:146-169) wraps the coefficients
    of a DTensor-like tensor back with from_local."""
    from gefen_amd.gefen import gefen_dequantize_unpacked_indices

    cb = torch.linspace(-1, 1, 16, device="cuda:0")
    idx = torch.randint(0, 16, (8, 4), dtype=torch.uint8, device="cuda:0")
    like = LocalShard(torch.zeros(8, 4, dtype=torch.bfloat16, device="cuda:0"))
    out = gefen_dequantize_unpacked_indices(cb, idx, like)
    assert type(out) is LocalShard and out.dtype == torch.bfloat16
    assert torch.equal(out.to_local(), cb[idx.long()].to(torch.bfloat16))

"""The reference's import surface (ndvbd/Gefen 1.2.3 __init__.py:1-13,
kernels/gefen_cuda.py:6-22, kernels/period_variance.py:49-72): code written
against the reference imports this implementation by the reference's names."""

import importlib

import numpy as np
import pytest
import torch

BINDING = ["automatic_gefen_fused_update_cuda", "automatic_gefen_fused_update_from_vmean_cuda",
           "automatic_gefen_period1_update_cuda", "automatic_gefen_muon_momentum_cuda",
           "automatic_vmean_update_cuda", "gefen_exact_histogram_cuda", "average_within_block_variance_cuda",
           "average_within_block_coefficient_of_variation_cuda", "average_adjacent_log_block_mean_difference_cuda",
           "gefen_lloyd_accumulate_cuda", "gefen_lloyd_mse_cuda"]


def test_reference_module_names_resolve_to_this_implementation():
    from gefen import Gefen, GefenMuon  # noqa: F401
    import gefen
    import gefen_amd

    assert gefen.Gefen is gefen_amd.Gefen and gefen.GefenMuon is gefen_amd.GefenMuon
    for ref, impl in [("gefen.gefen", "gefen_amd.gefen"), ("gefen.gefen_muon", "gefen_amd.gefen_muon"),
                      ("gefen.partitioning", "gefen_amd.partitioning"),
                      ("gefen.quantization", "gefen_amd.quantization"),
                      ("gefen.kernels.gefen_cuda", "gefen_amd.kernels.gefen_hip"),
                      ("gefen.kernels.automatic_gefen_fused", "gefen_amd.kernels.automatic_gefen_fused"),
                      ("gefen.kernels.automatic_vmean", "gefen_amd.kernels.automatic_vmean"),
                      ("gefen.kernels.exact_histogram_fused", "gefen_amd.kernels.exact_histogram_fused"),
                      ("gefen.kernels.period_variance", "gefen_amd.kernels.period_variance"),
                      ("gefen.kernels.lloyd_max_fused", "gefen_amd.kernels.lloyd_max_fused")]:
        assert importlib.import_module(ref) is importlib.import_module(impl), ref
    # the implementation keeps its own module spec
    assert importlib.import_module("gefen.gefen").__spec__.name == "gefen_amd.gefen"
    # module switches set through the reference name are the optimizer's
    import gefen.gefen as gg
    old = gg.FIND_PERIOD_BACKEND
    try:
        gg.FIND_PERIOD_BACKEND = "cuda"
        assert gefen_amd.gefen.FIND_PERIOD_BACKEND == "cuda"
    finally:
        gg.FIND_PERIOD_BACKEND = old
    from gefen.gefen_muon import _adjust_lr, _zeropower_via_newtonschulz  # noqa: F401
    from gefen.partitioning import divisors, find_period_by_block_variance  # noqa: F401
    from gefen.quantization import exact_dp  # noqa: F401


def test_load_extension_exposes_the_binding_functions():
    from gefen.kernels.gefen_cuda import load_extension

    ext = load_extension()
    assert ext is load_extension()
    for name in BINDING:
        assert callable(getattr(ext, name)), name
    assert callable(ext.gefen_step_tasks)  # and the C ABI beside them


def test_custom_op_is_registered():
    import gefen.kernels.period_variance as pv

    assert pv._OPAQUE_OP_AVAILABLE
    assert hasattr(torch.ops.gefen, "average_within_block_variance_cuda")


@pytest.mark.gpu
def test_step_and_custom_op_through_reference_names():
    from gefen import Gefen
    from gefen.kernels.gefen_cuda import load_extension

    torch.manual_seed(0)
    w = (torch.randn(64, 96) * 0.02).to(torch.bfloat16).cuda().requires_grad_(True)
    opt = Gefen([("w", w)])
    w0 = w.detach().clone()
    for _ in range(2):
        w.grad = (torch.randn(64, 96) * 1e-3).to(torch.bfloat16).cuda()
        opt.step()
    assert not torch.equal(w.detach(), w0) and opt.state[w]["step"] == 2
    v = (torch.randn(32 * 48) * 1e-2).cuda()
    ext = load_extension()
    var = ext.average_within_block_variance_cuda(v, 48, False)
    assert var.dtype == torch.float64 and var.shape == (1,)
    op = torch.ops.gefen.average_within_block_variance_cuda(v, 48, False)
    assert torch.equal(op, var)
    x = (v.double().cpu() ** 2).reshape(32, 48)
    ref = float(torch.sqrt(((x * x).mean(1) - x.mean(1) ** 2).clamp(min=0).mean()))
    assert abs(float(var.item()) - ref) <= 1e-4 * ref
    adj = ext.average_adjacent_log_block_mean_difference_cuda(v, 48, False, 1e-12)
    assert adj.dim() == 0 and adj.dtype == torch.float64

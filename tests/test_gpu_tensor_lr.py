"""A tensor learning rate with weight decay (gefen.py:1280-1281,
gefen_muon.py:325-326: p.mul_(1 - lr * wd)): torch forms the decay factor in the
tensor's dtype, fl32(1 - fl32(lr * fl32(wd))) for a float32 lr, which differs
from the double expression (float)(1 - lr * wd) in about 1% of cases.  The
optimizer hands the kernels the weight decay for which their factor is torch's
(gefen._kernel_weight_decay), so such steps keep the cached plan; the rest of
the step is the ordinary one."""

import numpy as np
import pytest
import torch

import gpu_util as gu
import traj_util as tu
from golden_util import load
from gefen_amd import synthetic as syn
from oracle import oracle as orc


def torch_decay_factor(lr: float, wd: float) -> np.float32:
    return np.float32(np.float32(1.0) - np.float32(np.float32(lr) * np.float32(wd)))


def test_decay_factor_model_matches_torch():
    rng = np.random.default_rng(5)
    lrs = rng.uniform(1e-5, 1e-1, 4000)
    wds = rng.uniform(1e-3, 0.5, 4000)
    differs = 0
    for lr, wd in zip(lrs, wds):
        f = (1 - torch.tensor(float(lr), dtype=torch.float32) * float(wd)).item()
        assert np.float32(f) == torch_decay_factor(lr, wd)
        differs += np.float32(f) != np.float32(1.0 - float(np.float32(lr)) * float(wd))
    assert differs > 0  # the double formula would be wrong somewhere in this sample


def _pick_lr_wd():
    """An (lr, wd) pair whose tensor factor differs from the double formula."""
    rng = np.random.default_rng(9)
    while True:
        lr, wd = float(np.float32(rng.uniform(1e-3, 5e-2))), float(rng.uniform(0.05, 0.5))
        if torch_decay_factor(lr, wd) != np.float32(1.0 - lr * wd):
            return lr, wd


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_gefen_tensor_lr_weight_decay_matches_oracle(dtype):
    from gefen_amd.gefen import Gefen

    lr, wd = _pick_lr_wd()
    data, _ = load("exact_dp")
    cb = data["hist_k256_forced/codebook"]
    shapes = [(64, 96), (200,), (32, 48)]
    tensors, arrs = [], []
    for i, shape in enumerate(shapes):
        n = int(np.prod(shape))
        p0 = syn.round_to(syn.normal(syn.make_key(21, i), n) * 0.02, dtype)
        tensors.append(gu.to_dev(p0, dtype).reshape(shape).requires_grad_(True))
        arrs.append({"p": p0.copy(), "dtype": dtype, "shape": shape, "lr": lr, "beta1": 0.9, "beta2": 0.999,
                     "eps": 1e-8, "weight_decay": 0.0})
    opt = Gefen([("t{}".format(i), t) for i, t in enumerate(tensors)], lr=torch.tensor(lr, dtype=torch.float32),
                weight_decay=wd)
    opt._gefen_codebook = torch.from_numpy(cb).to("cuda:0")
    ref = orc.GefenOracle(arrs, codebook=cb)
    fac = torch_decay_factor(lr, wd)
    planned = 0
    for step in range(1, 4):
        grads = []
        for i, (t, shape) in enumerate(zip(tensors, shapes)):
            rows = shape[0] if len(shape) > 1 else 1
            g = syn.round_to(syn.row_scaled_normal(21, 100 * step + i, rows, t.numel() // rows, -14, -4), dtype)
            grads.append(g.reshape(-1))
            t.grad = gu.to_dev(g.reshape(-1), dtype).reshape(shape)
        planned += opt._plan is not None
        opt.step()
        # the oracle step with the decay applied first with torch's factor
        for prm in arrs:
            prm["p"][...] = orc.from_f32(orc.to_f32(prm["p"], dtype) * fac, dtype)
        ref.step(grads)
    torch.cuda.synchronize()
    for i, t in enumerate(tensors):
        got = gu.to_np(t).reshape(-1)
        np.testing.assert_array_equal(gu.to_np(opt.state[t]["m_codebook"]).reshape(-1), ref.state[i].m_codebook)
        if dtype == "bf16":
            assert tu.ulp_distance_bf16(got, arrs[i]["p"]).max() <= 1
        else:
            np.testing.assert_allclose(got, arrs[i]["p"], rtol=1e-5, atol=1e-7)
    assert planned == 2  # the tensor lr with weight decay keeps the cached plan from the second step on

"""Checkpoint interop (gefen.py:1343-1397): a state dict in the reference's
format, holding the reference's own state after step 2 (m_codebook, m_magnitude,
vmean, automatic_period, period_one_divisor, gefen_codebook, gefen_global_step,
from the trajectory fixtures), is loaded into the GPU optimizer, which then
continues the reference's trajectory to step 20.

torch's Optimizer.load_state_dict casts every floating parameter's state tensors
to the parameter's dtype, the uint8 indices included; the reference's
load_state_dict (gefen.py:1372-1397) then restores each saved tensor's own dtype.
The F_FP32 case (float32 state for bf16 parameters) and the uint8 indices check
that restoration."""

import numpy as np
import pytest
import torch

import gpu_util as gu
import traj_util as tu
from test_gpu_optimizer import _build_gefen

pytestmark = pytest.mark.gpu

TORCH_DTYPE = {"torch.uint8": torch.uint8, "torch.float32": torch.float32, "torch.bfloat16": torch.bfloat16,
               "torch.float16": torch.float16}


def reference_state_dict(data, meta, step):
    """The reference's state_dict() after `step` steps, rebuilt from the fixture:
    tensors on the CPU in their saved dtypes (as torch.load(map_location="cpu")
    returns them), plain values from the recorded layout."""
    layout = meta["state_dict"]
    state = {}
    for pid, entries in layout["state"].items():
        i = int(pid)
        st = {}
        for key, e in entries.items():
            if e["tensor"]:
                arr = np.ascontiguousarray(tu.bits(data["s{}/{}/step{}".format(i, key, step)]).reshape(e["shape"]))
                dt = TORCH_DTYPE[e["dtype"]]
                if dt in (torch.bfloat16, torch.float16):  # 16-bit floats are stored as their bits
                    st[key] = torch.from_numpy(arr.view(np.int16)).view(dt)
                else:
                    st[key] = torch.from_numpy(arr)
                assert st[key].dtype == dt, key
            elif key == "step":
                st[key] = step
            elif e["type"] == "tuple":
                st[key] = tuple(e["value"])
            else:
                st[key] = e["value"]
        state[i] = st
    groups = [{k: (tuple(v) if isinstance(v, list) and k != "params" else v) for k, v in g.items()}
              for g in layout["param_groups"]]
    return {"state": state, "param_groups": groups, "gefen_global_step": step,
            "gefen_codebook": torch.from_numpy(np.ascontiguousarray(data["codebook_out"], dtype=np.float32))}


@pytest.mark.parametrize("name", ["llamamini_bf16", "gpt2mini_f32", "fp16mini", "groups_f32",
                                  "llamamini_bf16_f32state"])
def test_reference_checkpoint_continues_the_reference_trajectory(name, monkeypatch):
    from gefen_amd import gefen as gefen_mod

    print("checkpoint", name, flush=True)
    data, meta, params, skip = tu.build(name)
    dtype = meta["dtype"]
    sdtype = "f32" if meta.get("f_fp32") else dtype
    if meta.get("f_fp32"):
        monkeypatch.setattr(gefen_mod, "F_FP32", True)
    tensors = [gu.to_dev(tu.bits(data["p{}/step2".format(i)]).reshape(-1), dtype).reshape(prm["shape"]).clone()
               .requires_grad_(True) for i, prm in enumerate(params)]
    opt = _build_gefen(meta, tensors, params)
    opt.load_state_dict(reference_state_dict(data, meta, 2))
    assert opt._gefen_global_step == 2
    for i, t in enumerate(tensors):
        st = opt.state[t]
        assert st["m_codebook"].dtype == torch.uint8 and st["m_codebook"].is_cuda
        assert st["m_magnitude"].dtype == gu.TORCH[sdtype] and st["vmean"].dtype == gu.TORCH[sdtype]
        assert st["step"] == 2 and st["automatic_period"] == int(data["periods"][i])
    for step in range(3, meta["steps"] + 1):
        grads = tu.grads_for(meta, params, step, skip)
        for t, g, prm in zip(tensors, grads, params):
            t.grad = None if g is None else gu.to_dev(g.reshape(-1), dtype).reshape(prm["shape"])
        opt.step()
        if step in (5, 10, 20):
            for i, t in enumerate(tensors):
                got = gu.to_np(t).reshape(-1)
                ref = tu.bits(data["p{}/step{}".format(i, step)]).reshape(-1)
                if dtype == "f32":
                    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-7, err_msg="{} p{} {}".format(name, i, step))
                else:  # 16-bit sign-magnitude formats: distance in units in the last place
                    d = tu.ulp_distance_bf16(got, ref)
                    assert d.max() <= 1, "{} p{} step {}: {} ulps".format(name, i, step, d.max())
    assert opt._gefen_global_step == meta["steps"]
    for i, t in enumerate(tensors):
        st = opt.state[t]
        for key in ("m_codebook", "m_magnitude"):
            np.testing.assert_array_equal(gu.to_np(st[key]).reshape(-1),
                                          tu.bits(data["s{}/{}/step20".format(i, key)]).reshape(-1), err_msg=key)
        vg = gu.to_np(st["vmean"]).reshape(-1)
        vr = tu.bits(data["s{}/vmean/step20".format(i)]).reshape(-1)
        if sdtype == "f32":
            np.testing.assert_allclose(vg, vr, rtol=4e-6, atol=0)
        else:
            assert tu.ulp_distance_bf16(vg, vr).max() <= 1

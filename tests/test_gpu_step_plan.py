"""gefen_step_plan (the kept launches of the optimizer's cached plan) against
gefen_step_tasks, through the C ABI: parameters, codebook indices, magnitudes
and vmean bit-identical over several steps, including the runs that must leave
the kept launches (new gradient buffers, a misaligned gradient, tasks whose
stepsize tables differ inside one launch, a row naming other state tensors,
a table of another length), and the timing events around a run.  gefen_step_tasks
itself is checked against the oracle in test_gpu_step.py."""

import ctypes

import numpy as np
import pytest
import torch

import gpu_util as gu
from golden_util import load
from gefen_amd import _lib
from gefen_amd import synthetic as syn

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}

# (dtype, numel, period): period-one bf16 and f16 states (stepsize tables), block
# rows of several kernel shapes, a long row (two-sweep kernel), fp32, and enough
# small tensors of one shape that the plan has several launches of one key, some
# on the side stream beside the large ones
SPECS = ([("bf16", 1 << 21, 1), ("bf16", 96 * 2048, 2048), ("f32", 48 * 768, 768), ("f16", 3 * 4096, 1),
          ("bf16", 5000 * 6, 5000), ("f32", 4096, 1), ("bf16", 64 * 300, 64)]
         + [("bf16", 2048, 1)] * 34 + [("f32", 768, 768)] * 3)


def _tables(lib):
    data, _ = load("exact_dp")
    cb = torch.from_numpy(data["hist_k256_forced/codebook"]).to("cuda:0")
    tables = torch.empty(int(lib.gefen_codebook_tables_size()), dtype=torch.uint8, device="cuda:0")
    _lib.check(lib.gefen_prepare_codebook(cb.data_ptr(), cb.numel(), tables.data_ptr(), gu.stream()))
    return tables


class Set:
    """Parameters and state of every spec on the device (one copy per entry point)."""

    def __init__(self, seed):
        self.ps, self.states = [], []
        for i, (dt, n, period) in enumerate(SPECS):
            p = syn.round_to(syn.normal(syn.make_key(seed, i), n) * 0.02, dt)
            self.ps.append(gu.to_dev(p, dt))
            pod = max(d for d in range(1, 257) if n % d == 0) if period == 1 else 0
            rows = n // (pod if period == 1 else period)
            self.states.append({"idx": torch.zeros(n, dtype=torch.uint8, device="cuda:0"),
                                "mag": torch.zeros(rows, dtype=DT[dt], device="cuda:0"),
                                "vmean": torch.zeros(n // period, dtype=DT[dt], device="cuda:0"), "pod": pod})

    def tasks(self, grads, steps, lr=1e-3):
        t = np.zeros(len(SPECS), dtype=_lib.STEP_TASK)
        for i, ((dt, n, period), p, g, st) in enumerate(zip(SPECS, self.ps, grads, self.states)):
            t[i]["p"], t[i]["grad"] = p.data_ptr(), g.data_ptr()
            t[i]["m_codebook"], t[i]["m_magnitude"], t[i]["vmean"] = (st["idx"].data_ptr(), st["mag"].data_ptr(),
                                                                       st["vmean"].data_ptr())
            t[i]["numel"], t[i]["period"], t[i]["period_one_divisor"] = n, period, st["pod"]
            t[i]["param_dtype"] = t[i]["state_dtype"] = gu.CODE[dt]
            t[i]["beta1"], t[i]["beta2"], t[i]["lr"], t[i]["eps"] = 0.9, 0.999, lr, 1e-8
            t[i]["weight_decay"] = 0.01 if i % 3 == 1 else 0.0
            t[i]["bias_correction_1"] = 1 - 0.9 ** steps[i]
            t[i]["bias_correction_2"] = 1 - 0.999 ** steps[i]
        return t

    def host(self):
        return ([gu.to_np(p) for p in self.ps],
                [{k: gu.to_np(v) for k, v in st.items() if k != "pod"} for st in self.states])


def _grads(seed, step, misalign=()):
    """New gradient buffers for every spec; the indices in misalign get a view
    one element into a larger buffer (2- or 4-byte aligned only)."""
    out = []
    for i, (dt, n, _) in enumerate(SPECS):
        g = syn.round_to(syn.row_scaled_normal(seed, 100 * step + i, 1, n, -14, -6), dt).reshape(-1)
        if i in misalign:
            buf = gu.to_dev(np.concatenate([g[:1], g]), dt)
            out.append(buf[1:])
        else:
            out.append(gu.to_dev(g, dt))
    return out


def test_step_plan_runs_equal_step_tasks():
    lib = _lib.load()
    tables = _tables(lib)
    a, b = Set(31), Set(31)
    steps = [1] * len(SPECS)
    grads = _grads(31, 1)
    plan = ctypes.c_void_p()
    t0 = a.tasks(grads, steps)  # referenced until the call returns
    _lib.check(lib.gefen_step_plan_create(t0.ctypes.data, len(SPECS), tables.data_ptr(), ctypes.byref(plan)),
               "gefen_step_plan_create")
    try:
        _lib.check(lib.gefen_step_plan_time_runs(plan, 1))
        for step in range(1, 9):
            what = "kept launches"
            if step > 1:
                steps = [s + 1 for s in steps]
            misalign = ()
            if step == 3:
                misalign, what = (0, 1), "misaligned gradients"
            if step == 5:
                steps[-5] += 1
                what = "one period-one task one step ahead (two stepsize tables in one launch)"
            grads = _grads(31, step, misalign) if step != 2 else grads  # step 2: the same buffers again
            ta, tb = a.tasks(grads, steps), b.tasks(grads, steps)
            n = len(SPECS)
            if step == 6:
                # a row names another vmean tensor (both copies): a run that leaves the plan
                for s in (a, b):
                    s.states[2]["vmean"] = s.states[2]["vmean"].clone()
                ta, tb = a.tasks(grads, steps), b.tasks(grads, steps)
                what = "a row with another state tensor"
            if step == 7:
                n, what = n - 3, "a shorter table"
            print("step", step, what, flush=True)
            _lib.check(lib.gefen_step_plan_run(plan, ta.ctypes.data, n, gu.stream()), "gefen_step_plan_run")
            ms = ctypes.c_float()
            _lib.check(lib.gefen_step_plan_last_ms(plan, ctypes.byref(ms)))
            assert ms.value > 0.0
            _lib.check(lib.gefen_step_tasks(tb.ctypes.data, n, tables.data_ptr(), gu.stream()), "gefen_step_tasks")
            torch.cuda.synchronize()
            pa, sa = a.host()
            pb, sb = b.host()
            for i in range(len(SPECS)):
                np.testing.assert_array_equal(pa[i], pb[i], err_msg="step {} ({}) p{}".format(step, what, i))
                for k in ("idx", "mag", "vmean"):
                    np.testing.assert_array_equal(sa[i][k], sb[i][k], err_msg="step {} ({}) {}{}".format(
                        step, what, k, i))
    finally:
        lib.gefen_step_plan_destroy(plan)


def test_step_plan_rejects_invalid_rows_like_step_tasks():
    lib = _lib.load()
    tables = _tables(lib)
    a = Set(32)
    grads = _grads(32, 1)
    t = a.tasks(grads, [1] * len(SPECS))
    plan = ctypes.c_void_p()
    _lib.check(lib.gefen_step_plan_create(t.ctypes.data, len(SPECS), tables.data_ptr(), ctypes.byref(plan)))
    try:
        bad = t.copy()
        bad[4]["bias_correction_2"] = 0.0
        assert lib.gefen_step_plan_run(plan, bad.ctypes.data, len(SPECS), gu.stream()) == _lib.GEFEN_EINVAL
        assert b"bias_correction_2" in lib.gefen_last_error()
        bad = t.copy()
        bad[0]["period"] = 3  # does not divide numel: refused, not launched
        assert lib.gefen_step_plan_run(plan, bad.ctypes.data, len(SPECS), gu.stream()) == _lib.GEFEN_EINVAL
        ms = ctypes.c_float()
        assert lib.gefen_step_plan_last_ms(plan, ctypes.byref(ms)) == _lib.GEFEN_EINVAL  # timing never enabled
    finally:
        lib.gefen_step_plan_destroy(plan)
    bad = t.copy()
    bad[1]["period"] = 7
    plan = ctypes.c_void_p()
    assert lib.gefen_step_plan_create(bad.ctypes.data, len(SPECS), tables.data_ptr(),
                                      ctypes.byref(plan)) == _lib.GEFEN_EINVAL
    assert plan.value is None
    torch.cuda.synchronize()


def test_stream_handle_is_the_current_stream():
    """The optimizer's cached step launches on the raw handle of torch's current
    stream, on the default stream and inside a torch.cuda.stream context."""
    from gefen_amd.gefen import _stream_handle

    assert _stream_handle(0) == torch.cuda.current_stream(0).cuda_stream
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        assert _stream_handle(0) == s.cuda_stream == torch.cuda.current_stream().cuda_stream
    assert _stream_handle(0) == torch.cuda.current_stream(0).cuda_stream


def test_optimizer_step_with_and_without_step_hooks_agree():
    """Gefen.step through the cached plan, with torch's step pre/post hooks
    registered (the hooked entry) and without (the step alone): the same
    parameters and state bit for bit, the hooks called once per step, the plan
    kept in both."""
    from gefen_amd.gefen import Gefen

    def run(hooks):
        g = torch.Generator().manual_seed(3)
        ps = [torch.nn.Parameter((torch.randn(s, generator=g) * 0.02).to(torch.bfloat16).cuda())
              for s in [(64, 256), (512,), (96, 128)]]
        opt = Gefen([("p{}".format(i), p) for i, p in enumerate(ps)])
        calls = []
        if hooks:
            opt.register_step_pre_hook(lambda o, a, k: calls.append("pre"))
            opt.register_step_post_hook(lambda o, a, k: calls.append("post"))
        for step in range(4):
            gg = torch.Generator().manual_seed(10 + step)
            for p in ps:
                p.grad = (torch.randn(p.shape, generator=gg) * 1e-3).to(torch.bfloat16).cuda()
            opt.step()
        torch.cuda.synchronize()
        return ps, opt, calls

    a, oa, ca = run(False)
    b, ob, cb = run(True)
    assert ca == [] and cb == ["pre", "post"] * 4
    assert oa._plan is not None and ob._plan is not None
    assert oa._gefen_global_step == ob._gefen_global_step == 4
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))
        for k in ("m_codebook", "m_magnitude", "vmean"):
            assert torch.equal(oa.state[x][k], ob.state[y][k]), k


@pytest.mark.parametrize("opt_name", ["Gefen", "GefenMuon"])
def test_step_with_closure_returns_its_loss_and_equals_a_manual_backward(opt_name):
    """step(closure) (gefen.py:1399-1420, gefen_muon.py:331-350): the closure runs with
    gradients enabled even when the caller's mode is no_grad, step returns its loss,
    the caller's grad mode is unchanged afterwards, and the parameters equal a run
    that calls backward before a plain step(), bit for bit, over three steps (the
    later ones through the cached plan).  Gefen refreshes its codebook before it runs
    the closure, as the reference does, so its first step needs gradients already
    present (the first step of both runs is a plain one there); GefenMuon runs the
    closure first."""
    from gefen_amd import Gefen, GefenMuon

    cls = {"Gefen": Gefen, "GefenMuon": GefenMuon}[opt_name]

    def make():
        g = torch.Generator().manual_seed(11)
        w = torch.nn.Parameter((torch.randn(128, 256, generator=g) * 0.02).cuda())
        x = torch.randn(16, 256, generator=g).cuda()
        return w, x

    w1, x = make()
    w2, _ = make()
    o1, o2 = cls([("w", w1)]), cls([("w", w2)])
    for step in range(3):
        if step == 0 and opt_name == "Gefen":
            for w, o in ((w1, o1), (w2, o2)):
                o.zero_grad()
                (x @ w.t()).pow(2).mean().backward()
                o.step()
            continue

        def closure():
            assert torch.is_grad_enabled()
            o1.zero_grad()
            loss = (x @ w1.t()).pow(2).mean()
            loss.backward()
            return loss

        with torch.no_grad():
            loss1 = o1.step(closure)
            assert not torch.is_grad_enabled()
        o2.zero_grad()
        loss2 = (x @ w2.t()).pow(2).mean()
        loss2.backward()
        assert o2.step() is None
        torch.cuda.synchronize()
        assert torch.equal(loss1, loss2)
        assert torch.equal(w1.detach(), w2.detach())
    assert o1._gefen_global_step == o2._gefen_global_step == 3

"""CPU-side checks: the C-ABI library loads and exports every declared symbol,
the host logic of the drop-in (period selection, divisors, param groups,
argument validation) follows the reference."""

import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as orc

REPO = Path(__file__).resolve().parent.parent


def _declared(header):
    text = (REPO / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(gefen_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    from gefen_amd import _lib

    lib = _lib.load()
    names = _declared("gefen_hip.h")
    assert len(names) >= 20, names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)
    assert lib.gefen_struct_size(0) == _lib.STEP_TASK.itemsize
    assert lib.gefen_struct_size(1) == _lib.MUON_TASK.itemsize
    assert lib.gefen_struct_size(2) == _lib.MUON_APPLY_TASK.itemsize
    assert lib.gefen_abi_version() == 1


def test_entry_points_reject_invalid_arguments_without_a_device():
    from gefen_amd import _lib

    lib = _lib.load()
    with pytest.raises(ValueError, match="at most 256"):
        _lib.check(lib.gefen_prepare_codebook(1, 300, 1, None))
    with pytest.raises(ValueError, match="bins"):
        _lib.check(lib.gefen_exact_histogram(1, 0, 16, 4, 1, 5000, None))
    with pytest.raises(ValueError, match="divisible"):
        _lib.check(lib.gefen_exact_histogram(1, 0, 17, 4, 1, 4096, None))
    with pytest.raises(ValueError, match="Expected vmean to be float32"):
        _lib.check(lib.gefen_automatic_fused_update_from_vmean(1, 1, 0, 1, 1, 0, 1, 7, 1, 256, 1, 4, 4, 0.9, 1e-3,
                                                               0.5, 0.5, 1e-8, None))
    # a vmean of another dtype than the magnitudes is taken by the given-vmean
    # entry point, not by the period-one update, whose kernels keep both in one dtype
    with pytest.raises(ValueError, match="vmean dtype 1, m_magnitude dtype 0"):
        _lib.check(lib.gefen_automatic_period1_update(1, 1, 0, 1, 1, 0, 1, 1, 1, 256, 16, 4, 0.9, 0.999, 1e-3,
                                                      0.5, 0.5, 1e-8, None))
    with pytest.raises(ValueError, match="beta2"):
        _lib.check(lib.gefen_automatic_vmean_update(1, 0, 1, 0, 4, 4, 1.5, None))
    # the batched Newton-Schulz GEMM addresses a 256-row operand tile with 32-bit
    # byte offsets: rows of 2^22 bf16 elements are refused before any launch
    # (the pointers are never dereferenced: the checks precede every device call)
    long_ld = 1 << 22
    with pytest.raises(ValueError, match="rows too long"):
        _lib.check(lib.gefen_gemm_bf16_nt_batched(256, long_ld, 0, 256, 256, 0, 256, 256, 0, None, 0, 0, None, 0, 0,
                                                  0, 1, 256, 256, 256, 1.0, 0.0, 0, None))
    with pytest.raises(ValueError, match="multiples of 256"):
        _lib.check(lib.gefen_gemm_bf16_nt_batched(256, 320, 0, 256, 320, 0, 256, 320, 0, None, 0, 0, None, 0, 0,
                                                  0, 1, 320, 320, 320, 1.0, 0.0, 0, None))
    assert lib.gefen_exact_dp_workspace_size(4096, 256) > 256 * 4097 * 12
    # the step plan refuses a null result pointer, a negative task count and null
    # tables before touching a device
    import ctypes

    plan = ctypes.c_void_p()
    with pytest.raises(ValueError, match="null plan pointer"):
        _lib.check(lib.gefen_step_plan_create(None, 0, 1, None))
    with pytest.raises(ValueError, match="invalid task array"):
        _lib.check(lib.gefen_step_plan_create(None, -1, 1, ctypes.byref(plan)))
    with pytest.raises(ValueError, match="null codebook tables"):
        _lib.check(lib.gefen_step_plan_create(None, 0, None, ctypes.byref(plan)))
    assert plan.value is None
    with pytest.raises(ValueError, match="null step plan"):
        _lib.check(lib.gefen_step_plan_run(None, None, 0, None))
    with pytest.raises(ValueError, match="null step plan"):
        _lib.check(lib.gefen_step_plan_time_runs(None, 1))
    lib.gefen_step_plan_destroy(None)  # a null plan is ignored
    assert lib.gefen_device_allocations() == 0  # nothing allocated without a device


def test_batched_newton_schulz_shape_predicate_matches_the_byte_limit():
    """A matrix the batched Gram product would refuse (X^T spanning 2^31 bytes or
    more) goes to the one-matrix path: batched_shape_ok says no exactly where
    gefen_gram_bf16_batched raises, so GefenMuon never starts a step it cannot finish."""
    from gefen_amd import _lib
    from gefen_amd.newton_schulz import batched_shape_ok

    lib = _lib.load()
    # 32768 x 32768 bf16 = 2^31 bytes: refused; 32768 x 32512 = 2^31 - 2^24: accepted
    assert not batched_shape_ok(32768, 32768)
    assert batched_shape_ok(32768, 32512) and batched_shape_ok(32512, 32768)
    assert not batched_shape_ok(128256, 16384) and not batched_shape_ok(16384, 128256)
    assert batched_shape_ok(2048, 6144) and not batched_shape_ok(2048, 6000)
    for rows, cols in ((32768, 32768), (131072, 16384), (16384, 131072)):
        m, n = min(rows, cols), max(rows, cols)
        assert not batched_shape_ok(rows, cols)
        with pytest.raises(ValueError, match="operand too large"):
            _lib.check(lib.gefen_gram_bf16_batched(256, m, 0, 256, m, 0, 1, m, n, 1.0, None))


def test_divisors_and_period_selection_match_the_oracle_restatement():
    from gefen_amd import partitioning as part

    for n in [1, 2, 7, 12, 48, 1031 * 3, 2 ** 10 * 3 * 167, 50257 * 768]:
        assert part.divisors(n) == orc.divisors(n)
        assert part.divisors(n, max_divisor=100) == orc.divisors(n, max_divisor=100)
    rng = np.random.default_rng(0)
    for _ in range(200):
        n = int(rng.choice([4096, 6144, 98304, 2304 * 12, 3072 * 40]))
        divs = part.candidate_divisors(n)
        scores = rng.random(len(divs)).tolist()
        pairs = list(zip(divs, scores))
        assert part._finalize_period_results(pairs, False, n, 0.25) == orc.finalize_period(pairs, n)


def test_period_selection_hand_built_cases():
    """partitioning.py:277-347 on score lists whose answer is known by hand."""
    from gefen_amd.partitioning import _finalize_period_results as fin

    n = 96 * 768
    divs = [p for p in orc.divisors(n) if n // p >= 4]
    flat = [(p, 1.0) for p in divs]
    assert fin(flat, False, n, 0.25) == 1                      # no strict local maximum
    peak = [(p, 2.0 if p == 768 else 1.0) for p in divs]
    assert fin(peak, False, n, 0.25) == 768
    small = [(p, 2.0 if p == 8 else 1.0) for p in divs]
    assert fin(small, False, n, 0.25) == 1                     # p <= 8 never wins
    two = [(p, 3.0 if p == 768 else 2.0 if p == 96 else 1.0) for p in divs]
    assert fin(two, False, n, 0.25) == 768                     # highest score wins
    # caps: best 2304 -> 1152, 3072 -> 1536, 4096 -> 2048
    for n, best, capped in [(2304 * 12, 2304, 1152), (3072 * 40, 3072, 1536), (4096 * 8, 4096, 2048)]:
        d = [p for p in orc.divisors(n) if n // p >= 4]
        s = [(p, 5.0 if p == best else 1.0) for p in d]
        assert fin(s, False, n, 0.25) == capped
    last = [(p, 2.0 if p == divs[-1] else 1.0) for p in divs]
    assert fin(last, False, 96 * 768, 0.25) == 1               # the last divisor is excluded


def test_param_group_flattening_matches_reference():
    from gefen_amd.gefen import Gefen

    a = torch.zeros(4, 3, requires_grad=True)
    b = torch.zeros(5, requires_grad=True)
    c = torch.zeros(2, requires_grad=False)
    d = torch.zeros(6, requires_grad=True)
    opt = Gefen([{"params": [("Alpha", a), b, c], "lr": 2e-3, "betas": (0.8, 0.95)}, ("Beta", d)], weight_decay=0.1)
    names = [g["name"] for g in opt.param_groups]
    assert names == ["alpha", "group_0_param_1", "beta"]
    g0 = opt.param_groups[0]
    assert (g0["lr"], g0["beta1"], g0["beta2"], g0["eps"], g0["weight_decay"]) == (2e-3, 0.8, 0.95, 1e-8, 0.1)
    assert set(g0.keys()) == {"name", "params", "lr", "beta1", "beta2", "eps", "weight_decay"}
    with pytest.raises(ValueError, match="Invalid beta parameter at index 0"):
        Gefen([a], betas=(1.0, 0.9))
    with pytest.raises(ValueError, match="missing the 'params' key"):
        Gefen([{"lr": 1.0}])
    with pytest.raises(TypeError, match="can only optimize Tensors"):
        Gefen([{"params": [1.0]}])


def test_muon_constructor_checks():
    from gefen_amd.gefen_muon import GefenMuon

    w = torch.zeros(4, 4, requires_grad=True)
    opt = GefenMuon([w])
    g = opt.param_groups[0]
    assert g["beta1"] == 0.95 and g["beta2"] == 0.0 and g["eps"] == 1e-7 and g["weight_decay"] == 0.1
    assert g["nesterov"] is True and g["ns_steps"] == 5
    with pytest.raises(ValueError, match="only supports 2D"):
        GefenMuon([torch.zeros(3, requires_grad=True)])
    with pytest.raises(ValueError, match="not supported"):
        GefenMuon([w], adjust_lr_fn="bogus")


def test_step_on_cpu_tensors_fails_loudly():
    from gefen_amd.gefen import Gefen

    w = torch.zeros(8, 8, requires_grad=True)
    w.grad = torch.ones(8, 8)
    opt = Gefen([w])
    with pytest.raises((RuntimeError, ValueError), match="HIP"):
        opt.step()


def test_plan_core_checks_and_commits_only_when_the_plan_applies():
    """PlanCore.refresh (gefen_amd/csrc/host_plan.cpp) on CPU tensors: it fills each
    task row (gradient address, group hyperparameters, bias corrections 1 - beta **
    step as Python computes them) and advances the steps only when every parameter
    with a gradient is the recorded one with a gradient of the recorded layout and
    the state tensors are unchanged; any mismatch leaves table and steps alone."""
    import numpy as np
    import torch

    from gefen_amd import _gefen_host, _lib

    ps = [torch.nn.Parameter(torch.zeros(n)) for n in (8, 16, 4)]
    for p in ps:
        p.grad = torch.ones_like(p)
    states = [{"step": 3, "m_codebook": torch.zeros(1), "m_magnitude": torch.zeros(1), "vmean": torch.zeros(1)}
              for _ in ps]
    core = _gefen_host.PlanCore(list(ps), states, ("m_codebook", "m_magnitude", "vmean"))
    assert len(core) == 3
    groups = [{"params": [ps[0], ps[1]], "lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 0},
              {"params": [ps[2]], "lr": torch.tensor(2e-3, dtype=torch.float64), "beta1": 0.8, "beta2": 0.99,
               "eps": 1e-6, "weight_decay": 0.1}]
    table = np.zeros(3, dtype=_lib.STEP_TASK)
    steps = np.zeros(3, dtype=np.int64)
    cols = tuple(table.dtype.fields[c][1] for c in ("grad", "lr", "beta1", "beta2", "eps", "weight_decay",
                                                     "bias_correction_1", "bias_correction_2"))

    def refresh(gr):
        return core.refresh(gr, table.ctypes.data, table.itemsize, cols, steps.ctypes.data)

    assert refresh(groups)
    assert table["grad"].tolist() == [p.grad.data_ptr() for p in ps]
    assert steps.tolist() == [4, 4, 4] and [st["step"] for st in states] == [4, 4, 4]
    assert table["lr"].tolist() == [1e-3, 1e-3, 2e-3] and table["weight_decay"].tolist() == [0.0, 0.0, 0.1]
    assert table["beta1"].tolist() == [0.9, 0.9, 0.8] and table["eps"].tolist() == [1e-8, 1e-8, 1e-6]
    assert table["bias_correction_1"].tolist() == [1 - 0.9 ** 4, 1 - 0.9 ** 4, 1 - 0.8 ** 4]
    assert table["bias_correction_2"].tolist() == [1 - 0.999 ** 4, 1 - 0.999 ** 4, 1 - 0.99 ** 4]

    def unchanged_after(mutate, undo):
        table["grad"] = 0
        table["lr"] = 0.0
        mutate()
        before = [st["step"] for st in states]
        assert not refresh(groups)
        assert table["grad"].tolist() == [0, 0, 0] and table["lr"].tolist() == [0.0, 0.0, 0.0]
        assert [st["step"] for st in states] == before
        undo()
        assert refresh(groups)

    g1 = ps[1].grad
    unchanged_after(lambda: g1.resize_(12), lambda: g1.resize_(16))  # resized in place
    unchanged_after(lambda: setattr(ps[1], "grad", torch.ones(32)[::2]), lambda: setattr(ps[1], "grad", g1))
    unchanged_after(lambda: setattr(ps[1], "grad", None), lambda: setattr(ps[1], "grad", g1))
    unchanged_after(lambda: groups[0]["params"].reverse(), lambda: groups[0]["params"].reverse())
    extra = torch.nn.Parameter(torch.zeros(2))
    extra.grad = torch.ones(2)
    unchanged_after(lambda: groups[1]["params"].append(extra), lambda: groups[1]["params"].pop())
    vm = states[2]["vmean"]
    unchanged_after(lambda: states[2].__setitem__("vmean", vm.clone()), lambda: states[2].__setitem__("vmean", vm))
    unchanged_after(lambda: states[0].__setitem__("step", torch.tensor(5)), lambda: states[0].__setitem__("step", 9))
    unchanged_after(lambda: groups[1].__setitem__("lr", "fast"), lambda: groups[1].__setitem__("lr", 2e-3))
    # a bf16 lr tensor with weight decay: torch forms that decay factor in bf16 (no plan)
    unchanged_after(lambda: groups[1].__setitem__("lr", torch.tensor(2e-3, dtype=torch.bfloat16)),
                    lambda: groups[1].__setitem__("lr", 2e-3))
    assert [st["step"] for st in states] == [12, 13, 13] and steps.tolist() == [12, 13, 13]
    assert table["bias_correction_1"].tolist() == [1 - 0.9 ** 12, 1 - 0.9 ** 13, 1 - 0.8 ** 13]
    # values changed without a new dict entry are still seen: a 0-d lr tensor changed
    # in place, a state "step" written by the user, a state tensor replaced
    lr64 = torch.tensor(2e-3, dtype=torch.float64)
    groups[1]["lr"] = lr64
    assert refresh(groups) and table["lr"][2] == 2e-3
    lr64.fill_(3e-3)
    assert refresh(groups) and table["lr"][2] == 3e-3
    groups[1]["lr"] = 2e-3
    s0 = states[0]["step"]
    assert refresh(groups) and refresh(groups) and states[0]["step"] == s0 + 2
    states[0]["step"] = 100
    assert refresh(groups) and states[0]["step"] == 101 and steps[0] == 101
    states[0]["step"] = s0 + 3
    vm0 = states[0]["vmean"]
    states[0]["vmean"] = vm0.clone()
    assert not refresh(groups)
    states[0]["vmean"] = vm0
    assert refresh(groups) and states[0]["step"] == s0 + 4
    states[0]["step"], states[1]["step"], states[2]["step"] = 12, 13, 13
    assert refresh(groups)
    for st in states:
        st["step"] -= 1
    # a float32 lr tensor with weight decay keeps the plan: the row carries the
    # weight decay for which the kernels' double factor is torch's float32 one
    from gefen_amd.gefen import _kernel_weight_decay

    lr32 = torch.tensor(2e-3, dtype=torch.float32)
    groups[1]["lr"] = lr32
    assert refresh(groups)
    assert table["lr"][2] == float(lr32.item())
    assert table["weight_decay"][2] == _kernel_weight_decay(lr32, 0.1) != 0.1
    assert np.float32(1.0 - table["lr"][2] * table["weight_decay"][2]) == (1 - lr32 * 0.1).item()


def test_plan_core_step_runs_between_the_table_rows_and_the_step_counts():
    """PlanCore.step (gefen_amd/csrc/host_plan.cpp) calls the run function once,
    with (plan, table, rows, stream), after the table rows are written and before
    the state dicts' "step" entries and steps_out advance; it returns the run's
    status and advances the counts whatever that status; when a check fails it
    returns -1 without calling the run or changing table or counts."""
    import ctypes

    import numpy as np
    import torch

    from gefen_amd import _gefen_host, _lib

    ps = [torch.nn.Parameter(torch.zeros(n)) for n in (8, 4)]
    for p in ps:
        p.grad = torch.ones_like(p)
    states = [{"step": 5, "m_codebook": torch.zeros(1), "m_magnitude": torch.zeros(1), "vmean": torch.zeros(1)}
              for _ in ps]
    core = _gefen_host.PlanCore(list(ps), states, ("m_codebook", "m_magnitude", "vmean"))
    groups = [{"params": list(ps), "lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 0}]
    table = np.zeros(2, dtype=_lib.STEP_TASK)
    steps = np.zeros(2, dtype=np.int64)
    cols = tuple(table.dtype.fields[c][1] for c in ("grad", "lr", "beta1", "beta2", "eps", "weight_decay",
                                                     "bias_correction_1", "bias_correction_2"))
    seen = []
    status = [0]

    @ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p)
    def run(plan, tasks, n, stream):
        seen.append((plan, tasks, n, stream, table["grad"].tolist(), table["bias_correction_1"].tolist(),
                     [st["step"] for st in states], steps.tolist()))
        return status[0]

    run_fn = ctypes.cast(run, ctypes.c_void_p).value

    def step(gr):
        return core.step(gr, table.ctypes.data, table.itemsize, cols, steps.ctypes.data, run_fn, 0x1234, 0x5678)

    assert step(groups) == 0
    grads = [p.grad.data_ptr() for p in ps]
    assert seen == [(0x1234, table.ctypes.data, 2, 0x5678, grads, [1 - 0.9 ** 6] * 2, [5, 5], [0, 0])]
    assert [st["step"] for st in states] == [6, 6] and steps.tolist() == [6, 6]
    # a failed run still advances the counts (its launches may have started)
    status[0] = 7
    assert step(groups) == 7
    assert seen[-1][6] == [6, 6] and [st["step"] for st in states] == [7, 7] and steps.tolist() == [7, 7]
    # a failed check: no run, nothing written
    g1 = ps[1].grad
    ps[1].grad = torch.ones(8)[::2]  # not contiguous
    table["grad"] = 0
    assert step(groups) == -1
    assert len(seen) == 2 and table["grad"].tolist() == [0, 0]
    assert [st["step"] for st in states] == [7, 7] and steps.tolist() == [7, 7]
    ps[1].grad = g1
    status[0] = 0
    assert step(groups) == 0 and seen[-1][6] == [7, 7] and [st["step"] for st in states] == [8, 8]
    with pytest.raises(ValueError):
        core.step(groups, table.ctypes.data, table.itemsize, cols, steps.ctypes.data, 0, 0x1234, 0x5678)


def test_kernel_weight_decay_reproduces_torch_float32_factor():
    """_kernel_weight_decay: for a float32 tensor lr, the kernels' double expression
    (float)(1 - lr * wd') equals torch's float32 factor 1 - lr * wd for every
    sampled pair (including ones where the double expression with wd itself does
    not), and decays exactly when that factor is below one; a 16-bit lr, a zero
    factor or lr <= 0 are left to torch (None)."""
    import numpy as np
    import torch

    from gefen_amd.gefen import _kernel_weight_decay

    rng = np.random.default_rng(17)
    lrs = np.concatenate([10.0 ** rng.uniform(-8, 0.5, 20000), [1e-3, 0.5, 1.0, 2.0, 3e-45, 1e-30]])
    wds = np.concatenate([10.0 ** rng.uniform(-6, 1, 20000), [0.1, 2.0, 1.0, 0.5, 1e-3, 1e-9]])
    differs = 0
    for lr_v, wd in zip(lrs, wds):
        lr = torch.tensor(float(lr_v), dtype=torch.float32)
        torch_f = (1 - lr * float(wd)).item()
        w = _kernel_weight_decay(lr, float(wd))
        if torch_f == 0.0 or not lr.item() > 0.0:
            assert w is None
            continue
        kernel_f = np.float32(1.0 - float(lr.item()) * w)
        assert kernel_f == np.float32(torch_f), (lr_v, wd)
        assert (w > 0.0) == (torch_f < 1.0)
        differs += np.float32(1.0 - float(lr.item()) * float(wd)) != np.float32(torch_f)
    assert differs > 100
    assert _kernel_weight_decay(torch.tensor(1e-3, dtype=torch.bfloat16), 0.1) is None
    assert _kernel_weight_decay(torch.tensor(0.5, dtype=torch.float32), 2.0) is None  # factor 0
    assert _kernel_weight_decay(torch.tensor(1e-3, dtype=torch.float64), 0.1) == 0.1
    assert _kernel_weight_decay(1e-3, 0.1) == 0.1 and _kernel_weight_decay(torch.tensor(1e-3), 0.0) == 0.0


def _entry_optimizers():
    """An optimizer whose step goes through gefen.py's _step_entry and one that
    torch wraps itself (profile_hook_step), both logging their calls."""
    from gefen_amd.gefen import _step_entry

    def body(self, closure=None):
        self.log.append(("step", closure))
        return "loss"

    class Entry(torch.optim.Optimizer):
        def __init__(self, params):
            super().__init__(params, {})
            self.log = []

        step = _step_entry(body)

    class Torch(torch.optim.Optimizer):
        def __init__(self, params):
            super().__init__(params, {})
            self.log = []

        def step(self, closure=None):
            return body(self, closure)

    return Entry([torch.nn.Parameter(torch.zeros(2))]), Torch([torch.nn.Parameter(torch.zeros(2))])


def test_step_entry_calls_hooks_and_profiler_range_as_torch_does():
    """The Gefen optimizers' step entry (gefen.py: _step_entry) keeps
    torch.optim.Optimizer's step contract: instance and global pre/post hooks in
    torch's order, a pre-hook may replace the arguments, and a profiler sees the
    'Optimizer.step#<class>.step' range; with no hook and no profiler the step
    runs alone (torch's wrapper, which also calls _optimizer_step_code, is not
    entered)."""
    from torch.optim import optimizer as optim

    entry, ref = _entry_optimizers()
    assert type(entry).step.hooked
    for opt in (entry, ref):
        opt.code_calls = 0

        def code(opt=opt):
            opt.code_calls += 1

        opt._optimizer_step_code = code
    assert entry.step() == "loss" and entry.code_calls == 0
    assert ref.step() == "loss" and ref.code_calls == 1
    logs = []
    for opt in (entry, ref):
        log = []
        hs = [opt.register_step_pre_hook(lambda o, a, k, log=log: log.append("pre")),
              opt.register_step_post_hook(lambda o, a, k, log=log: log.append("post")),
              opt.register_step_pre_hook(lambda o, a, k: ((a[0], "replaced"), {})),
              optim.register_optimizer_step_pre_hook(lambda o, a, k, log=log: log.append("global pre")),
              optim.register_optimizer_step_post_hook(lambda o, a, k, log=log: log.append("global post"))]
        try:
            assert opt.step() == "loss"
        finally:
            for h in hs:
                h.remove()
        logs.append((log, opt.log[-1]))
    assert logs[0] == logs[1] == (["global pre", "pre", "post", "global post"], ("step", "replaced"))
    assert entry.code_calls == 1
    assert entry.step() == "loss" and entry.code_calls == 1  # hooks removed: the step alone again
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
        entry.step()
    assert "Optimizer.step#Entry.step" in [e.name for e in prof.events()]
    assert entry.code_calls == 2

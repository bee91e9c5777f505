"""Randomised parity of the batched step with the CPU oracle: one
gefen_step_tasks call per step over 130 tensors of random dtype pairs, periods
(period one with its largest divisor <= 256, short and long rows, odd sizes),
hyperparameters (beta1, beta2, lr, eps and weight decay per tensor, so one
launch carries many stepsize settings) and gradient scales, with zero blocks;
then the same steps through a kept step plan (gefen_step_plan_run), which must
equal gefen_step_tasks bit for bit.

Against the oracle (the reference's CPU path, oracle/gefen_oracle.c): indices
and magnitudes bit-exact; period-one vmean and parameters bit-exact; block
vmean of 16-bit state within one ulp, of float32 state within 2^-18 relative
(its float32 sum runs in another order than torch's); float32 parameters within
rtol 1e-5 / atol 1e-7; 16-bit parameters within one ulp, except in rows whose
vmean has rounded the other way at some step, where they stay within 2^-7 of
the summed update plus one ulp per step.  (A half state can underflow to zero
at small gradients and eps = 1e-10, and its parameters then overflow to inf, as
on the reference's path; they are compared like the others.)"""

import numpy as np
import pytest
import torch

import gpu_util as gu
from golden_util import load
from gefen_amd import _lib
from gefen_amd import synthetic as syn
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

STEPS = 4
PAIRS = [("bf16", "bf16")] * 4 + [("f16", "f16"), ("f32", "f32"), ("f32", "f32"), ("bf16", "f32"), ("f16", "f32")]
PERIODS = [2, 3, 5, 7, 8, 9, 12, 16, 24, 31, 48, 64, 96, 100, 128, 192, 256, 384, 500, 512, 768, 1000, 1024,
           1536, 2048, 3072, 4096, 5000]


def _codebook():
    data, _ = load("exact_dp")
    return np.ascontiguousarray(data["hist_k256_forced/codebook"], dtype=np.float32)


def _specs(rng, count):
    specs = []
    for i in range(count):
        dt, sdt = PAIRS[rng.integers(len(PAIRS))]
        if rng.random() < 0.3:
            period = 1
            n = int(rng.integers(1, 20000))
            pod = orc.largest_divisor_at_most(n, 256)
        else:
            period = int(PERIODS[rng.integers(len(PERIODS))])
            n = period * int(rng.integers(1, max(2, 40000 // period)))
            pod = 0
        e_lo = int(rng.integers(-20, -7))
        specs.append({
            "dt": dt, "sdt": sdt, "n": n, "period": period, "pod": pod,
            "b1": float(rng.uniform(0.8, 0.95)), "b2": float(rng.uniform(0.95, 0.9999)),
            "lr": float(10.0 ** rng.uniform(-4, -2.5)), "eps": float([1e-8, 1e-6, 1e-10][rng.integers(3)]),
            "wd": 0.0 if rng.random() < 0.5 else float(rng.uniform(0.01, 0.2)),
            "e_lo": e_lo, "e_hi": e_lo + int(rng.integers(2, 11)), "zero_block": bool(rng.random() < 0.15),
        })
    return specs


def _host(x):
    return x.view(np.uint16) if x.dtype == np.float16 else x


def _task_rows(specs, dev):
    tasks = np.zeros(len(specs), dtype=_lib.STEP_TASK)
    for t, s, d in zip(tasks, specs, dev):
        t["p"], t["grad"], t["m_codebook"] = d["p"].data_ptr(), d["g"].data_ptr(), d["idx"].data_ptr()
        t["m_magnitude"], t["vmean"] = d["mag"].data_ptr(), d["v"].data_ptr()
        t["numel"], t["period"], t["period_one_divisor"] = s["n"], s["period"], s["pod"]
        t["param_dtype"], t["state_dtype"] = gu.CODE[s["dt"]], gu.CODE[s["sdt"]]
        t["beta1"], t["beta2"], t["lr"], t["eps"], t["weight_decay"] = s["b1"], s["b2"], s["lr"], s["eps"], s["wd"]
    return tasks


def _set_step(tasks, specs, step):
    for t, s in zip(tasks, specs):
        t["bias_correction_1"] = 1 - s["b1"] ** step
        t["bias_correction_2"] = 1 - s["b2"] ** step


@pytest.mark.parametrize("seed", [20261202, 7, 1234567])
def test_random_batched_steps_match_oracle_and_plan(seed):
    import ctypes

    rng = np.random.default_rng(seed)
    specs = _specs(rng, 130)
    print("seed", seed, "tasks", len(specs), "elements", sum(s["n"] for s in specs), flush=True)
    cb = _codebook()
    cb_dev = torch.from_numpy(cb).to("cuda:0")
    lib = _lib.load()
    tables = torch.empty(int(lib.gefen_codebook_tables_size()), dtype=torch.uint8, device="cuda:0")
    _lib.check(lib.gefen_prepare_codebook(cb_dev.data_ptr(), cb.size, tables.data_ptr(), gu.stream()))

    ref, dev, plan_dev = [], [], []
    for i, s in enumerate(specs):
        n, period, pod, dt, sdt = s["n"], s["period"], s["pod"], s["dt"], s["sdt"]
        rows_m = n // (pod if period == 1 else period)
        rows_v = n // period
        p = _host(syn.round_to(syn.normal(syn.make_key(seed, i), n) * 0.02, dt))
        r = {"p": p.copy(), "idx": np.zeros(n, np.uint8), "mag": np.zeros(rows_m, orc.NP_STORAGE[sdt]),
             "v": np.zeros(rows_v, orc.NP_STORAGE[sdt]), "moved": np.zeros(n), "flag": np.zeros(rows_v, bool)}
        ref.append(r)
        for out in (dev, plan_dev):
            out.append({"p": gu.to_dev(p, dt), "g": torch.empty(n, dtype=gu.TORCH[dt], device="cuda:0"),
                        "idx": torch.zeros(n, dtype=torch.uint8, device="cuda:0"),
                        "mag": torch.zeros(rows_m, dtype=gu.TORCH[sdt], device="cuda:0"),
                        "v": torch.zeros(rows_v, dtype=gu.TORCH[sdt], device="cuda:0")})
    tasks = _task_rows(specs, dev)
    ptasks = _task_rows(specs, plan_dev)
    _set_step(ptasks, specs, 1)
    plan = ctypes.c_void_p()
    _lib.check(lib.gefen_step_plan_create(ptasks.ctypes.data, len(ptasks), tables.data_ptr(), ctypes.byref(plan)))
    try:
        for step in range(1, STEPS + 1):
            grads = []
            for i, s in enumerate(specs):
                blk = s["pod"] if s["period"] == 1 else s["period"]
                g = syn.round_to(syn.row_scaled_normal(seed + 1 + i, step, s["n"] // blk, blk, s["e_lo"], s["e_hi"]),
                                 s["dt"]).reshape(-1).copy()
                if s["zero_block"] and step == 1:
                    g[:blk] = 0
                g = _host(g)
                grads.append(g)
                gd = gu.to_dev(g, s["dt"])
                dev[i]["g"].copy_(gd)
                plan_dev[i]["g"].copy_(gd)
            _set_step(tasks, specs, step)
            _set_step(ptasks, specs, step)
            _lib.check(lib.gefen_step_tasks(tasks.ctypes.data, len(tasks), tables.data_ptr(), gu.stream()))
            _lib.check(lib.gefen_step_plan_run(plan, ptasks.ctypes.data, len(ptasks), gu.stream()))
            for i, s in enumerate(specs):
                r, g = ref[i], grads[i]
                before = r["p"].copy()
                rc = orc.lib().orc_gefen_step(gu.CODE[s["dt"]], gu.CODE[s["sdt"]], orc._ptr(r["p"]), orc._ptr(g),
                                              orc._ptr(r["idx"]), orc._ptr(r["mag"]), orc._ptr(r["v"]), s["n"],
                                              s["period"], s["pod"], orc._ptr(cb), cb.size, s["b1"], s["b2"], s["lr"],
                                              s["eps"], s["wd"], 1 - s["b1"] ** step, 1 - s["b2"] ** step, 1)
                assert rc == 0
                with np.errstate(invalid="ignore"):  # parameters that overflowed to inf
                    r["moved"] += np.abs(orc.to_f32(r["p"], s["dt"]).astype(np.float64) -
                                         orc.to_f32(before, s["dt"]).astype(np.float64))
            torch.cuda.synchronize()
            beyond = 0
            for i, s in enumerate(specs):
                r, d, pd = ref[i], dev[i], plan_dev[i]
                dt, sdt, period = s["dt"], s["sdt"], s["period"]
                tag = "task {} {}/{} n={} P={} step {}".format(i, dt, sdt, s["n"], period, step)
                for k in ("p", "idx", "mag", "v"):
                    assert torch.equal(d[k].view(torch.uint8), pd[k].view(torch.uint8)), tag + " plan " + k
                np.testing.assert_array_equal(gu.to_np(d["idx"]), r["idx"], err_msg=tag + " idx")
                np.testing.assert_array_equal(gu.to_np(d["mag"]), r["mag"], err_msg=tag + " mag")
                gv, gp = gu.to_np(d["v"]), gu.to_np(d["p"])
                if period == 1:
                    np.testing.assert_array_equal(gv, r["v"], err_msg=tag + " vmean")
                    np.testing.assert_array_equal(gp, r["p"], err_msg=tag + " params")
                    continue
                if sdt == "f32":
                    np.testing.assert_allclose(gv, r["v"], rtol=2.0 ** -18, atol=0, err_msg=tag + " vmean")
                else:
                    dv = gu.ulps16(gv, r["v"])
                    assert dv.max() <= 1, tag + " vmean"
                    r["flag"] |= dv == 1
                if dt == "f32":
                    np.testing.assert_allclose(gp, r["p"], rtol=1e-5, atol=1e-7, err_msg=tag + " params")
                    continue
                dp = gu.ulps16(gp, r["p"])
                far = np.nonzero(dp > 1)[0]
                if far.size:
                    assert np.all(r["flag"][far // period]), (tag, far[:8])
                    diff = np.abs(orc.to_f32(gp[far], dt).astype(np.float64) -
                                  orc.to_f32(r["p"][far], dt).astype(np.float64))
                    assert np.all(diff <= 2.0 ** -7 * r["moved"][far] + step * gu.ulp_at16(r["p"][far], dt)), (tag, far[:8])
                    beyond += far.size
            print("step", step, "all", len(specs), "tasks match the oracle;", beyond,
                  "16-bit parameters beyond one ulp (vmean rounding)", flush=True)
    finally:
        lib.gefen_step_plan_destroy(plan)


@pytest.mark.parametrize("seed", [11, 2026])
def test_random_muon_momentum_tasks_match_oracle(seed):
    """GefenMuon's quantised momentum (gefen_muon_tasks) over 100 tensors of random
    dtype pairs, block lengths, momentum and Nesterov settings in one call per
    step: indices, magnitudes and the Nesterov / momentum output bit-exact
    against the oracle (gefen_muon.py:216-260 on the CPU path) over 4 steps."""
    rng = np.random.default_rng(seed)
    cb = _codebook()
    lib = _lib.load()
    tables = torch.empty(int(lib.gefen_codebook_tables_size()), dtype=torch.uint8, device="cuda:0")
    cb_dev = torch.from_numpy(cb).to("cuda:0")
    _lib.check(lib.gefen_prepare_codebook(cb_dev.data_ptr(), cb.size, tables.data_ptr(), gu.stream()))
    specs, ref, dev = [], [], []
    for i in range(100):
        dt, sdt = PAIRS[rng.integers(len(PAIRS))]
        block = int(PERIODS[rng.integers(len(PERIODS))]) if rng.random() < 0.8 else int(rng.integers(1, 257))
        n = block * int(rng.integers(1, max(2, 30000 // block)))
        e_lo = int(rng.integers(-20, -7))
        specs.append({"dt": dt, "sdt": sdt, "n": n, "block": block, "mom": float(rng.uniform(0.8, 0.99)),
                      "nest": int(rng.integers(2)), "e_lo": e_lo, "e_hi": e_lo + int(rng.integers(2, 11))})
        ref.append({"idx": np.zeros(n, np.uint8), "mag": np.zeros(n // block, orc.NP_STORAGE[sdt])})
        dev.append({"g": torch.empty(n, dtype=gu.TORCH[dt], device="cuda:0"),
                    "idx": torch.zeros(n, dtype=torch.uint8, device="cuda:0"),
                    "mag": torch.zeros(n // block, dtype=gu.TORCH[sdt], device="cuda:0"),
                    "out": torch.empty(n, dtype=gu.TORCH[dt], device="cuda:0")})
    print("seed", seed, "muon tasks", len(specs), "elements", sum(s["n"] for s in specs), flush=True)
    tasks = np.zeros(len(specs), dtype=_lib.MUON_TASK)
    for t, s, d in zip(tasks, specs, dev):
        t["grad"], t["m_codebook"], t["m_magnitude"] = d["g"].data_ptr(), d["idx"].data_ptr(), d["mag"].data_ptr()
        t["out"], t["numel"], t["block"] = d["out"].data_ptr(), s["n"], s["block"]
        t["grad_dtype"], t["state_dtype"] = gu.CODE[s["dt"]], gu.CODE[s["sdt"]]
        t["momentum"], t["nesterov"] = s["mom"], s["nest"]
    for step in range(1, STEPS + 1):
        grads = []
        for i, s in enumerate(specs):
            g = _host(syn.round_to(syn.row_scaled_normal(seed * 1000 + i, step, s["n"] // s["block"], s["block"],
                                                         s["e_lo"], s["e_hi"]), s["dt"]).reshape(-1).copy())
            grads.append(g)
            dev[i]["g"].copy_(gu.to_dev(g, s["dt"]))
        _lib.check(lib.gefen_muon_tasks(tasks.ctypes.data, len(tasks), tables.data_ptr(), gu.stream()))
        torch.cuda.synchronize()
        for i, s in enumerate(specs):
            r, d = ref[i], dev[i]
            out = np.empty(s["n"], dtype=orc.NP_STORAGE[s["dt"]])
            assert orc.lib().orc_muon_momentum(gu.CODE[s["dt"]], gu.CODE[s["sdt"]], orc._ptr(grads[i]),
                                               orc._ptr(r["idx"]), orc._ptr(r["mag"]), orc._ptr(out), s["n"],
                                               s["block"], orc._ptr(cb), cb.size, s["mom"], s["nest"]) == 0
            tag = "muon task {} {}/{} n={} block={} step {}".format(i, s["dt"], s["sdt"], s["n"], s["block"], step)
            np.testing.assert_array_equal(gu.to_np(d["idx"]), r["idx"], err_msg=tag + " idx")
            np.testing.assert_array_equal(gu.to_np(d["mag"]), r["mag"], err_msg=tag + " mag")
            np.testing.assert_array_equal(gu.to_np(d["out"]), out, err_msg=tag + " out")
        print("step", step, "all", len(specs), "momentum tasks match the oracle", flush=True)


@pytest.mark.parametrize("seed", [5, 77])
def test_random_muon_apply_tasks_match_oracle(seed):
    """GefenMuon's parameter update (gefen_muon_apply_tasks) over 60 parameters of
    random dtypes, shapes (tall ones take the transposed-update rounding), lr,
    weight decay and adjusted lr in one call: bit-exact against oracle.muon_apply
    (gefen_muon.py:325-329 on the CPU path)."""
    rng = np.random.default_rng(seed)
    lib = _lib.load()
    specs, dev, ref = [], [], []
    for i in range(60):
        dt = ["bf16", "bf16", "f16", "f32"][rng.integers(4)]
        rows, cols = int(rng.integers(1, 300)), int(rng.integers(1, 300))
        lr = float(10.0 ** rng.uniform(-4, -1.5))
        wd = 0.0 if rng.random() < 0.4 else float(rng.uniform(0.01, 0.3))
        adj = lr * float(rng.uniform(0.2, 3.0))
        p = _host(syn.round_to(syn.normal(syn.make_key(seed, i), rows * cols) * 0.05, dt))
        u = syn.round_to(syn.normal(syn.make_key(seed + 1, i), rows * cols), "bf16")
        specs.append({"dt": dt, "shape": (rows, cols), "lr": lr, "wd": wd, "adj": adj, "u": u})
        ref.append(p.copy())
        dev.append({"p": gu.to_dev(p, dt), "u": gu.to_dev(u, "bf16")})
    tasks = np.zeros(len(specs), dtype=_lib.MUON_APPLY_TASK)
    for t, s, d in zip(tasks, specs, dev):
        t["p"], t["update"], t["numel"] = d["p"].data_ptr(), d["u"].data_ptr(), s["shape"][0] * s["shape"][1]
        t["param_dtype"], t["transposed"] = gu.CODE[s["dt"]], 1 if s["shape"][0] > s["shape"][1] else 0
        t["lr"], t["weight_decay"], t["adjusted_lr"] = s["lr"], s["wd"], s["adj"]
    _lib.check(lib.gefen_muon_apply_tasks(tasks.ctypes.data, len(tasks), gu.stream()))
    torch.cuda.synchronize()
    for i, s in enumerate(specs):
        orc.muon_apply(ref[i], s["u"], s["dt"], s["shape"], s["lr"], s["wd"], s["adj"])
        np.testing.assert_array_equal(gu.to_np(dev[i]["p"]), ref[i],
                                      err_msg="apply task {} {} {}".format(i, s["dt"], s["shape"]))
    print("seed", seed, "all", len(specs), "parameter updates match the oracle", flush=True)

"""Parity of the fused HIP step kernels with the CPU oracle (the reference's CPU path).

Codebook indices and magnitudes must be bit-exact.  vmean of period-one tensors
is an element-wise formula and must be bit-exact too; the block mean of
period > 1 tensors is summed in another order than torch's, so vmean agrees to
a few fp32 ulps and the parameters to rtol 1e-5 / atol 1e-7 (fp32) or 1 ulp
(bf16 / f16).
"""

import ctypes

import numpy as np
import pytest
import torch

import gpu_util as gu
from golden_util import load
from gefen_amd import _lib
from gefen_amd import synthetic as syn
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _codebook():
    data, _ = load("exact_dp")
    return np.ascontiguousarray(data["hist_k256_forced/codebook"], dtype=np.float32)


def _tables(cb_dev):
    lib = _lib.load()
    t = torch.empty(int(lib.gefen_codebook_tables_size()), dtype=torch.uint8, device="cuda:0")
    _lib.check(lib.gefen_prepare_codebook(cb_dev.data_ptr(), cb_dev.numel(), t.data_ptr(), gu.stream()))
    return t


def _ulps(a, b):
    a = a.astype(np.int32)
    b = b.astype(np.int32)
    ka = np.where(a & 0x8000, 0x8000 - (a & 0x7FFF), 0x8000 + (a & 0x7FFF))
    kb = np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + (b & 0x7FFF))
    return np.abs(ka - kb)


# (name, dtype, state dtype, numel, period, weight decay); periods chosen to hit every
# kernel shape: vector widths 8/4/1, 1-8 vectors per lane, lane groups of 4..64, the
# two-sweep path for long rows, period one, and an fp32 state for bf16 parameters.
CASES = [
    ("bf16_P2048", "bf16", "bf16", 2048 * 24, 2048, 0.0),
    ("bf16_P768_wd", "bf16", "bf16", 768 * 40, 768, 0.1),
    ("bf16_P64", "bf16", "bf16", 64 * 300, 64, 0.0),
    ("bf16_P12", "bf16", "bf16", 12 * 500, 12, 0.0),
    ("bf16_P9", "bf16", "bf16", 9 * 700, 9, 0.0),
    ("bf16_P5000_long", "bf16", "bf16", 5000 * 6, 5000, 0.0),
    ("bf16_P1", "bf16", "bf16", 256 * 50, 1, 0.0),
    ("bf16_P1_pod250", "bf16", "bf16", 1000 * 7, 1, 0.05),
    ("bf16_P4104_long", "bf16", "bf16", 4104 * 5, 4104, 0.0),
    ("f32_P768", "f32", "f32", 768 * 30, 768, 0.0),
    ("f32_P3072_long", "f32", "f32", 3072 * 5, 3072, 0.1),
    ("f32_P1", "f32", "f32", 4096, 1, 0.0),
    ("f32_P48", "f32", "f32", 48 * 333, 48, 0.0),
    ("f16_P96", "f16", "f16", 96 * 128, 96, 0.0),
    ("f16_P1", "f16", "f16", 3000, 1, 0.0),
    ("bf16_fp32state_P256", "bf16", "f32", 256 * 64, 256, 0.0),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_step_tasks_match_oracle(case):
    _run_case(*case)


# Period-one bf16 states over the whole bf16 range: per-row gradient scales from
# 2^-66 to 2^18 put the new vmean on subnormals, zero, every exponent in between
# and large values, each read through the kernel's square-root table; eps = 0 and
# eps = 2^101 lie outside the settings whose launches read the table
# (root_table_ok: 2^-126 <= eps <= 2^100), so those steps compute every stepsize.
WIDE_CASES = [
    ("bf16_P1_wide_b2_half", 256 * 96, 0.5, 1e-8, -66, 18),
    ("bf16_P1_wide_eps_small", 256 * 96, 0.999, 1e-12, -66, 18),
    ("bf16_P1_wide_eps_large", 64 * 75, 0.9, 1e-3, -40, 10),
    ("bf16_P1_wide_eps_zero_no_table", 256 * 96, 0.999, 0.0, -66, 18),
    ("bf16_P1_wide_eps_huge_no_table", 64 * 75, 0.999, 2.0 ** 101, -40, 10),
]


@pytest.mark.parametrize("case", WIDE_CASES, ids=[c[0] for c in WIDE_CASES])
def test_period_one_bf16_stepsize_over_the_value_range(case):
    name, n, b2, eps, e_lo, e_hi = case
    _run_case(name, "bf16", "bf16", n, 1, 0.0, e_lo=e_lo, e_hi=e_hi, b2=b2, eps=eps)


def _run_case(name, dt, sdt, n, period, wd, e_lo=-14, e_hi=-4, b2=0.999, eps=1e-8):
    print("case", name, flush=True)
    cb = _codebook()
    seed = sum(map(ord, name))
    pod = orc.largest_divisor_at_most(n, 256) if period == 1 else 0
    rows_v = n // period
    rows_m = n // (pod if period == 1 else period)
    p_np = syn.round_to(syn.normal(syn.make_key(seed, 1), n) * 0.02, dt)
    p_np = p_np.view(np.uint16) if p_np.dtype == np.float16 else p_np
    st_np = {"idx": np.zeros(n, np.uint8), "mag": np.zeros(rows_m, orc.NP_STORAGE[sdt]),
             "v": np.zeros(rows_v, orc.NP_STORAGE[sdt])}
    p_dev = gu.to_dev(p_np, dt)
    idx_dev = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
    mag_dev = torch.zeros(rows_m, dtype=gu.TORCH[sdt], device="cuda:0")
    v_dev = torch.zeros(rows_v, dtype=gu.TORCH[sdt], device="cuda:0")
    cb_dev = torch.from_numpy(cb).to("cuda:0")
    tables = _tables(cb_dev)
    lib = _lib.load()
    b1, lr = 0.9, 1e-3
    for step in range(1, 5):
        grows = n // period if period > 1 else (n // 64 if n % 64 == 0 else 1)
        g = syn.round_to(syn.row_scaled_normal(seed, step, grows, n // grows, e_lo, e_hi), dt).reshape(-1)
        g = g.view(np.uint16) if g.dtype == np.float16 else g
        g_dev = gu.to_dev(g, dt)
        bc1, bc2 = 1 - b1 ** step, 1 - b2 ** step
        task = np.zeros(1, dtype=_lib.STEP_TASK)
        task["p"], task["grad"], task["m_codebook"] = p_dev.data_ptr(), g_dev.data_ptr(), idx_dev.data_ptr()
        task["m_magnitude"], task["vmean"] = mag_dev.data_ptr(), v_dev.data_ptr()
        task["numel"], task["period"], task["period_one_divisor"] = n, period, pod
        task["param_dtype"], task["state_dtype"] = gu.CODE[dt], gu.CODE[sdt]
        task["beta1"], task["beta2"], task["lr"], task["eps"], task["weight_decay"] = b1, b2, lr, eps, wd
        task["bias_correction_1"], task["bias_correction_2"] = bc1, bc2
        _lib.check(lib.gefen_step_tasks(task.ctypes.data, 1, tables.data_ptr(), gu.stream()))
        rc = orc.lib().orc_gefen_step(gu.CODE[dt], gu.CODE[sdt], orc._ptr(p_np), orc._ptr(np.ascontiguousarray(g)),
                                      orc._ptr(st_np["idx"]), orc._ptr(st_np["mag"]), orc._ptr(st_np["v"]), n, period,
                                      pod, orc._ptr(cb), cb.size, b1, b2, lr, eps, wd, bc1, bc2, 1)
        assert rc == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(gu.to_np(idx_dev), st_np["idx"], err_msg="{} idx step {}".format(name, step))
        np.testing.assert_array_equal(gu.to_np(mag_dev), st_np["mag"], err_msg="{} mag step {}".format(name, step))
        vg = orc.to_f32(gu.to_np(v_dev), sdt)
        vo = orc.to_f32(st_np["v"], sdt)
        if period == 1:
            np.testing.assert_array_equal(vg, vo, err_msg="{} vmean step {}".format(name, step))
        elif sdt == "f32":
            np.testing.assert_allclose(vg, vo, rtol=4e-7 * 8, atol=0, err_msg="{} vmean".format(name))
        else:
            assert _ulps(gu.to_np(v_dev), st_np["v"]).max() <= 1
        pg = gu.to_np(p_dev)
        if dt == "f32":
            np.testing.assert_allclose(pg, p_np, rtol=1e-5, atol=1e-7, err_msg="{} p step {}".format(name, step))
            if period == 1:
                np.testing.assert_array_equal(pg, p_np)
        else:
            assert _ulps(pg, p_np).max() <= 1, "{} p step {}".format(name, step)
            if period == 1:
                np.testing.assert_array_equal(pg, p_np)


def _special_codebook(kind):
    if kind == "dense":   # thresholds ~1.9 cells of 2^-12 apart: the two-probe search
        cb = np.concatenate([[-1.0], np.linspace(-0.06, 0.06, 254), [1.0]]).astype(np.float32)
    elif kind == "denser":  # several thresholds per cell: the probing loop path
        cb = np.concatenate([[-1.0], np.linspace(-0.02, 0.02, 254), [1.0]]).astype(np.float32)
    elif kind == "wide":  # entries beyond [-1, 1] (a loaded, not learned, codebook)
        cb = np.sort(np.concatenate([np.linspace(-2.0, 2.0, 200), np.linspace(-0.1, 0.1, 56)])).astype(np.float32)
    else:                 # padded codebook with repeated entries
        cb = np.sort(np.concatenate([[-1.0, 1.0], np.repeat(np.linspace(-0.5, 0.5, 9), 28)[:254]])).astype(np.float32)
    return np.ascontiguousarray(cb)


@pytest.mark.parametrize("kind", ["dense", "denser", "wide", "repeated"])
@pytest.mark.parametrize("dt,period", [("bf16", 2048), ("bf16", 256), ("f32", 96), ("bf16", 1)])
def test_step_with_unusual_codebooks_and_nonfinite_gradients(kind, dt, period):
    """The two-probe search (dense), the general search (many thresholds per
    cell, thresholds below -1, duplicate codewords) and rows whose magnitude is
    0, inf or NaN: indices and magnitudes bit-exact, vmean and parameters NaN
    exactly where the oracle's are and otherwise within the usual bounds."""
    print("case", kind, dt, period, flush=True)
    cb = _special_codebook(kind)
    n = (period if period > 1 else 256) * 16
    pod = orc.largest_divisor_at_most(n, 256) if period == 1 else 0
    rows_m = n // (pod if period == 1 else period)
    rows_v = n // period
    p_np = syn.round_to(syn.normal(syn.make_key(77, 1), n) * 0.02, dt)
    st_np = {"idx": np.zeros(n, np.uint8), "mag": np.zeros(rows_m, orc.NP_STORAGE[dt]),
             "v": np.zeros(rows_v, orc.NP_STORAGE[dt])}
    p_dev = gu.to_dev(p_np, dt)
    idx_dev = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
    mag_dev = torch.zeros(rows_m, dtype=gu.TORCH[dt], device="cuda:0")
    v_dev = torch.zeros(rows_v, dtype=gu.TORCH[dt], device="cuda:0")
    tables = _tables(torch.from_numpy(cb).to("cuda:0"))
    lib = _lib.load()
    blk = pod if period == 1 else period
    for step in range(1, 4):
        g = syn.round_to(syn.row_scaled_normal(78, step, n // blk, blk, -14, -4), dt).reshape(-1).copy()
        if step == 1:
            g[:blk] = 0                      # zero magnitude block
        if step == 2:
            g[blk + 3] = np.float32(np.inf) if dt == "f32" else 0x7F80  # inf magnitude block
            g[2 * blk + 5] = np.float32(np.nan) if dt == "f32" else 0x7FC0  # NaN block
        g_dev = gu.to_dev(g, dt)
        bc1, bc2 = 1 - 0.9 ** step, 1 - 0.999 ** step
        task = np.zeros(1, dtype=_lib.STEP_TASK)
        task["p"], task["grad"], task["m_codebook"] = p_dev.data_ptr(), g_dev.data_ptr(), idx_dev.data_ptr()
        task["m_magnitude"], task["vmean"] = mag_dev.data_ptr(), v_dev.data_ptr()
        task["numel"], task["period"], task["period_one_divisor"] = n, period, pod
        task["param_dtype"] = task["state_dtype"] = gu.CODE[dt]
        task["beta1"], task["beta2"], task["lr"], task["eps"] = 0.9, 0.999, 1e-3, 1e-8
        task["bias_correction_1"], task["bias_correction_2"] = bc1, bc2
        _lib.check(lib.gefen_step_tasks(task.ctypes.data, 1, tables.data_ptr(), gu.stream()))
        orc.lib().orc_gefen_step(gu.CODE[dt], gu.CODE[dt], orc._ptr(p_np), orc._ptr(g), orc._ptr(st_np["idx"]),
                                 orc._ptr(st_np["mag"]), orc._ptr(st_np["v"]), n, period, pod, orc._ptr(cb), cb.size,
                                 0.9, 0.999, 1e-3, 1e-8, 0.0, bc1, bc2, 1)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(gu.to_np(idx_dev), st_np["idx"], err_msg="idx step {}".format(step))
        np.testing.assert_array_equal(gu.to_np(mag_dev), st_np["mag"], err_msg="mag step {}".format(step))
        # vmean and parameters, NaN where the oracle has NaN (any payload), else as in _run_case
        for what, got, want in (("vmean", gu.to_np(v_dev), st_np["v"]), ("params", gu.to_np(p_dev), p_np)):
            gf, wf = orc.to_f32(got, dt), orc.to_f32(want, dt)
            tag = "{} step {}".format(what, step)
            np.testing.assert_array_equal(np.isnan(gf), np.isnan(wf), err_msg=tag + " NaN positions")
            ok = ~np.isnan(wf)
            if period == 1:
                np.testing.assert_array_equal(gf[ok], wf[ok], err_msg=tag)
            elif dt == "f32":
                np.testing.assert_allclose(gf[ok], wf[ok], rtol=1e-5 if what == "params" else 2.0 ** -18,
                                           atol=1e-7 if what == "params" else 0, err_msg=tag)
            else:
                assert _ulps(got[ok], want[ok]).max(initial=0) <= 1, tag


def test_misaligned_views_take_the_scalar_path():
    """Parameters that start at an odd element offset still give identical indices."""
    cb = _codebook()
    n, period = 768 * 8, 768
    base = syn.round_to(syn.normal(syn.make_key(3, 1), n + 1) * 0.02, "bf16")
    p_np = base[1:].copy()
    big = gu.to_dev(base, "bf16")
    p_dev = big[1:]
    g = syn.round_to(syn.row_scaled_normal(3, 2, 8, 768, -14, -4), "bf16").reshape(-1)
    gbig = gu.to_dev(np.concatenate([np.zeros(1, np.uint16), g]), "bf16")
    g_dev = gbig[1:]
    idx_dev = torch.zeros(n + 1, dtype=torch.uint8, device="cuda:0")[1:]
    mag_dev = torch.zeros(8, dtype=torch.bfloat16, device="cuda:0")
    v_dev = torch.zeros(8, dtype=torch.bfloat16, device="cuda:0")
    st = {"idx": np.zeros(n, np.uint8), "mag": np.zeros(8, np.uint16), "v": np.zeros(8, np.uint16)}
    cb_dev = torch.from_numpy(cb).to("cuda:0")
    tables = _tables(cb_dev)
    task = np.zeros(1, dtype=_lib.STEP_TASK)
    task["p"], task["grad"], task["m_codebook"] = p_dev.data_ptr(), g_dev.data_ptr(), idx_dev.data_ptr()
    task["m_magnitude"], task["vmean"] = mag_dev.data_ptr(), v_dev.data_ptr()
    task["numel"], task["period"] = n, period
    task["param_dtype"], task["state_dtype"] = 2, 2
    task["beta1"], task["beta2"], task["lr"], task["eps"] = 0.9, 0.999, 1e-3, 1e-8
    task["bias_correction_1"], task["bias_correction_2"] = 0.1, 1 - 0.999
    _lib.check(_lib.load().gefen_step_tasks(task.ctypes.data, 1, tables.data_ptr(), gu.stream()))
    orc.lib().orc_gefen_step(2, 2, orc._ptr(p_np), orc._ptr(g), orc._ptr(st["idx"]), orc._ptr(st["mag"]),
                             orc._ptr(st["v"]), n, period, 0, orc._ptr(cb), 256, 0.9, 0.999, 1e-3, 1e-8, 0.0, 0.1,
                             1 - 0.999, 1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(gu.to_np(idx_dev), st["idx"])
    np.testing.assert_array_equal(gu.to_np(mag_dev), st["mag"])
    assert _ulps(gu.to_np(p_dev), p_np).max() <= 1


def test_many_tasks_in_one_call():
    """Tensors of mixed dtypes and periods in one gefen_step_tasks call: 36 tasks of each
    kernel shape, so each shape takes more than one launch (at most 30 tasks per launch)."""
    cb = _codebook()
    cb_dev = torch.from_numpy(cb).to("cuda:0")
    tables = _tables(cb_dev)
    specs = [("bf16", 2048 * 3, 2048), ("bf16", 1024, 1), ("f32", 96 * 10, 96), ("bf16", 768 * 4, 768)] * 36
    tasks = np.zeros(len(specs), dtype=_lib.STEP_TASK)
    devs, oracle = [], []
    for i, (dt, n, period) in enumerate(specs):
        pod = orc.largest_divisor_at_most(n, 256) if period == 1 else 0
        rows_m = n // (pod if period == 1 else period)
        p = syn.round_to(syn.normal(syn.make_key(11, i), n) * 0.02, dt)
        g = syn.round_to(syn.row_scaled_normal(11, 1000 + i, max(1, n // 64), 64, -14, -4), dt).reshape(-1)
        assert g.size == n
        d = {"p": gu.to_dev(p, dt), "g": gu.to_dev(g, dt), "idx": torch.zeros(n, dtype=torch.uint8, device="cuda:0"),
             "mag": torch.zeros(rows_m, dtype=gu.TORCH[dt], device="cuda:0"),
             "v": torch.zeros(n // period, dtype=gu.TORCH[dt], device="cuda:0")}
        devs.append(d)
        o = {"p": p.copy(), "g": g, "idx": np.zeros(n, np.uint8), "mag": np.zeros(rows_m, orc.NP_STORAGE[dt]),
             "v": np.zeros(n // period, orc.NP_STORAGE[dt]), "dt": dt, "n": n, "period": period, "pod": pod}
        oracle.append(o)
        t = tasks[i]
        t["p"], t["grad"], t["m_codebook"] = d["p"].data_ptr(), d["g"].data_ptr(), d["idx"].data_ptr()
        t["m_magnitude"], t["vmean"] = d["mag"].data_ptr(), d["v"].data_ptr()
        t["numel"], t["period"], t["period_one_divisor"] = n, period, pod
        t["param_dtype"] = t["state_dtype"] = gu.CODE[dt]
        t["beta1"], t["beta2"], t["lr"], t["eps"] = 0.9, 0.999, 1e-3, 1e-8
        t["bias_correction_1"], t["bias_correction_2"] = 0.1, 1 - 0.999
    _lib.check(_lib.load().gefen_step_tasks(tasks.ctypes.data, len(specs), tables.data_ptr(), gu.stream()))
    for o in oracle:
        orc.lib().orc_gefen_step(gu.CODE[o["dt"]], gu.CODE[o["dt"]], orc._ptr(o["p"]), orc._ptr(o["g"]),
                                 orc._ptr(o["idx"]), orc._ptr(o["mag"]), orc._ptr(o["v"]), o["n"], o["period"],
                                 o["pod"], orc._ptr(cb), 256, 0.9, 0.999, 1e-3, 1e-8, 0.0, 0.1, 1 - 0.999, 1)
    torch.cuda.synchronize()
    for d, o in zip(devs, oracle):
        np.testing.assert_array_equal(gu.to_np(d["idx"]), o["idx"])
        np.testing.assert_array_equal(gu.to_np(d["mag"]), o["mag"])


def test_small_launches_on_the_side_stream_match_the_oracle():
    """A call mixing large launches (at least 2^20 elements) with small ones: the
    small launches run on the library's second stream, forked from and joined back
    to the caller's stream.  Every tensor matches the oracle, including period-one
    tensors on both streams (each reading the shared stepsize table) and a read of
    the results right after the call on the caller's stream."""
    cb = _codebook()
    cb_dev = torch.from_numpy(cb).to("cuda:0")
    tables = _tables(cb_dev)
    specs = [("bf16", 2048 * 600, 2048), ("bf16", 256 * 4200, 1), ("bf16", 256 * 12, 1), ("bf16", 768 * 5, 768),
             ("f32", 96 * 8, 96), ("bf16", 2304, 18), ("f32", 1024 * 1100, 1024)]
    tasks = np.zeros(len(specs), dtype=_lib.STEP_TASK)
    devs, oracle = [], []
    for i, (dt, n, period) in enumerate(specs):
        pod = orc.largest_divisor_at_most(n, 256) if period == 1 else 0
        rows_m = n // (pod if period == 1 else period)
        p = syn.round_to(syn.normal(syn.make_key(21, i), n) * 0.02, dt)
        g = syn.round_to(syn.row_scaled_normal(21, 500 + i, n // 64, 64, -14, -4), dt).reshape(-1)
        assert g.size == n and p.size == n
        d = {"p": gu.to_dev(p, dt), "g": gu.to_dev(g, dt), "idx": torch.zeros(n, dtype=torch.uint8, device="cuda:0"),
             "mag": torch.zeros(rows_m, dtype=gu.TORCH[dt], device="cuda:0"),
             "v": torch.zeros(n // period, dtype=gu.TORCH[dt], device="cuda:0")}
        devs.append(d)
        oracle.append({"p": p.copy(), "g": g, "idx": np.zeros(n, np.uint8), "mag": np.zeros(rows_m, orc.NP_STORAGE[dt]),
                       "v": np.zeros(n // period, orc.NP_STORAGE[dt]), "dt": dt, "n": n, "period": period, "pod": pod})
        t = tasks[i]
        t["p"], t["grad"], t["m_codebook"] = d["p"].data_ptr(), d["g"].data_ptr(), d["idx"].data_ptr()
        t["m_magnitude"], t["vmean"] = d["mag"].data_ptr(), d["v"].data_ptr()
        t["numel"], t["period"], t["period_one_divisor"] = n, period, pod
        t["param_dtype"] = t["state_dtype"] = gu.CODE[dt]
        t["beta1"], t["beta2"], t["lr"], t["eps"] = 0.9, 0.999, 1e-3, 1e-8
        t["bias_correction_1"], t["bias_correction_2"] = 0.1, 1 - 0.999
    _lib.check(_lib.load().gefen_step_tasks(tasks.ctypes.data, len(specs), tables.data_ptr(), gu.stream()))
    # read on the caller's stream without a device-wide synchronisation first
    got = [{k: d[k].clone() for k in ("p", "idx", "mag", "v")} for d in devs]
    for o in oracle:
        orc.lib().orc_gefen_step(gu.CODE[o["dt"]], gu.CODE[o["dt"]], orc._ptr(o["p"]), orc._ptr(o["g"]),
                                 orc._ptr(o["idx"]), orc._ptr(o["mag"]), orc._ptr(o["v"]), o["n"], o["period"],
                                 o["pod"], orc._ptr(cb), 256, 0.9, 0.999, 1e-3, 1e-8, 0.0, 0.1, 1 - 0.999, 1)
    torch.cuda.synchronize()
    for (dt, n, period), d, o in zip(specs, got, oracle):
        print("side stream case", dt, n, period, flush=True)
        np.testing.assert_array_equal(gu.to_np(d["idx"]), o["idx"])
        np.testing.assert_array_equal(gu.to_np(d["mag"]), o["mag"])
        pg = gu.to_np(d["p"])
        if period == 1:
            np.testing.assert_array_equal(gu.to_np(d["v"]), o["v"])
            np.testing.assert_array_equal(pg, o["p"])
        elif dt == "f32":
            np.testing.assert_allclose(pg, o["p"], rtol=1e-5, atol=1e-7)
        else:
            assert _ulps(pg, o["p"]).max() <= 1


def test_invalid_arguments_raise_value_error():
    lib = _lib.load()
    task = np.zeros(1, dtype=_lib.STEP_TASK)
    x = torch.zeros(10, device="cuda:0")
    task["p"] = task["grad"] = task["m_codebook"] = task["m_magnitude"] = task["vmean"] = x.data_ptr()
    task["numel"], task["period"] = 10, 3
    task["bias_correction_1"] = task["bias_correction_2"] = 0.5
    tables = torch.zeros(int(lib.gefen_codebook_tables_size()), dtype=torch.uint8, device="cuda:0")
    with pytest.raises(ValueError, match="does not divide"):
        _lib.check(lib.gefen_step_tasks(task.ctypes.data, 1, tables.data_ptr(), gu.stream()))
    task["period"] = 5
    task["bias_correction_1"] = 0.0
    with pytest.raises(ValueError, match="bias_correction_1"):
        _lib.check(lib.gefen_step_tasks(task.ctypes.data, 1, tables.data_ptr(), gu.stream()))


@pytest.mark.parametrize("kind", ["dense", "denser", "wide", "repeated"])
@pytest.mark.parametrize("dt,block", [("bf16", 2048), ("bf16", 256), ("f32", 96), ("f32", 1024)])
def test_muon_momentum_with_unusual_codebooks_and_nonfinite_gradients(kind, dt, block):
    """GefenMuon momentum through gefen_muon_tasks: general search path, row tables
    (whole-wave rows) and rows whose magnitude is 0, inf or NaN, bit-exact against
    the oracle including the Nesterov output."""
    print("muon case", kind, dt, block, flush=True)
    cb = _special_codebook(kind)
    rows = 12
    n = rows * block
    idx_np = np.zeros(n, np.uint8)
    mag_np = np.zeros(rows, orc.NP_STORAGE[dt])
    idx_dev = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
    mag_dev = torch.zeros(rows, dtype=gu.TORCH[dt], device="cuda:0")
    tables = _tables(torch.from_numpy(cb).to("cuda:0"))
    lib = _lib.load()
    for step in range(1, 4):
        g = syn.round_to(syn.row_scaled_normal(79, step, rows, block, -14, -4), dt).reshape(-1).copy()
        if step == 1:
            g[:block] = 0
        if step == 2:
            g[block + 3] = np.float32(np.inf) if dt == "f32" else 0x7F80
            g[2 * block + 5] = np.float32(np.nan) if dt == "f32" else 0x7FC0
        g_dev = gu.to_dev(g, dt)
        out_dev = torch.empty(n, dtype=gu.TORCH[dt], device="cuda:0")
        task = np.zeros(1, dtype=_lib.MUON_TASK)
        task["grad"], task["m_codebook"], task["m_magnitude"] = g_dev.data_ptr(), idx_dev.data_ptr(), mag_dev.data_ptr()
        task["out"], task["numel"], task["block"] = out_dev.data_ptr(), n, block
        task["grad_dtype"] = task["state_dtype"] = gu.CODE[dt]
        task["momentum"], task["nesterov"] = 0.95, 1
        _lib.check(lib.gefen_muon_tasks(task.ctypes.data, 1, tables.data_ptr(), gu.stream()))
        ref = np.empty(n, dtype=orc.NP_STORAGE[dt])
        assert orc.lib().orc_muon_momentum(gu.CODE[dt], gu.CODE[dt], orc._ptr(g), orc._ptr(idx_np), orc._ptr(mag_np),
                                           orc._ptr(ref), n, block, orc._ptr(cb), cb.size, 0.95, 1) == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(gu.to_np(idx_dev), idx_np, err_msg="idx step {}".format(step))
        np.testing.assert_array_equal(gu.to_np(mag_dev), mag_np, err_msg="mag step {}".format(step))
        got = gu.to_np(out_dev)
        both_nan = np.isnan(orc.to_f32(got, dt)) & np.isnan(orc.to_f32(ref, dt))
        np.testing.assert_array_equal(np.where(both_nan, 0, got), np.where(both_nan, 0, ref), err_msg="out step {}".format(step))


# CodebookTables (gefen_amd/csrc/common.h): cb 256 f32, thr 260 f32, bucket8 4112 u8,
# bucket_fine 8208 u8, bucket 4100 u16, K, max_probe, max_probe_fine, pad i32, then
# the 16-byte aligned bf16 table
_BUCKET8_OFFSET, _FINE_OFFSET = 2064, 6176
_MAX_PROBE_OFFSET = 22588  # max_probe, then max_probe_fine
_NB16_OFFSET = 22608
_NB16_LO, _NB16_SIDE = 0x3580, 0x3F82 - 0x3580


@pytest.mark.parametrize("kind,probes", [("learned", 1), ("uniform", 1), ("dense", 2), ("denser", 3),
                                         ("repeated", 3)])
def test_codebook_tables_choose_the_search(kind, probes):
    """bucket8[e] and bucket_fine[e] are the oracle's nearest index of the bucket
    edges -1 + e/2048 and -1 + e/4096 (the count of thresholds below them) for
    every e, and max_probe_fine puts each codebook on the search the 16-bit
    parameter step kernels take for it: one probe for the learned and the
    uniform codebook, two for thresholds ~1.9 fine cells apart, the general loop
    (3 and more) for denser or repeated codewords.  A coarse bucket holds two
    fine ones, so max_probe (the other kernels' choice) is never below it."""
    print("tables", kind, flush=True)
    if kind == "learned":
        cb = _codebook()
    elif kind == "uniform":
        cb = np.linspace(-1.0, 1.0, 256).astype(np.float32)
    else:
        cb = _special_codebook(kind)
    tables = gu.to_np(_tables(torch.from_numpy(cb).to("cuda:0")))
    for off, cells in ((_BUCKET8_OFFSET, 4096), (_FINE_OFFSET, 8192)):
        edges = (-1.0 + np.arange(cells + 1, dtype=np.float64) * (2.0 / cells)).astype(np.float32)
        np.testing.assert_array_equal(tables[off:off + cells + 1], orc.nearest(cb, edges).astype(np.uint8))
    max_probe, max_probe_fine = (int(v) for v in tables[_MAX_PROBE_OFFSET:_MAX_PROBE_OFFSET + 8].view(np.int32))
    if probes < 3:
        assert max_probe_fine == probes
    else:
        assert max_probe_fine >= 3
    assert max_probe >= max_probe_fine


@pytest.mark.parametrize("cbkind", ["learned", "zero_threshold"])
def test_bf16_nearest_table_matches_oracle(cbkind):
    """Every entry of the codebook tables' bf16 nearest-index table (entry
    side + i for the bf16 bits lo + i, side - 1 - i for their negatives) equals
    the oracle's nearest search for that value."""
    print("nb16", cbkind, flush=True)
    if cbkind == "learned":
        data, _ = load("exact_dp")
        cb = np.ascontiguousarray(data["hist_k256_forced/codebook"], dtype=np.float32)
    else:
        cb = np.linspace(-1.0, 1.0, 256).astype(np.float32)
    lib = _lib.load()
    assert int(lib.gefen_codebook_tables_size()) == _NB16_OFFSET + (2 * _NB16_SIDE + 15) // 16 * 16
    tables = gu.to_np(_tables(torch.from_numpy(cb).to("cuda:0")))
    got = tables[_NB16_OFFSET:_NB16_OFFSET + 2 * _NB16_SIDE]
    i = np.arange(_NB16_SIDE, dtype=np.uint32)
    bits = np.empty(2 * _NB16_SIDE, np.uint32)
    bits[_NB16_SIDE + i] = _NB16_LO + i
    bits[_NB16_SIDE - 1 - i] = 0x8000 | (_NB16_LO + i)
    x = (bits << 16).view(np.float32)
    np.testing.assert_array_equal(got, orc.nearest(cb, x).astype(np.uint8))


@pytest.mark.parametrize("cbkind", ["learned", "zero_threshold"])
@pytest.mark.parametrize("block", [2048, 1536, 256])
@pytest.mark.parametrize("shifts", [(0,), (-100, 0, 100, 110)])
def test_muon_momentum_quotients_across_forty_octaves(cbkind, block, shifts):
    """bf16 GefenMuon momentum whose quotients x = m / magnitude spread over
    2^-40 .. 1 (gradients sign * 2^e, e uniform in [-40, 0]): the bf16 nearest
    table covers 2^-20 <= |x| <= 1.0078 and the rest takes the two-probe search.
    With a codebook whose decision threshold between its two middle entries is
    0 (linspace(-1, 1, 256)), +-tiny quotients and zeros land on either side.
    Row r's gradients are scaled by 2^shifts[r % len(shifts)]: with (-100, 0,
    100, 110) rows reach bf16 subnormals and magnitudes beyond 2^100 (which
    take the float64 quotient).  Bit-exact against the oracle over three steps."""
    print("muon octaves", cbkind, block, shifts, flush=True)
    if cbkind == "learned":
        data, _ = load("exact_dp")
        cb = np.ascontiguousarray(data["hist_k256_forced/codebook"], dtype=np.float32)
    else:
        cb = np.linspace(-1.0, 1.0, 256).astype(np.float32)
    rows = 16
    n = rows * block
    rng = np.random.default_rng(block)
    idx_np = np.zeros(n, np.uint8)
    mag_np = np.zeros(rows, np.uint16)
    idx_dev = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
    mag_dev = torch.zeros(rows, dtype=torch.bfloat16, device="cuda:0")
    tables = _tables(torch.from_numpy(cb).to("cuda:0"))
    lib = _lib.load()
    for step in range(1, 4):
        e = rng.integers(-40, 1, n).astype(np.float64)
        shift = np.asarray(shifts, np.float64)[(np.arange(n) // block) % len(shifts)]
        g32 = (np.where(rng.random(n) < 0.5, -1.0, 1.0) * np.exp2(e + shift) * (1.0 + rng.random(n))).astype(np.float32)
        g32[rng.random(n) < 0.01] = 0.0
        g = syn.round_to(g32, "bf16").reshape(-1).copy()
        g_dev = gu.to_dev(g, "bf16")
        out_dev = torch.empty(n, dtype=torch.bfloat16, device="cuda:0")
        task = np.zeros(1, dtype=_lib.MUON_TASK)
        task["grad"], task["m_codebook"], task["m_magnitude"] = g_dev.data_ptr(), idx_dev.data_ptr(), mag_dev.data_ptr()
        task["out"], task["numel"], task["block"] = out_dev.data_ptr(), n, block
        task["grad_dtype"] = task["state_dtype"] = gu.CODE["bf16"]
        task["momentum"], task["nesterov"] = 0.95, 1
        _lib.check(lib.gefen_muon_tasks(task.ctypes.data, 1, tables.data_ptr(), gu.stream()))
        ref = np.empty(n, dtype=np.uint16)
        assert orc.lib().orc_muon_momentum(gu.CODE["bf16"], gu.CODE["bf16"], orc._ptr(g), orc._ptr(idx_np),
                                           orc._ptr(mag_np), orc._ptr(ref), n, block, orc._ptr(cb), cb.size,
                                           0.95, 1) == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(gu.to_np(idx_dev), idx_np, err_msg="idx step {}".format(step))
        np.testing.assert_array_equal(gu.to_np(mag_dev), mag_np, err_msg="mag step {}".format(step))
        np.testing.assert_array_equal(gu.to_np(out_dev), ref, err_msg="out step {}".format(step))

"""Randomised parity of the reference's operator entry points (gefen.kernels.*,
automatic_gefen_fused.py) with the CPU oracle: the given-stepsize and
given-vmean updates, the period-one update and GefenMuon's momentum, each over
random dtypes, block counts and lengths (odd lengths, rows of one element,
long rows), codebook sizes, hyperparameters and, where the reference allows
it, packed 4-bit indices (a byte shared by two rows, a kept high nibble past
an odd end, sentinel bytes after the buffer that must stay as they were).
The stepsize / vmean is given per block, so every output is bit-exact against
the oracle: indices (or packed bytes), magnitudes, parameters and the momentum
output, over three steps."""

import numpy as np
import pytest
import torch

import gpu_util as gu
from golden_util import load
from gefen_amd import synthetic as syn
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SENTINEL = 8
PAIRS = [("bf16", "bf16"), ("bf16", "bf16"), ("f16", "f16"), ("f32", "f32"), ("bf16", "f32"), ("f16", "f32")]


def _codebook(k):
    if k == 256:
        data, _ = load("exact_dp")
        return np.ascontiguousarray(data["hist_k256_forced/codebook"], dtype=np.float32)
    t = np.linspace(-1.0, 1.0, k)
    return np.ascontiguousarray(np.sign(t) * np.abs(t) ** 1.5, dtype=np.float32)


def _bits(a):
    return a.view(np.uint16) if a.dtype == np.float16 else a


def _period(rng):
    return int([1, 2, 3, 5, 8, 13, 64, 96, 100, 257, 768, 1025, 2048, 3000][rng.integers(14)])


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_given_stepsize_and_vmean_updates_match_oracle(seed):
    from gefen_amd.kernels.automatic_gefen_fused import (automatic_gefen_fused_update_cuda,
                                                         automatic_gefen_fused_update_from_vmean_cuda)

    rng = np.random.default_rng(seed)
    for case in range(40):
        entry = ["stepsize", "vmean"][rng.integers(2)]
        packed = bool(rng.random() < 0.4)
        dt, sdt = PAIRS[rng.integers(len(PAIRS))]
        vdt = sdt if rng.random() < 0.7 else ["bf16", "f16", "f32"][rng.integers(3)]
        k = 16 if packed else int([16, 64, 256, 256][rng.integers(4)])
        period = _period(rng)
        rows = int(rng.integers(1, max(2, min(60, 40000 // period))))
        n = rows * period
        b1, lr, eps = float(rng.uniform(0.8, 0.95)), float(10.0 ** rng.uniform(-4, -2.5)), [1e-8, 1e-6][rng.integers(2)]
        tag = "case {} {} packed={} {}/{}/{} rows={} period={} k={}".format(case, entry, packed, dt, sdt, vdt,
                                                                              rows, period, k)
        cb = _codebook(k)
        cbd = torch.from_numpy(cb).to("cuda:0")
        p_np = _bits(syn.round_to(syn.normal(syn.make_key(seed, case), n) * 0.02, dt))
        mag_np = orc.from_f32(rng.uniform(1e-4, 1e-2, rows).astype(np.float32), sdt)
        pd = gu.to_dev(p_np, dt)
        mag = gu.to_dev(mag_np, sdt).reshape(rows, 1)
        if packed:
            idx_np = rng.integers(0, 256, (n + 1) // 2 + SENTINEL, dtype=np.uint8)
            buf = torch.from_numpy(idx_np.copy()).to("cuda:0")
            sign = buf[: idx_np.size - SENTINEL]
        else:
            idx_np = rng.integers(0, k, n, dtype=np.uint8)
            buf = sign = torch.from_numpy(idx_np.copy()).to("cuda:0")
        for step in (1, 2, 3):
            g_np = _bits(syn.round_to(syn.row_scaled_normal(seed * 97 + case, step, rows, period, -16, -4), dt))
            g_np = g_np.reshape(-1)
            gd = gu.to_dev(g_np, dt).reshape(rows, period)
            bc1, bc2 = 1 - b1 ** step, 1 - 0.999 ** step
            idx = orc.unpack_nibbles(idx_np[: idx_np.size - SENTINEL], n) if packed else idx_np
            if entry == "vmean":
                vm_np = orc.from_f32(rng.uniform(1e-12, 1e-4, rows).astype(np.float32), vdt)
                automatic_gefen_fused_update_from_vmean_cuda(pd, gd, sign, mag, gu.to_dev(vm_np, vdt).reshape(rows, 1),
                                                             cbd, packed, b1, lr, bc1, bc2, eps)
                orc.gefen_update_given(dt, sdt, p_np, g_np, idx, mag_np, period, cb, b1, lr, vmean=vm_np, vdtype=vdt,
                                       bc1=bc1, bc2=bc2, eps=eps)
            else:
                ss = rng.uniform(1.0, 100.0, rows).astype(np.float32)
                automatic_gefen_fused_update_cuda(pd, gd, sign, mag, torch.from_numpy(ss).to("cuda:0").reshape(rows, 1),
                                                  cbd, packed, b1, lr)
                orc.gefen_update_given(dt, sdt, p_np, g_np, idx, mag_np, period, cb, b1, lr, stepsize=ss)
            if packed:
                body = idx_np[: idx_np.size - SENTINEL]
                orc.pack_nibbles(idx, body)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(gu.to_np(buf), idx_np, err_msg=tag + " indices step {}".format(step))
            np.testing.assert_array_equal(gu.to_np(mag).reshape(-1), mag_np, err_msg=tag + " magnitudes")
            np.testing.assert_array_equal(gu.to_np(pd), p_np, err_msg=tag + " parameters")
    print("seed", seed, "40 given-stepsize / given-vmean cases match the oracle", flush=True)


@pytest.mark.parametrize("seed", [4, 5])
def test_random_period_one_updates_match_oracle(seed):
    from gefen_amd.kernels.automatic_gefen_fused import automatic_gefen_period1_update_cuda

    rng = np.random.default_rng(seed)
    for case in range(30):
        dt, sdt = PAIRS[rng.integers(len(PAIRS))]
        n = int(rng.integers(1, 30000))
        divs = [d for d in orc.divisors(n) if d <= 256]
        pod = int(divs[rng.integers(len(divs))])          # any divisor the entry point accepts
        b1, b2 = float(rng.uniform(0.8, 0.95)), float(rng.uniform(0.9, 0.9999))
        lr, eps = float(10.0 ** rng.uniform(-4, -2.5)), [1e-8, 1e-6, 1e-10][rng.integers(3)]
        tag = "case {} {}/{} n={} pod={}".format(case, dt, sdt, n, pod)
        cb = _codebook(256)
        cbd = torch.from_numpy(cb).to("cuda:0")
        p_np = _bits(syn.round_to(syn.normal(syn.make_key(seed, case), n) * 0.02, dt))
        st = {"idx": np.zeros(n, np.uint8), "mag": np.zeros(n // pod, orc.NP_STORAGE[sdt]),
              "v": np.zeros(n, orc.NP_STORAGE[sdt])}
        pd = gu.to_dev(p_np, dt)
        sign = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
        mag = torch.zeros(n // pod, 1, dtype=gu.TORCH[sdt], device="cuda:0")
        vm = torch.zeros(n, 1, dtype=gu.TORCH[sdt], device="cuda:0")
        for step in (1, 2, 3):
            g_np = _bits(syn.round_to(syn.row_scaled_normal(seed * 89 + case, step, n // pod, pod, -16, -4), dt))
            g_np = g_np.reshape(-1)
            bc1, bc2 = 1 - b1 ** step, 1 - b2 ** step
            automatic_gefen_period1_update_cuda(pd, gu.to_dev(g_np, dt), sign, mag, vm, cbd, pod, b1, b2, lr, bc1, bc2,
                                                eps)
            rc = orc.lib().orc_gefen_step(orc.DT[dt], orc.DT[sdt], orc._ptr(p_np), orc._ptr(g_np), orc._ptr(st["idx"]),
                                          orc._ptr(st["mag"]), orc._ptr(st["v"]), n, 1, pod, orc._ptr(cb), cb.size,
                                          b1, b2, lr, eps, 0.0, bc1, bc2, 1)
            assert rc == 0
            torch.cuda.synchronize()
            np.testing.assert_array_equal(gu.to_np(sign), st["idx"], err_msg=tag + " indices step {}".format(step))
            np.testing.assert_array_equal(gu.to_np(mag).reshape(-1), st["mag"], err_msg=tag + " magnitudes")
            np.testing.assert_array_equal(gu.to_np(vm).reshape(-1), st["v"], err_msg=tag + " vmean")
            np.testing.assert_array_equal(gu.to_np(pd), p_np, err_msg=tag + " parameters")
    print("seed", seed, "30 period-one cases match the oracle", flush=True)


@pytest.mark.parametrize("seed", [6, 7])
def test_random_muon_momentum_entry_point_matches_oracle(seed):
    from gefen_amd.kernels.automatic_gefen_fused import automatic_gefen_muon_momentum_cuda

    rng = np.random.default_rng(seed)
    for case in range(30):
        packed = bool(rng.random() < 0.4)
        dt, sdt = PAIRS[rng.integers(len(PAIRS))]
        k = 16 if packed else int([16, 256][rng.integers(2)])
        period = _period(rng)
        rows = int(rng.integers(1, max(2, min(60, 40000 // period))))
        n = rows * period
        mom = float(rng.uniform(0.8, 0.99))
        tag = "case {} packed={} {}/{} rows={} period={} k={}".format(case, packed, dt, sdt, rows, period, k)
        cb = _codebook(k)
        cbd = torch.from_numpy(cb).to("cuda:0")
        mag_np = orc.from_f32(rng.uniform(1e-4, 1e-2, rows).astype(np.float32), sdt)
        mag = gu.to_dev(mag_np, sdt).reshape(rows, 1)
        if packed:
            idx_np = rng.integers(0, 256, (n + 1) // 2 + SENTINEL, dtype=np.uint8)
            buf = torch.from_numpy(idx_np.copy()).to("cuda:0")
            sign = buf[: idx_np.size - SENTINEL]
        else:
            idx_np = rng.integers(0, k, n, dtype=np.uint8)
            buf = sign = torch.from_numpy(idx_np.copy()).to("cuda:0")
        for step in (1, 2, 3):
            g_np = _bits(syn.round_to(syn.row_scaled_normal(seed * 83 + case, step, rows, period, -14, -6), dt))
            g_np = np.ascontiguousarray(g_np.reshape(-1))
            out = torch.empty(rows, period, dtype=gu.TORCH[dt], device="cuda:0")
            automatic_gefen_muon_momentum_cuda(gu.to_dev(g_np, dt).reshape(rows, period), sign, mag, cbd, out,
                                               packed, mom)
            idx = orc.unpack_nibbles(idx_np[: idx_np.size - SENTINEL], n) if packed else idx_np
            ref = np.empty(n, dtype=orc.NP_STORAGE[dt])
            assert orc.lib().orc_muon_momentum(orc.DT[dt], orc.DT[sdt], orc._ptr(g_np), orc._ptr(idx),
                                               orc._ptr(mag_np), orc._ptr(ref), n, period, orc._ptr(cb), cb.size,
                                               mom, 0) == 0
            if packed:
                orc.pack_nibbles(idx, idx_np[: idx_np.size - SENTINEL])
            torch.cuda.synchronize()
            np.testing.assert_array_equal(gu.to_np(buf), idx_np, err_msg=tag + " indices step {}".format(step))
            np.testing.assert_array_equal(gu.to_np(mag).reshape(-1), mag_np, err_msg=tag + " magnitudes")
            np.testing.assert_array_equal(gu.to_np(out).reshape(-1), ref, err_msg=tag + " momentum")
    print("seed", seed, "30 momentum cases match the oracle", flush=True)

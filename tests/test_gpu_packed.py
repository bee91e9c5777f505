"""Packed 4-bit codebook indices (automatic_gefen_fused_kernel.cu:14-57) through the
given-vmean, given-stepsize and GefenMuon momentum entry points.

The oracle of a packed call is the unpacked update on the unpacked nibbles,
followed by packing the new indices (low four bits, the other nibble of each
byte untouched).  Cases cover odd periods (a byte shared by two rows), odd
element counts (the high nibble past the end is kept), rows of one element,
and all three lane-group widths of the packed kernels; the packed buffer is a
slice of a larger one whose tail must stay as it was."""

import numpy as np
import pytest
import torch

import gpu_util as gu
from golden_util import load
from gefen_amd import synthetic as syn
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SENTINEL = 8


def _codebook(k):
    if k == 256:
        data, _ = load("exact_dp")
        return np.ascontiguousarray(data["hist_k256_forced/codebook"], dtype=np.float32)
    t = np.linspace(-1.0, 1.0, k)
    return np.ascontiguousarray(np.sign(t) * np.abs(t) ** 1.5, dtype=np.float32)


def _state(seed, n, rows, sdt):
    """Random packed nibbles (plus sentinel bytes) and random positive magnitudes."""
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, (n + 1) // 2 + SENTINEL, dtype=np.uint8)
    mag = orc.from_f32(rng.uniform(1e-4, 1e-2, rows).astype(np.float32), sdt)
    return packed, mag


def _bits(a):
    """float16 storage as its uint16 bit patterns (the oracle and gpu_util convention)."""
    return a.view(np.uint16) if a.dtype == np.float16 else a


def _packed_dev(packed):
    buf = torch.from_numpy(packed.copy()).to("cuda:0")
    return buf, buf[: packed.size - SENTINEL]


def _ref_packed(packed_np, n, new_idx):
    ref = packed_np.copy()
    body = ref[: ref.size - SENTINEL]
    orc.pack_nibbles(new_idx, body)
    return ref


UPDATE_CASES = [
    # (entry, param dtype, state dtype, rows, period, codebook size)
    ("vmean", "f32", "f32", 10, 96, 16),
    ("vmean", "bf16", "bf16", 7, 33, 256),     # odd period, odd numel
    ("vmean", "f32", "f32", 5, 3000, 16),      # 256 lanes per row
    ("vmean", "bf16", "f32", 3, 1025, 16),     # odd long rows
    ("stepsize", "f16", "f16", 9, 5, 16),      # odd period, odd numel, 16 lanes per row
    ("stepsize", "bf16", "f32", 301, 1, 256),  # rows of one element
    ("stepsize", "f32", "f32", 40, 130, 256),
]


@pytest.mark.parametrize("entry,dt,sdt,rows,period,k", UPDATE_CASES)
def test_packed_update_matches_the_unpacked_oracle(entry, dt, sdt, rows, period, k):
    from gefen_amd.kernels.automatic_gefen_fused import (automatic_gefen_fused_update_cuda,
                                                         automatic_gefen_fused_update_from_vmean_cuda)

    print("packed update", entry, dt, sdt, rows, period, k, flush=True)
    n = rows * period
    cb = _codebook(k)
    cbd = torch.from_numpy(cb).to("cuda:0")
    p_np = _bits(syn.round_to(syn.normal(syn.make_key(5, 1), n) * 0.02, dt))
    packed_np, mag_np = _state(n + k, n, rows, sdt)
    rng = np.random.default_rng(rows * period)
    vm_np = orc.from_f32(rng.uniform(1e-10, 1e-4, rows).astype(np.float32), sdt)
    pd = gu.to_dev(p_np, dt)
    buf, packed = _packed_dev(packed_np)
    mag = gu.to_dev(mag_np, sdt).reshape(rows, 1)
    b1, lr, eps = 0.9, 1e-3, 1e-8
    for step in (1, 2, 3):
        g_np = syn.round_to(syn.row_scaled_normal(17, step, rows, period, -14, -4), dt).reshape(-1)
        gd = gu.to_dev(g_np, dt).reshape(rows, period)
        bc1, bc2 = 1 - b1 ** step, 1 - 0.999 ** step
        idx = orc.unpack_nibbles(packed_np[: packed_np.size - SENTINEL], n)
        if entry == "vmean":
            automatic_gefen_fused_update_from_vmean_cuda(pd, gd, packed, mag, gu.to_dev(vm_np, sdt).reshape(rows, 1),
                                                         cbd, True, b1, lr, bc1, bc2, eps)
            orc.gefen_update_given(dt, sdt, p_np, g_np, idx, mag_np, period, cb, b1, lr, vmean=vm_np,
                                   bc1=bc1, bc2=bc2, eps=eps)
        else:
            ss = rng.uniform(1.0, 100.0, rows).astype(np.float32)
            automatic_gefen_fused_update_cuda(pd, gd, packed, mag, torch.from_numpy(ss).to("cuda:0").reshape(rows, 1),
                                              cbd, True, b1, lr)
            orc.gefen_update_given(dt, sdt, p_np, g_np, idx, mag_np, period, cb, b1, lr, stepsize=ss)
        packed_np = _ref_packed(packed_np, n, idx)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(gu.to_np(buf), packed_np, err_msg="packed indices, step {}".format(step))
        np.testing.assert_array_equal(gu.to_np(mag).reshape(-1), mag_np, err_msg="magnitudes")
        np.testing.assert_array_equal(gu.to_np(pd), p_np, err_msg="parameters")


MUON_CASES = [
    ("bf16", "bf16", 12, 64, 16),
    ("bf16", "bf16", 5, 77, 256),   # odd period, odd numel
    ("f32", "f32", 100, 1, 16),     # rows of one element
    ("bf16", "f32", 3, 2500, 16),   # 256 lanes per row
]


@pytest.mark.parametrize("dt,sdt,rows,period,k", MUON_CASES)
def test_packed_muon_momentum_matches_the_unpacked_oracle(dt, sdt, rows, period, k):
    from gefen_amd.kernels.automatic_gefen_fused import automatic_gefen_muon_momentum_cuda

    print("packed muon", dt, sdt, rows, period, k, flush=True)
    n = rows * period
    cb = _codebook(k)
    cbd = torch.from_numpy(cb).to("cuda:0")
    packed_np, mag_np = _state(7 * n + k, n, rows, sdt)
    buf, packed = _packed_dev(packed_np)
    mag = gu.to_dev(mag_np, sdt).reshape(rows, 1)
    for step in (1, 2, 3):
        g_np = syn.round_to(syn.row_scaled_normal(23, step, rows, period, -12, -8), dt).reshape(-1)
        out = torch.empty(rows, period, dtype=gu.TORCH[dt], device="cuda:0")
        automatic_gefen_muon_momentum_cuda(gu.to_dev(g_np, dt).reshape(rows, period), packed, mag, cbd, out,
                                           True, 0.95)
        idx = orc.unpack_nibbles(packed_np[: packed_np.size - SENTINEL], n)
        ref = np.empty(n, dtype=orc.NP_STORAGE[dt])
        rc = orc.lib().orc_muon_momentum(orc.DT[dt], orc.DT[sdt], orc._ptr(np.ascontiguousarray(g_np)),
                                         orc._ptr(idx), orc._ptr(mag_np), orc._ptr(ref), n, period,
                                         orc._ptr(cb), cb.size, 0.95, 0)
        assert rc == 0
        packed_np = _ref_packed(packed_np, n, idx)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(gu.to_np(buf), packed_np, err_msg="packed indices, step {}".format(step))
        np.testing.assert_array_equal(gu.to_np(mag).reshape(-1), mag_np, err_msg="magnitudes")
        np.testing.assert_array_equal(gu.to_np(out).reshape(-1), ref, err_msg="momentum")

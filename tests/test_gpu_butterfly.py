"""The wave butterflies of the step and GefenMuon kernels
(common.h: wave_group_max_u32 / wave_group_sum, lane exchanges by DPP,
ds_swizzle and ds_bpermute) give, in every lane and for every group width
1..64, the values of the ds_bpermute loops they replace (group_max_u32 /
group_sum), and both equal a host restatement of the xor butterfly: after the
steps off = width/2, ..., 1, lane i holds v[i] op v[i ^ off] of the previous
step, float32 sums rounded at every step."""

import ctypes
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "hip" / "libbutterfly_check.so"
N = 256 * 64


def _host_butterfly(v, width, op):
    out = np.empty_like(v)
    lanes = np.arange(64)
    for w0 in range(0, v.size, 64):
        x = v[w0:w0 + 64].copy()
        off = width >> 1
        while off:
            x = op(x, x[lanes ^ off])
            off >>= 1
        out[w0:w0 + 64] = x
    return out


def test_wave_butterflies_equal_the_loops_and_the_xor_butterfly():
    import torch

    assert torch.cuda.is_available()
    assert LIB.exists(), "build the test helper first (gefen_amd/build.py)"
    lib = ctypes.CDLL(str(LIB))
    lib.gefen_test_butterfly.restype = ctypes.c_int
    lib.gefen_test_butterfly.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    rng = np.random.default_rng(5)
    # float words of mixed signs and exponents (the sums round at every step);
    # the maxima see them as unsigned keys
    f = (rng.standard_normal(N) * np.exp2(rng.integers(-20, 20, N))).astype(np.float32)
    words = f.view(np.uint32)
    dev_in = torch.from_numpy(words.view(np.int32).copy()).cuda()
    dev_out = torch.empty(4 * 7 * N, dtype=torch.int32, device="cuda")
    assert lib.gefen_test_butterfly(dev_in.data_ptr(), dev_out.data_ptr(), N,
                                    torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    out = dev_out.cpu().numpy().view(np.uint32).reshape(4, 7, N)
    for l in range(7):
        width = 1 << l
        mx = _host_butterfly(words, width, np.maximum)
        sm = _host_butterfly(f, width, lambda a, b: (a + b).astype(np.float32)).view(np.uint32)
        np.testing.assert_array_equal(out[1, l], mx, err_msg="group_max_u32 width {}".format(width))
        np.testing.assert_array_equal(out[0, l], mx, err_msg="wave_group_max_u32 width {}".format(width))
        np.testing.assert_array_equal(out[3, l], sm, err_msg="group_sum width {}".format(width))
        np.testing.assert_array_equal(out[2, l], sm, err_msg="wave_group_sum width {}".format(width))
        print("width", width, "maxima and sums equal the xor butterfly in every lane", flush=True)

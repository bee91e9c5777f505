"""The period-one step kernel computes 1 / h as fma(fma(-h, r, 1), r, r) with
r = v_rcp_f32(h) (csrc/step.hip: root_stepsize) wherever root_ok holds,
2^-126 <= h < 2^126.  This checks, on the GPU, that this equals the IEEE
quotient for every float in that range (2.1e9 values, under a second)."""

import ctypes
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "hip" / "libreciprocal_check.so"


def test_rcp_with_one_correction_is_the_ieee_reciprocal_over_the_kernels_range():
    import torch

    assert torch.cuda.is_available()
    assert LIB.exists(), "build the test helper first (gefen_amd/build.py)"
    lib = ctypes.CDLL(str(LIB))
    lib.gefen_test_reciprocal.restype = ctypes.c_int
    lib.gefen_test_reciprocal.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
    out = np.zeros(2, dtype=np.uint64)
    first = np.zeros(8, dtype=np.uint32)
    print("reciprocal check over [2^-126, 2^126)", flush=True)
    assert lib.gefen_test_reciprocal(0x00800000, 0x7E800000, out.ctypes.data, first.ctypes.data) == 0
    assert out[1] == 0, "IEEE division disagrees with the float64 quotient"
    assert out[0] == 0, "reciprocal differs at h bits {}".format([hex(x) for x in first[: int(min(out[0], 8))]])

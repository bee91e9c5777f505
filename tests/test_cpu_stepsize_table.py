"""The period-one stepsize of a bf16 state through a 384-entry square-root table
(csrc/step_kernels.h: root_h, root_ok, root_table_ok, root_stepsize;
csrc/step.hip: k_build_root) equals the direct float32 expression of
gefen.py:1326-1327, h = sqrt(v) / sqrt(bc2) + eps, stepsize = (1 / bc1) / h,
for every bf16 bit pattern (NaN for NaN), at every setting the host lets a
launch read the table (root_table_ok), and h stays inside the reciprocal's
range [2^-126, 2^126) there.

numpy's float32 sqrt, division and addition are correctly rounded and ldexp is
exact on normal results, so this checks the identity the kernel relies on,
fl(fl(sqrt(M 2^E)) / c) = fl(fl(sqrt(M 2^par)) / c) 2^floor(E/2), exhaustively
over the bf16 inputs and for bias corrections and eps across their range.  The
kernel's reciprocal (v_rcp_f32 and one fma correction) is checked against the
IEEE quotient over every float in root_ok's range by a GPU test
(test_gpu_reciprocal.py); here the reciprocal is numpy's IEEE one."""

import numpy as np
import pytest

F32 = np.float32


def _direct(v, c, eps, inv_bc1):
    h = np.sqrt(v) / c + eps
    return (F32(1.0) / h) * inv_bc1


def _root_table(c):
    """k_build_root: (par, M) = (i >> 7, 128 + (i & 127)) for i < 256, (1, i - 256) above."""
    i = np.arange(384)
    par = np.where(i < 256, i >> 7, 1)
    m = np.where(i < 256, 128 + (i & 127), i - 256).astype(F32)
    root = np.ldexp(np.sqrt(m * np.where(par == 1, F32(2.0), F32(1.0)).astype(F32)) / c, np.int32(-67))
    assert root.dtype == F32
    return root


def _root_table_ok(c, eps):
    """root_table_ok: the settings at which a launch reads the table."""
    return bool(2.0 ** -60 <= c <= 2.0 ** 30 and 2.0 ** -126 <= eps <= 2.0 ** 100)


def _table(bits, c, eps, inv_bc1):
    """root_h, root_ok, root_stepsize (IEEE reciprocal), and stepsize_of where root_ok
    fails or the setting is outside root_table_ok; also h and where the table applied."""
    root = _root_table(c)
    i = np.where(bits < 0x80, bits + 256, bits & 0xFF)
    scaled = np.ldexp(root[i], (bits >> 8).astype(np.int32))
    assert scaled.dtype == F32
    h = scaled + eps
    ok = (bits < 0x7F80) & _root_table_ok(c, eps)
    table = (F32(1.0) / h) * inv_bc1
    v = (bits << 16).view(F32)
    return np.where(ok, table, _direct(v, c, eps, inv_bc1)), ok, h


@pytest.mark.parametrize("beta2,step,eps", [
    (0.999, 1, 1e-8), (0.999, 2, 1e-8), (0.999, 1000, 1e-8), (0.999, 10 ** 6, 1e-8),
    (0.99999, 1, 1e-12), (0.0, 1, 1e-8), (0.95, 7, 1e-3), (0.999, 3, 1e-30), (0.5, 1, 1e-6),
])
def test_square_root_table_matches_the_direct_expression(beta2, step, eps):
    bits = np.arange(0x10000, dtype=np.uint32)  # every bf16 bit pattern
    v = (bits << 16).view(F32)
    bc1 = 1.0 - 0.9 ** step
    bc2 = 1.0 - beta2 ** step
    c, eps_f, inv_bc1 = F32(np.sqrt(bc2)), F32(eps), F32(1.0 / bc1)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        want = _direct(v, c, eps_f, inv_bc1)
        got, ok, h = _table(bits, c, eps_f, inv_bc1)
    assert ok[bits < 0x7F80].all()  # every finite v >= 0 takes the table at these settings
    hb = h[bits < 0x7F80].view(np.uint32)
    assert ((hb >= 0x00800000) & (hb < 0x7E800000)).all()  # h in [2^-126, 2^126): the exact reciprocal
    nan = np.isnan(want)
    assert np.isfinite(want[bits < 0x7F80]).all()
    assert nan.sum() == (bits > 0x8000).sum() + 127  # every v < 0 but -0, and the 127 positive NaNs
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_values_outside_the_table_range_take_the_direct_path():
    bits = np.array([0x0000, 0x7F80, 0x8000, 0x8001, 0xFF80, 0x7FC0], dtype=np.uint32)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        got, ok, _ = _table(bits, F32(1.0), F32(0.0), F32(1.0))  # eps = 0: no table (h = 0 for v = 0)
    np.testing.assert_array_equal(ok, [False, False, False, False, False, False])
    assert got[0] == np.inf and got[1] == 0.0 and np.isinf(got[2]) and np.isnan(got[3:]).all()
    got, ok, _ = _table(bits, F32(1.0), F32(1e-8), F32(1.0))  # in bounds: only finite v >= 0
    np.testing.assert_array_equal(ok, [True, False, False, False, False, False])


@pytest.mark.parametrize("c,eps", [(2.0 ** -60, 2.0 ** -126), (2.0 ** 30, 2.0 ** -126), (2.0 ** -60, 2.0 ** 100),
                                   (2.0 ** 30, 2.0 ** 100)])
def test_table_bounds_keep_h_in_the_reciprocal_range(c, eps):
    """At the corners of root_table_ok the table still equals the direct
    expression and h stays in [2^-126, 2^126) for every finite v >= 0."""
    bits = np.arange(0x7F80, dtype=np.uint32)
    v = (bits << 16).view(F32)
    assert _root_table_ok(c, eps)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        want = _direct(v, F32(c), F32(eps), F32(1.0))
        got, ok, h = _table(bits, F32(c), F32(eps), F32(1.0))
    assert ok.all()
    hb = h.view(np.uint32)
    assert ((hb >= 0x00800000) & (hb < 0x7E800000)).all()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    assert not _root_table_ok(c * 2.0 if c > 1 else c / 2.0, eps)
    assert not _root_table_ok(c, eps * 2.0 if eps > 1 else eps / 2.0)


def test_table_index_covers_subnormals_zero_and_both_exponent_parities():
    bits = np.array([0x0000, 0x0001, 0x007F, 0x0080, 0x0100, 0x3F80, 0x4000, 0x7F7F], dtype=np.uint32)
    e8 = (bits >> 7).astype(np.int32)
    m = (bits & 0x7F).astype(np.int32) | np.where(e8 > 0, 0x80, 0)
    e = np.maximum(e8, 1) - 134
    # v = m * 2^e reproduces each value exactly; floor(e / 2) = (bits >> 8) - 67
    v = (bits << 16).view(F32).astype(np.float64)
    np.testing.assert_array_equal(np.ldexp(m.astype(np.float64), e), v)
    np.testing.assert_array_equal(e >> 1, (bits >> 8).astype(np.int32) - 67)
    assert set((e & 1).tolist()) == {0, 1}

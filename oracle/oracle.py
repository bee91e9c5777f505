"""Python face of the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module.  It wraps ``liboracle.so`` (built from
``gefen_oracle.c`` by ``oracle/Makefile``) and adds the pure-Python parts of
the reference algorithm that are integer logic or small host code:

* ``divisors`` (partitioning.py:13-30), ``largest_divisor_at_most``
  (gefen.py:72-82);
* ``finalize_period`` (partitioning.py:277-347) and ``find_period``
  (partitioning.py:119-167 + gefen.py:812-828);
* ``learn_codebook`` (gefen.py:305-419: histograms, fp32 accumulation, DP);
* Newton-Schulz (gefen_muon.py:16-51) one torch op at a time (``ns_normalize``,
  ``ns_gram``, ``ns_poly``, ``ns_update``: exact products, one bf16 rounding
  each), ``muon_apply`` (gefen_muon.py:325-329) and ``adjust_lr``
  (gefen_muon.py:54-67);
* ``GefenOracle`` / ``GefenMuonOracle``: whole optimizer steps on numpy arrays,
  following ``Gefen.step`` / ``GefenMuon.step`` on the CPU path.

Arrays of dtype 'bf16' and 'f16' are held as uint16 bit patterns.
"""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

HERE = Path(__file__).resolve().parent
DT = {"f32": 0, "f16": 1, "bf16": 2}
NP_STORAGE = {"f32": np.float32, "f16": np.uint16, "bf16": np.uint16}

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            raise RuntimeError("oracle/liboracle.so is not built (run make -C oracle)")
        L = ctypes.CDLL(str(path))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        D = ctypes.c_double
        I = ctypes.c_int
        L.orc_gefen_step.argtypes = [I, I, P, P, P, P, P, I64, I64, I64, P, I, D, D, D, D, D, D, D, I]
        L.orc_vmean_update.argtypes = [I, P, I, P, I64, I64, D]
        L.orc_nearest.argtypes = [P, I, P, P, I64]
        L.orc_histogram.argtypes = [I, P, I64, I64, I, P]
        L.orc_accumulate_counts.argtypes = [P, P, I]
        L.orc_exact_dp.argtypes = [P, I, I, I, P]
        L.orc_period_scores.argtypes = [I, P, I64, P, I, I, D, P]
        L.orc_muon_momentum.argtypes = [I, I, P, P, P, P, I64, I64, P, I, D, I]
        L.orc_f32_to_bf16.argtypes = [P, P, I64]
        L.orc_f32_to_f16.argtypes = [P, P, I64]
        L.orc_fma32.argtypes = [P, ctypes.c_float, P, P, I64]
        L.orc_gefen_update_given.argtypes = [I, I, P, P, P, P, P, I, P, I64, I64, P, I, D, D, D, D, D]
        L.orc_unpack_nibbles.argtypes = [P, I64, P]
        L.orc_pack_nibbles.argtypes = [P, I64, P]
        L.orc_lloyd_accumulate.argtypes = [I, P, I64, I64, P, I, P, P]
        L.orc_lloyd_mse.argtypes = [I, P, I64, I64, P, P, I, P]
        L.orc_block_variance.argtypes = [I, P, I64, I64, I, I, P]
        for name in ("orc_gefen_step", "orc_vmean_update", "orc_nearest", "orc_histogram",
                     "orc_accumulate_counts", "orc_exact_dp", "orc_period_scores",
                     "orc_muon_momentum", "orc_f32_to_bf16", "orc_f32_to_f16", "orc_fma32",
                     "orc_gefen_update_given", "orc_unpack_nibbles", "orc_pack_nibbles",
                     "orc_lloyd_accumulate", "orc_lloyd_mse", "orc_block_variance"):
            getattr(L, name).restype = ctypes.c_int
        _LIB = L
    return _LIB


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data


# ----------------------------------------------------------------- dtype helpers
def to_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return np.asarray(a, dtype=np.float32)
    if dtype == "bf16":
        return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)
    return np.asarray(a, dtype=np.uint16).view(np.float16).astype(np.float32)


def from_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "f32":
        return x.copy()
    out = np.empty(x.shape, dtype=np.uint16)
    fn = lib().orc_f32_to_bf16 if dtype == "bf16" else lib().orc_f32_to_f16
    fn(_ptr(x), _ptr(out), x.size)
    return out


def round_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    return to_f32(from_f32(x, dtype), dtype)


# ----------------------------------------------------------------- partition logic
def divisors(n: int, max_divisor: Optional[int] = None) -> List[int]:
    """partitioning.py:13-30 (n itself included for n > 1, ascending)."""
    if max_divisor is not None:
        max_divisor = int(max_divisor)
        if max_divisor < 1:
            raise ValueError("max_divisor must be positive, got {}.".format(max_divisor))
    small, large = [], []
    for i in range(1, int(n ** 0.5) + 1):
        if n % i == 0:
            if i != n and (max_divisor is None or i <= max_divisor):
                small.append(i)
            paired = n // i
            if i != paired and (max_divisor is None or paired <= max_divisor):
                large.append(paired)
    return small + large[::-1]


def largest_divisor_at_most(value: int, limit: int) -> int:
    """gefen.py:72-82."""
    if value <= 0 or limit <= 0:
        raise ValueError("expected positive value and limit")
    if value <= limit:
        return value
    return divisors(value, max_divisor=limit)[-1]


def finalize_period(periods_scores: Sequence[Tuple[int, float]], n: int) -> int:
    """partitioning.py:277-347: best interior strict local maximum with p > 8,
    capped to the smallest divisor of n in (1024, best] that divides best."""
    if len(periods_scores) == 0:
        raise ValueError("Expected at least one valid period candidate.")
    last_period = periods_scores[-1][0]
    cands = []
    for i in range(1, len(periods_scores) - 1):
        p, s = periods_scores[i]
        if p <= 8 or p == last_period:
            continue
        if s <= periods_scores[i - 1][1] or s <= periods_scores[i + 1][1]:
            continue
        cands.append((s, p))
    if not cands:
        best = 1
    else:
        best_score, best = max(cands)
        if not math.isfinite(best_score):
            raise ValueError("Expected finite best score, got {}.".format(best_score))
    if best > 1024:
        best = min(p for p in divisors(n) if 1024 < p <= best and best % p == 0)
    return best


def period_scores(g: np.ndarray, dtype: str, divs: Sequence[int], mode: int = 1,
                  eps: float = 1e-12) -> np.ndarray:
    g = np.ascontiguousarray(g.reshape(-1))
    d = np.ascontiguousarray(np.array(divs, dtype=np.int64))
    out = np.empty(len(divs), dtype=np.float64)
    rc = lib().orc_period_scores(DT[dtype], _ptr(g), g.size, _ptr(d), len(divs), mode, eps, _ptr(out))
    if rc == 4:
        raise ValueError("Expected values plus epsilon to be positive before log transform.")
    if rc:
        raise RuntimeError("orc_period_scores failed: {}".format(rc))
    return out


def find_period(g: np.ndarray, dtype: str, min_num_blocks: int = 4,
                max_period: Optional[int] = None) -> int:
    """Gefen._predict_period_from_grad_sq on the CPU backend (gefen.py:765-828)."""
    n = int(np.asarray(g).size)
    if n == 1:
        return 1
    divs = [p for p in divisors(n, max_divisor=max_period) if n // p >= min_num_blocks]
    if not divs:
        return 1
    sc = period_scores(g, dtype, divs, mode=1)
    return finalize_period(list(zip(divs, sc.tolist())), n)


# ----------------------------------------------------------------- histogram / DP
def histogram(g: np.ndarray, dtype: str, period: int, bins: int = 4096,
              counts: Optional[np.ndarray] = None) -> np.ndarray:
    g = np.ascontiguousarray(g.reshape(-1))
    if counts is None:
        counts = np.zeros(bins, dtype=np.int64)
    rc = lib().orc_histogram(DT[dtype], _ptr(g), g.size, period, bins, _ptr(counts))
    if rc:
        raise ValueError("orc_histogram: bad period {} for numel {}".format(period, g.size))
    return counts


def exact_dp(counts_f32: np.ndarray, k: int = 256, force: bool = True) -> np.ndarray:
    c = np.ascontiguousarray(counts_f32, dtype=np.float32)
    out = np.empty(k, dtype=np.float32)
    rc = lib().orc_exact_dp(_ptr(c), c.size, k, int(force), _ptr(out))
    if rc == 2:
        raise ValueError("Cannot run exact DP on an empty histogram.")
    if rc:
        raise RuntimeError("orc_exact_dp failed: {}".format(rc))
    return out


def learn_codebook(grad_periods: Sequence[Tuple[np.ndarray, str, int]], k: int = 256) -> Optional[np.ndarray]:
    """gefen.py:305-419: per-tensor 4096-bin histograms, fp32 sum in order, exact DP."""
    bins = k * 16
    acc = np.zeros(bins, dtype=np.float32)
    total = 0
    for g, dtype, period in grad_periods:
        cnt = histogram(g, dtype, period, bins)
        lib().orc_accumulate_counts(_ptr(acc), _ptr(cnt), bins)
        total += g.size
    if total == 0:
        return None
    return exact_dp(acc, k, True)


def nearest(cb: np.ndarray, x: np.ndarray) -> np.ndarray:
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().orc_nearest(_ptr(cb), cb.size, _ptr(x), _ptr(out), x.size)
    return out


# ----------------------------------------------------------------- Newton-Schulz
# Each torch op of gefen_muon.py:16-51 on bf16 tensors, as a bf16 rounding of
# the exact result: the products are formed in float64 (exact for these sizes up
# to the final rounding), rounded to float32 and then to bf16.  torch-CPU sums
# its bf16 products in float32, so its result differs from this one only where
# the float32 accumulation error reaches a bf16 rounding boundary: within one
# bf16 ulp plus 2(K+1)*2^-24 * sum|terms| of every element (checked against the
# reference's own products, tests/golden/ns_products.npz).

def _bf16_of(x64: np.ndarray) -> np.ndarray:
    return from_f32(np.asarray(x64, dtype=np.float64).astype(np.float32), "bf16")


def _f64_of(bits: np.ndarray) -> np.ndarray:
    return to_f32(bits, "bf16").astype(np.float64)


def ns_normalize(g_bits: np.ndarray, eps: float = 1e-7) -> np.ndarray:
    """gefen_muon.py:33-37: X = bf16(G), transposed when rows > cols, then
    X.div_(X.norm().clamp(min=eps)): the norm and the clamp are bf16 tensors,
    the quotient is rounded to bf16.  Returns X (bf16 bits, [min, max] shape)."""
    x = _f64_of(g_bits)
    if x.shape[0] > x.shape[1]:
        x = x.T
    nrm = float(round_f32(np.array([np.sqrt(np.sum(x * x))], dtype=np.float32), "bf16")[0])
    nrm = float(round_f32(np.array([max(nrm, np.float32(eps))], dtype=np.float32), "bf16")[0])
    return _bf16_of(x / nrm)


def ns_gram(x_bits: np.ndarray) -> np.ndarray:
    """gefen_muon.py:39: A = X @ X.T."""
    x = _f64_of(x_bits)
    return _bf16_of(x @ x.T)


def ns_poly(a_bits: np.ndarray, b: float, c: float) -> np.ndarray:
    """gefen_muon.py:40-46: B = torch.addmm(A, A, A, beta=b, alpha=c) = b A + c A A."""
    a = _f64_of(a_bits)
    return _bf16_of(b * a + c * (a @ a))


def ns_update(b_bits: np.ndarray, x_bits: np.ndarray, a: float) -> np.ndarray:
    """gefen_muon.py:47: X' = torch.addmm(X, B, X, beta=a) = a X + B X."""
    x = _f64_of(x_bits)
    return _bf16_of(a * x + _f64_of(b_bits) @ x)


def ns_term_bound(op: str, lhs_bits: np.ndarray, rhs_bits: Optional[np.ndarray] = None,
                  a: float = 0.0, b: float = 0.0, c: float = 0.0) -> np.ndarray:
    """2(K+1) * 2^-24 * sum|terms| of each element of a product above (float64):
    what two float32 accumulations of the same K products may differ by."""
    u = 2.0 ** -24
    if op == "gram":
        x = np.abs(_f64_of(lhs_bits))
        return 2 * (x.shape[1] + 1) * u * (x @ x.T)
    if op == "poly":
        m = np.abs(_f64_of(lhs_bits))
        return 2 * (m.shape[1] + 1) * u * (abs(b) * m + abs(c) * (m @ m))
    bm, x = np.abs(_f64_of(lhs_bits)), np.abs(_f64_of(rhs_bits))
    return 2 * (bm.shape[1] + 1) * u * (abs(a) * x + bm @ x)


def ulp_bf16(bits: np.ndarray) -> np.ndarray:
    """The bf16 ulp at each value (float64), 2^-133 for zero and subnormals."""
    v = np.abs(_f64_of(bits))
    e = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
    return np.ldexp(1.0, (e - 7).astype(np.int64))


def newton_schulz_bf16(u_f32: np.ndarray, coeffs=(3.4445, -4.7750, 2.0315), steps: int = 5,
                       eps: float = 1e-7) -> np.ndarray:
    """gefen_muon.py:16-51: ns_normalize, then `steps` times ns_gram, ns_poly,
    ns_update; the result is transposed back for a tall input.  float32 values
    of the bf16 result."""
    a, b, c = coeffs
    x = ns_normalize(from_f32(np.asarray(u_f32, dtype=np.float32), "bf16"), eps)
    for _ in range(steps):
        x = ns_update(ns_poly(ns_gram(x), b, c), x, a)
    if u_f32.shape[0] > u_f32.shape[1]:
        x = np.ascontiguousarray(x.T)
    return to_f32(x, "bf16")


def adjust_lr(lr: float, adjust_lr_fn: Optional[str], shape) -> float:
    """gefen_muon.py:54-67."""
    rows, cols = shape[:2]
    if adjust_lr_fn is None or adjust_lr_fn == "original":
        ratio = math.sqrt(max(1, rows / cols))
    elif adjust_lr_fn == "match_rms_adamw":
        ratio = 0.2 * math.sqrt(max(rows, cols))
    else:
        ratio = 1.0
    return lr * ratio


# ----------------------------------------------------------------- optimizer state
class TensorState:
    def __init__(self, numel: int, period: int, dtype: str, sdtype: str):
        self.period = period
        self.step = 0
        self.pod = largest_divisor_at_most(numel, 256) if period == 1 else None
        mrows = numel // (self.pod if period == 1 else period)
        self.m_codebook = np.zeros(numel, dtype=np.uint8)
        self.m_magnitude = np.zeros(mrows, dtype=NP_STORAGE[sdtype])
        self.vmean = np.zeros(numel // period, dtype=NP_STORAGE[sdtype])


class GefenOracle:
    """Gefen.step on the CPU path for a list of numpy parameters (gefen.py:1399-1420).

    params: list of dicts {"p": array (storage dtype, updated in place), "dtype": str,
    "shape": tuple, "lr", "beta1", "beta2", "eps", "weight_decay"} and optionally
    "sdtype" (state dtype, default "dtype").
    step(grads): one array or None per parameter.
    """

    def __init__(self, params: List[Dict], codebook: Optional[np.ndarray] = None, nthreads: int = 0):
        self.params = params
        self.codebook = None if codebook is None else np.ascontiguousarray(codebook, dtype=np.float32)
        self.periods: List[Optional[int]] = [None] * len(params)
        self.state: List[Optional[TensorState]] = [None] * len(params)
        self.nthreads = nthreads
        self.global_step = 0

    def _predict(self, i: int, g: np.ndarray) -> int:
        # gefen.py:908-913 / 1232-1257: reuse a stored period, numel 1 -> 1, else predict
        if self.periods[i] is None:
            self.periods[i] = 1 if g.size == 1 else find_period(g, self.params[i]["dtype"])
        return self.periods[i]

    def refresh_codebook(self, grads: Sequence[Optional[np.ndarray]]) -> None:
        """_maybe_refresh_gefen_codebook (gefen.py:969-980)."""
        if self.codebook is not None:
            return
        gp = []
        for i, g in enumerate(grads):
            if g is None or g.size == 0:
                continue
            gp.append((g, self.params[i]["dtype"], self._predict(i, g)))
        self.codebook = learn_codebook(gp)

    def _ensure_state(self, i: int, g: np.ndarray) -> TensorState:
        """State dtype = the gradient dtype, or "sdtype" of the parameter (float32
        under the reference's F_FP32 flag, gefen.py:53-69)."""
        if self.state[i] is None:
            dt = self.params[i]["dtype"]
            self.state[i] = TensorState(g.size, self._predict(i, g), dt, self.params[i].get("sdtype", dt))
        return self.state[i]

    def step(self, grads: Sequence[Optional[np.ndarray]]) -> None:
        self.refresh_codebook(grads)
        for i, (prm, g) in enumerate(zip(self.params, grads)):
            if g is None or g.size == 0:
                continue
            dt = prm["dtype"]
            st = self._ensure_state(i, g)
            st.step += 1
            b1, b2 = prm["beta1"], prm["beta2"]
            bc1 = 1 - b1 ** st.step
            bc2 = 1 - b2 ** st.step
            p = prm["p"]
            gg = np.ascontiguousarray(g.reshape(-1))
            rc = lib().orc_gefen_step(
                DT[dt], DT[prm.get("sdtype", dt)], _ptr(p), _ptr(gg), _ptr(st.m_codebook), _ptr(st.m_magnitude),
                _ptr(st.vmean), gg.size, st.period, st.pod or 0, _ptr(self.codebook),
                self.codebook.size, b1, b2, prm["lr"], prm["eps"], prm["weight_decay"],
                bc1, bc2, self.nthreads)
            if rc:
                raise RuntimeError("orc_gefen_step failed: {}".format(rc))
        self.global_step += 1


def muon_momentum(g: np.ndarray, dtype: str, st: TensorState, codebook: np.ndarray,
                  momentum: float, nesterov: bool) -> np.ndarray:
    gg = np.ascontiguousarray(g.reshape(-1))
    out = np.empty(gg.shape, dtype=NP_STORAGE[dtype])
    mblk = st.pod if st.period == 1 else st.period
    rc = lib().orc_muon_momentum(DT[dtype], DT[dtype], _ptr(gg), _ptr(st.m_codebook), _ptr(st.m_magnitude),
                                 _ptr(out), gg.size, mblk, _ptr(codebook), codebook.size,
                                 momentum, int(nesterov))
    if rc:
        raise RuntimeError("orc_muon_momentum failed: {}".format(rc))
    return out


def gefen_update_given(dtype: str, sdtype: str, p: np.ndarray, g: np.ndarray, idx: np.ndarray,
                       mag: np.ndarray, period: int, codebook: np.ndarray, beta1: float, lr: float,
                       vmean: Optional[np.ndarray] = None, vdtype: Optional[str] = None,
                       stepsize: Optional[np.ndarray] = None, bc1: float = 1.0, bc2: float = 1.0,
                       eps: float = 0.0) -> None:
    """The given-stepsize / given-vmean update (automatic_gefen_fused.py:10-249) on the
    CPU-path arithmetic; p, idx and mag are updated in place."""
    gg = np.ascontiguousarray(g.reshape(-1))
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    st = None if stepsize is None else np.ascontiguousarray(stepsize, dtype=np.float32)
    vm = None if vmean is None else np.ascontiguousarray(vmean)
    rc = lib().orc_gefen_update_given(
        DT[dtype], DT[sdtype], _ptr(p), _ptr(gg), _ptr(idx), _ptr(mag), None if vm is None else _ptr(vm),
        DT[vdtype or sdtype], None if st is None else _ptr(st), gg.size, period, _ptr(cb), cb.size,
        beta1, lr, bc1, bc2, eps)
    if rc:
        raise RuntimeError("orc_gefen_update_given failed: {}".format(rc))


def lloyd_accumulate(g: np.ndarray, dtype: str, period: int, codebook: np.ndarray):
    """Per-codeword sums (float64) and counts of the block-normalised values
    (lloyd_max_fused_kernel.cu:50-107 semantics, see gefen_oracle.c)."""
    g = np.ascontiguousarray(g.reshape(-1))
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    sums = np.zeros(cb.size, dtype=np.float64)
    counts = np.zeros(cb.size, dtype=np.int64)
    rc = lib().orc_lloyd_accumulate(DT[dtype], _ptr(g), g.size, period, _ptr(cb), cb.size, _ptr(sums), _ptr(counts))
    if rc:
        raise ValueError("orc_lloyd_accumulate: bad arguments")
    return sums, counts


def lloyd_mse(g: np.ndarray, dtype: str, period: int, old_codebook: np.ndarray, new_codebook: np.ndarray):
    """(normalised, original) squared-error sums in float64 (lloyd_max_fused_kernel.cu:109-195)."""
    g = np.ascontiguousarray(g.reshape(-1))
    oc = np.ascontiguousarray(old_codebook, dtype=np.float32)
    nc = np.ascontiguousarray(new_codebook, dtype=np.float32)
    out = np.zeros(2, dtype=np.float64)
    rc = lib().orc_lloyd_mse(DT[dtype], _ptr(g), g.size, period, _ptr(oc), _ptr(nc), oc.size, _ptr(out))
    if rc:
        raise ValueError("orc_lloyd_mse: bad arguments")
    return float(out[0]), float(out[1])


def block_variance(v: np.ndarray, dtype: str, period: int, input_is_squared: bool, cov: bool) -> np.ndarray:
    """[sqrt(mean block variance), 0, 0] or [sum CoV, count, negative count]
    (period_variance_kernel.cu:13-106 semantics in float64)."""
    v = np.ascontiguousarray(v.reshape(-1))
    out = np.zeros(3, dtype=np.float64)
    rc = lib().orc_block_variance(DT[dtype], _ptr(v), v.size, period, int(input_is_squared), int(cov), _ptr(out))
    if rc:
        raise ValueError("orc_block_variance: bad arguments")
    return out


def unpack_nibbles(packed: np.ndarray, n: int) -> np.ndarray:
    """Packed 4-bit indices -> one byte per element (automatic_gefen_fused_kernel.cu:14-27)."""
    out = np.empty(n, dtype=np.uint8)
    lib().orc_unpack_nibbles(_ptr(np.ascontiguousarray(packed)), n, _ptr(out))
    return out


def pack_nibbles(idx: np.ndarray, packed: np.ndarray) -> None:
    """Store idx & 0xF into the nibbles of `packed` in place (automatic_gefen_fused_kernel.cu:29-57)."""
    idx = np.ascontiguousarray(idx, dtype=np.uint8)
    assert packed.size == (idx.size + 1) // 2
    lib().orc_pack_nibbles(_ptr(idx), idx.size, _ptr(packed))


class GefenMuonOracle(GefenOracle):
    """GefenMuon.step on the CPU path (gefen_muon.py:216-350)."""

    def __init__(self, params: List[Dict], codebook: Optional[np.ndarray] = None, momentum=0.95,
                 nesterov=True, ns_coefficients=(3.4445, -4.7750, 2.0315), ns_steps=5, eps=1e-7,
                 adjust_lr_fn=None):
        super().__init__(params, codebook)
        self.momentum = momentum
        self.nesterov = nesterov
        self.ns = (ns_coefficients, ns_steps, eps)
        self.adjust_lr_fn = adjust_lr_fn
        # per tensor, of its last step: the Nesterov blend (Newton-Schulz input,
        # gradient dtype) and the Newton-Schulz result (bf16 bits)
        self.last_blend: List[Optional[np.ndarray]] = [None] * len(params)
        self.last_update: List[Optional[np.ndarray]] = [None] * len(params)

    def step(self, grads: Sequence[Optional[np.ndarray]]) -> None:
        self.refresh_codebook(grads)
        for i, (prm, g) in enumerate(zip(self.params, grads)):
            if g is None or g.size == 0:
                continue
            dt = prm["dtype"]
            st = self._ensure_state(i, g)
            upd = muon_momentum(g, dt, st, self.codebook, self.momentum, self.nesterov)
            st.step += 1
            shape = prm["shape"]
            u32 = to_f32(upd, dt).reshape(shape)
            coeffs, steps, eps = self.ns
            U = newton_schulz_bf16(u32, coeffs, steps, eps)
            self.last_blend[i] = upd
            self.last_update[i] = from_f32(U, "bf16")
            lr = prm["lr"]
            muon_apply(prm["p"], self.last_update[i], dt, shape, lr, prm["weight_decay"],
                       adjust_lr(lr, self.adjust_lr_fn, shape))
        self.global_step += 1


def muon_apply(p: np.ndarray, u_bits: np.ndarray, dtype: str, shape, lr: float, weight_decay: float,
               adjusted_lr: float) -> None:
    """gefen_muon.py:325-329 on the CPU path, p updated in place (storage dtype):
    p.mul_(1 - lr * wd) when wd > 0, then p.add_(U, alpha=-adjusted_lr) with the
    bf16 Newton-Schulz result U in the parameter's layout."""
    pf = to_f32(p, dtype).reshape(-1)
    if weight_decay > 0.0:
        pf = round_f32(pf * np.float32(1 - lr * weight_decay), dtype)
    Uf = np.ascontiguousarray(to_f32(u_bits, "bf16").reshape(-1))
    if dtype == "f32":
        # p.add_(U, alpha): promote(f32, bf16) = f32, one fused multiply-add
        newp = _fma32(Uf, np.float32(-adjusted_lr), pf)
    else:
        # reduced-float add_ with alpha rounded to the dtype.  The update of a
        # tall matrix (rows > cols) is a transposed view, which takes the
        # element-wise path where the product is rounded to the dtype too.
        al = round_f32(np.array([-adjusted_lr], dtype=np.float32), dtype)[0]
        prod = (Uf * al).astype(np.float32)
        if shape[0] > shape[1]:
            prod = round_f32(prod, dtype)
        newp = round_f32((pf + prod).astype(np.float32), dtype)
    p[...] = from_f32(newp, dtype).reshape(p.shape)


def _fma32(a: np.ndarray, b: np.float32, c: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    c = np.ascontiguousarray(c, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.float32)
    lib().orc_fma32(_ptr(a), ctypes.c_float(b), _ptr(c), _ptr(out), a.size)
    return out

"""Deterministic synthetic inputs for tests, golden fixtures and the benchmark.

Every value is produced from 64-bit integer arithmetic followed only by IEEE
operations that are correctly rounded on every platform (+, -, *, /, sqrt and
float64 -> float32 / bfloat16 round-to-nearest-even).  The same bytes therefore
come out of numpy on any host and out of the HIP twin of this generator
(``gefen_synth_*`` in ``csrc/synthetic.hip``), so CPU and GPU runs see
byte-identical gradients without copying them around.

Generator
---------
* ``splitmix64`` stream: word ``c`` of key ``k`` is ``splitmix64(k + c * GAMMA)``.
* ``normal``: Irwin-Hall sum of twelve 16-bit uniforms taken from three words,
  centred and scaled exactly: ``z = (2*S - 12*65535) / 131072`` (variance ~1,
  support [-6, 6]).
* ``scale``: a log-uniform-like dyadic factor ``(8 + m) / 8 * 2**e``.
* ``student_t3``: ``z0 / sqrt((z1^2 + z2^2 + z3^2) / 3)``.
"""

from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_KEYMUL = np.uint64(0xD1B54A32D192ED03)


def splitmix64(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = x + GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def make_key(seed: int, stream: int) -> np.uint64:
    """Key of one independent stream (a tensor, a step, a role)."""
    with np.errstate(over="ignore"):
        s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) * _KEYMUL + np.uint64(stream & 0xFFFFFFFFFFFFFFFF)
    return splitmix64(np.array([s], dtype=np.uint64))[0]


def words(key: np.uint64, start: int, count: int) -> np.ndarray:
    c = np.arange(start, start + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return splitmix64(np.uint64(key) + c * GAMMA)


_CHUNK = 1 << 20  # elements per pass: keeps the temporaries in cache


def normal(key: np.uint64, n: int, start: int = 0) -> np.ndarray:
    """n approximately N(0,1) float64 values (exact dyadic rationals)."""
    out = np.empty(n, dtype=np.float64)
    mask = np.uint64(0xFFFF)
    for c0 in range(0, n, _CHUNK):
        m = min(_CHUNK, n - c0)
        w = words(key, 3 * (start + c0), 3 * m).reshape(m, 3)
        s = np.zeros(m, dtype=np.int64)
        for j in range(3):
            col = w[:, j]
            for k in range(4):
                s += ((col >> np.uint64(16 * k)) & mask).astype(np.int64)
        out[c0:c0 + m] = (2 * s - 12 * 65535).astype(np.float64) / 131072.0
    return out


def dyadic_scale(key: np.uint64, n: int, e_lo: int, e_hi: int) -> np.ndarray:
    """n factors (8+m)/8 * 2**e, e uniform in [e_lo, e_hi], m uniform in [0, 7]."""
    w = words(key, 0, n)
    span = np.uint64(e_hi - e_lo + 1)
    e = (w % span).astype(np.int64) + e_lo
    m = ((w >> np.uint64(32)) % np.uint64(8)).astype(np.float64)
    return np.ldexp((8.0 + m) / 8.0, e)


def student_t3(key: np.uint64, n: int) -> np.ndarray:
    z = normal(key, 4 * n).reshape(n, 4)
    chi = (z[:, 1] * z[:, 1] + z[:, 2] * z[:, 2]) + z[:, 3] * z[:, 3]
    return z[:, 0] / np.sqrt(chi / 3.0)


def to_bf16_bits(x32: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x32, dtype=np.float32))
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    r = r.astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_to(x64: np.ndarray, dtype: str) -> np.ndarray:
    """float64 -> storage array of ``dtype`` ('f32', 'f16' or 'bf16' as uint16 bits)."""
    x32 = np.asarray(x64, dtype=np.float64).astype(np.float32)
    if dtype == "f32":
        return x32
    if dtype == "f16":
        # float64 -> float16 directly (single rounding), like torch's .half() of a double
        return np.asarray(x64, dtype=np.float64).astype(np.float16)
    if dtype == "bf16":
        return to_bf16_bits(x32)
    raise ValueError("unknown dtype {}".format(dtype))


def row_scaled_normal(seed: int, stream: int, rows: int, cols: int, e_lo: int, e_hi: int) -> np.ndarray:
    """N(0,1) values scaled by one dyadic log-uniform factor per row (float64)."""
    key = make_key(seed, stream)
    z = normal(key, rows * cols).reshape(rows, cols)
    s = dyadic_scale(make_key(seed, stream ^ 0x5CA1E), rows, e_lo, e_hi)
    return z * s[:, None]


def checksum(arr: np.ndarray) -> int:
    """Order-sensitive 64-bit checksum of the raw bytes."""
    b = np.ascontiguousarray(arr).view(np.uint8)
    pad = (-b.size) % 8
    if pad:
        b = np.concatenate([b, np.zeros(pad, dtype=np.uint8)])
    w = b.view(np.uint64)
    with np.errstate(over="ignore"):
        h = splitmix64(w ^ (np.arange(w.size, dtype=np.uint64) * GAMMA))
        return int(np.bitwise_xor.reduce(h)) if h.size else 0


# --------------------------------------------------------------------------- device twin
_SYNTH = None


def _synth_lib():
    global _SYNTH
    if _SYNTH is None:
        import ctypes
        import os
        from pathlib import Path

        path = Path(__file__).resolve().parent / "libgefen_synth.so"
        if not path.exists():
            raise ImportError("{} is missing; build it with `python -m gefen_amd.build`".format(path))
        lib = ctypes.CDLL(str(path), mode=os.RTLD_LOCAL)
        lib.gefen_synth_fill.restype = ctypes.c_int
        lib.gefen_synth_fill.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_double, ctypes.c_void_p]
        lib.gefen_synth_copy.restype = ctypes.c_int
        lib.gefen_synth_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        lib.gefen_last_error.restype = ctypes.c_char_p
        _SYNTH = lib
    return _SYNTH


KIND_ROW_SCALED, KIND_NORMAL, KIND_STUDENT_T3 = 0, 1, 2


def fill_device(t, seed: int, stream: int, kind: int, cols: int = 0, e_lo: int = 0, e_hi: int = 0,
                mult: float = 1.0) -> None:
    """Fill a contiguous HIP tensor with the values numpy would produce:
    kind 0 = row_scaled_normal(seed, stream, numel//cols, cols, e_lo, e_hi),
    kind 1 = normal(make_key(seed, stream), numel) * mult,
    kind 2 = student_t3(make_key(seed, stream), numel) * mult."""
    import torch

    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[t.dtype]
    if not t.is_contiguous():
        raise ValueError("fill_device needs a contiguous tensor")
    n = t.numel()
    cols = cols or max(n, 1)
    with torch.cuda.device(t.device):
        rc = _synth_lib().gefen_synth_fill(t.data_ptr(), code, n, cols, seed & 0xFFFFFFFFFFFFFFFF,
                                           stream & 0xFFFFFFFFFFFFFFFF, e_lo, e_hi, kind, float(mult),
                                           torch.cuda.current_stream(t.device).cuda_stream)
    if rc:
        raise RuntimeError(_synth_lib().gefen_last_error().decode())


def copy_device(src, dst) -> None:
    """dst <- src with a plain 16-byte-vector copy kernel (known traffic: the
    bytes of src read once and written once), for scaling profiler counters."""
    import torch

    n = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != n or not (src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("copy_device needs two contiguous tensors of the same size")
    with torch.cuda.device(src.device):
        rc = _synth_lib().gefen_synth_copy(src.data_ptr(), dst.data_ptr(), n,
                                           torch.cuda.current_stream(src.device).cuda_stream)
    if rc:
        raise RuntimeError(_synth_lib().gefen_last_error().decode())

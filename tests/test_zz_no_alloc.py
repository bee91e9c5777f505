"""gefen_step_tasks_noalloc (the step entry point that allocates nothing) against
gefen_step_tasks, through the C ABI: bit-identical parameters, indices,
magnitudes and vmean on two calls in a row, the second with smaller tensors;
the host-side rejection of a call whose stepsize tables exceed the scratch
buffer; the library's device-allocation count unchanged by it in a fresh
process; and two calls on two streams ordered by the scratch buffer's event."""

import numpy as np
import pytest
import torch

import gpu_util as gu
from golden_util import load
from gefen_amd import _lib
from gefen_amd import synthetic as syn

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _tensor_set(seed, shapes):
    """(dtype, numel, period, pod, p, g) per tensor: period-one tensors with bf16
    and f16 states (these take the stepsize tables), block rows, fp32."""
    out = []
    for i, (dt, n, period) in enumerate(shapes):
        p = syn.round_to(syn.normal(syn.make_key(seed, 10 + i), n) * 0.02, dt)
        g = syn.round_to(syn.row_scaled_normal(seed, 20 + i, 1, n, -14, -6), dt).reshape(-1)
        pod = 0
        if period == 1:
            pod = max(d for d in range(1, 257) if n % d == 0)
        out.append((dt, n, period, pod, p, g))
    return out


def _state(dt, n, period, pod):
    dev = "cuda:0"
    rows = n // (pod if period == 1 else period)
    return {"idx": torch.zeros(n, dtype=torch.uint8, device=dev),
            "mag": torch.zeros(rows, dtype=DT[dt], device=dev),
            "vmean": torch.zeros(n // period, dtype=DT[dt], device=dev)}


def _tasks(specs, ps, gs, states, step, eps_of=lambda i: 1e-8):
    t = np.zeros(len(specs), dtype=_lib.STEP_TASK)
    for i, ((dt, n, period, pod, _, _), p, g, st) in enumerate(zip(specs, ps, gs, states)):
        t[i]["p"], t[i]["grad"] = p.data_ptr(), g.data_ptr()
        t[i]["m_codebook"], t[i]["m_magnitude"], t[i]["vmean"] = (st["idx"].data_ptr(), st["mag"].data_ptr(),
                                                                   st["vmean"].data_ptr())
        t[i]["numel"], t[i]["period"], t[i]["period_one_divisor"] = n, period, pod
        t[i]["param_dtype"] = t[i]["state_dtype"] = gu.CODE[dt]
        t[i]["beta1"], t[i]["beta2"], t[i]["lr"], t[i]["eps"] = 0.9, 0.999, 1e-3, eps_of(i)
        t[i]["weight_decay"] = 0.01 if i % 2 else 0.0
        t[i]["bias_correction_1"], t[i]["bias_correction_2"] = 1 - 0.9 ** step, 1 - 0.999 ** step
    return t


def _tables(lib):
    data, _ = load("exact_dp")
    cb = torch.from_numpy(data["hist_k256_forced/codebook"]).to("cuda:0")
    tables = torch.empty(int(lib.gefen_codebook_tables_size()), dtype=torch.uint8, device="cuda:0")
    _lib.check(lib.gefen_prepare_codebook(cb.data_ptr(), cb.numel(), tables.data_ptr(), gu.stream()))
    return tables


def _run(entry, specs, steps):
    lib = _lib.load()
    tables = _tables(lib)
    ps = [gu.to_dev(s[4], s[0]) for s in specs]
    gs = [gu.to_dev(s[5], s[0]) for s in specs]
    states = [_state(*s[:4]) for s in specs]
    for step in range(1, steps + 1):
        t = _tasks(specs, ps, gs, states, step)
        _lib.check(getattr(lib, entry)(t.ctypes.data, len(specs), tables.data_ptr(), gu.stream()), entry)
    torch.cuda.synchronize()
    return [gu.to_np(p) for p in ps], [{k: gu.to_np(v) for k, v in st.items()} for st in states]


def test_noalloc_step_equals_step_tasks_on_two_calls():
    big = [("bf16", 1 << 20, 1), ("f16", 3 * 4096, 1), ("bf16", 96 * 2048, 2048), ("f32", 48 * 768, 768),
           ("f16", 1000, 1), ("bf16", 5 * 300, 1)]
    small = [("bf16", 4096, 1), ("f16", 512, 1), ("bf16", 2 * 2048, 2048)]
    for label, shapes, steps in (("first call", big, 3), ("second, smaller call", small, 2)):
        print("noalloc", label, flush=True)
        specs = _tensor_set(11 if label == "first call" else 12, shapes)
        ref_p, ref_s = _run("gefen_step_tasks", specs, steps)
        got_p, got_s = _run("gefen_step_tasks_noalloc", specs, steps)
        for i in range(len(specs)):
            np.testing.assert_array_equal(got_p[i], ref_p[i], err_msg="{} p{}".format(label, i))
            for k in ("idx", "mag", "vmean"):
                np.testing.assert_array_equal(got_s[i][k], ref_s[i][k], err_msg="{} {}{}".format(label, k, i))


def test_noalloc_rejects_tables_beyond_its_scratch_buffer():
    """Nine period-one f16 tensors with nine eps values need nine 128 KiB stepsize
    tables, more than the 1 MiB scratch buffer: rejected on the host (nothing is
    launched), while gefen_step_tasks takes the same call."""
    lib = _lib.load()
    tables = _tables(lib)
    specs = _tensor_set(13, [("f16", 512, 1)] * 9)
    ps = [gu.to_dev(s[4], s[0]) for s in specs]
    gs = [gu.to_dev(s[5], s[0]) for s in specs]
    states = [_state(*s[:4]) for s in specs]
    t = _tasks(specs, ps, gs, states, 1, eps_of=lambda i: 1e-8 * (i + 1))
    rc = lib.gefen_step_tasks_noalloc(t.ctypes.data, len(specs), tables.data_ptr(), gu.stream())
    assert rc == _lib.GEFEN_EINVAL
    assert b"scratch buffer" in lib.gefen_last_error()
    _lib.check(lib.gefen_step_tasks(t.ctypes.data, len(specs), tables.data_ptr(), gu.stream()))
    torch.cuda.synchronize()


_CHILD = r'''
import sys
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
import torch
import test_zz_no_alloc as t
from gefen_amd import _lib

lib = _lib.load()
tables = t._tables(lib)
before = lib.gefen_device_allocations()
specs = t._tensor_set(14, [("bf16", 1 << 16, 1), ("f16", 4096, 1), ("bf16", 8 * 2048, 2048)])
ps = [t.gu.to_dev(s[4], s[0]) for s in specs]
gs = [t.gu.to_dev(s[5], s[0]) for s in specs]
states = [t._state(*s[:4]) for s in specs]
for step in (1, 2):
    tk = t._tasks(specs, ps, gs, states, step)
    _lib.check(lib.gefen_step_tasks_noalloc(tk.ctypes.data, len(specs), tables.data_ptr(), t.gu.stream()))
torch.cuda.synchronize()
after_noalloc = lib.gefen_device_allocations()
tk = t._tasks(specs, ps, gs, states, 3)
_lib.check(lib.gefen_step_tasks(tk.ctypes.data, len(specs), tables.data_ptr(), t.gu.stream()))
torch.cuda.synchronize()
print("allocations", before, after_noalloc, lib.gefen_device_allocations(), flush=True)
'''


def test_noalloc_allocates_nothing():
    """In a fresh process (no stepsize-table pool yet), two no-allocation calls with
    period-one bf16 and f16 states leave the library's device-allocation count
    unchanged, while gefen_step_tasks on the same tensors allocates its pool: the
    count sees the allocation the no-allocation entry point avoids."""
    import subprocess
    import sys
    from pathlib import Path

    repo = str(Path(__file__).resolve().parent.parent)
    r = subprocess.run([sys.executable, "-c", _CHILD, repo], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    line = [ln for ln in r.stdout.splitlines() if ln.startswith("allocations")][-1]
    before, after_noalloc, after_step = map(int, line.split()[1:])
    print(line, flush=True)
    assert after_noalloc == before
    assert after_step > after_noalloc


def test_noalloc_calls_on_two_streams_are_ordered():
    """Two no-allocation calls on two streams, back to back, with different eps (so
    the second call rewrites the stepsize tables in the shared scratch buffer while
    the first call's launches may still read them): the second waits for the first,
    and each equals gefen_step_tasks bit for bit."""
    lib = _lib.load()
    tables = _tables(lib)
    shapes = [("bf16", 1 << 23, 1), ("f16", 1 << 20, 1)]
    runs = {}
    for entry in ("gefen_step_tasks", "gefen_step_tasks_noalloc"):
        sets = []
        for k, seed in enumerate((15, 16)):
            specs = _tensor_set(seed, shapes)
            ps = [gu.to_dev(s[4], s[0]) for s in specs]
            gs = [gu.to_dev(s[5], s[0]) for s in specs]
            states = [_state(*s[:4]) for s in specs]
            sets.append((specs, ps, gs, states, _tasks(specs, ps, gs, states, 1, eps_of=lambda i, k=k: 1e-8 * (k + 1))))
        torch.cuda.synchronize()
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        for (specs, _, _, _, tk), s in zip(sets, streams):
            _lib.check(getattr(lib, entry)(tk.ctypes.data, len(specs), tables.data_ptr(), s.cuda_stream), entry)
        torch.cuda.synchronize()
        runs[entry] = [([gu.to_np(p) for p in ps], [{k: gu.to_np(v) for k, v in st.items()} for st in states])
                       for (_, ps, _, states, _) in sets]
    for k in range(2):
        for i in range(len(shapes)):
            ref_p, ref_s = runs["gefen_step_tasks"][k]
            got_p, got_s = runs["gefen_step_tasks_noalloc"][k]
            np.testing.assert_array_equal(got_p[i], ref_p[i], err_msg="call {} p{}".format(k, i))
            for key in ("idx", "mag", "vmean"):
                np.testing.assert_array_equal(got_s[i][key], ref_s[i][key], err_msg="call {} {}{}".format(k, key, i))

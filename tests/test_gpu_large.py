"""Full sizes, through block locality.  Every output of the step depends only on
its own magnitude block, the codebook and scalars, so the last blocks of a tensor
of more than 2^31 elements, stepped inside it, must equal the same blocks stepped
as a tensor of their own -- bit for bit, through two steps -- and every tensor of
the full 8B-shaped step must equal itself stepped alone.  The first-step
histogram of such a tensor is the sum of its parts' histograms."""

import numpy as np
import pytest
import torch

import gpu_util as gu
from golden_util import load
from gefen_amd import _lib
from gefen_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _tables():
    data, _ = load("exact_dp")
    cb = torch.from_numpy(np.ascontiguousarray(data["hist_k256_forced/codebook"], dtype=np.float32)).to("cuda:0")
    lib = _lib.load()
    t = torch.empty(int(lib.gefen_codebook_tables_size()), dtype=torch.uint8, device="cuda:0")
    _lib.check(lib.gefen_prepare_codebook(cb.data_ptr(), cb.numel(), t.data_ptr(), gu.stream()))
    return t


@pytest.mark.parametrize("period", [2048, 1])
def test_blocks_past_2_31_elements_match_a_tensor_of_their_own(period):
    print("large tensor, period", period, flush=True)
    n = 2048 * (2 ** 20 + 64)  # 2^31 + 131072 elements
    tail = 2048 * 64
    assert n > 2 ** 31
    dev = "cuda:0"
    pod = 256 if period == 1 else 0
    blk = pod if period == 1 else period
    p = torch.empty(n, dtype=torch.bfloat16, device=dev)
    g = torch.empty(n, dtype=torch.bfloat16, device=dev)
    syn.fill_device(p, 31, 1, syn.KIND_NORMAL, mult=0.02)
    syn.fill_device(g, 31, 2, syn.KIND_ROW_SCALED, cols=2048, e_lo=-17, e_hi=-7)
    idx = torch.zeros(n, dtype=torch.uint8, device=dev)
    mag = torch.zeros(n // blk, dtype=torch.bfloat16, device=dev)
    vm = torch.zeros(n // period, dtype=torch.bfloat16, device=dev)
    # the last `tail` elements as a tensor of their own
    ps, gs = p[-tail:].clone(), g[-tail:].clone()
    idxs = torch.zeros(tail, dtype=torch.uint8, device=dev)
    mags = torch.zeros(tail // blk, dtype=torch.bfloat16, device=dev)
    vms = torch.zeros(tail // period, dtype=torch.bfloat16, device=dev)
    tables = _tables()
    lib = _lib.load()
    tasks = np.zeros(2, dtype=_lib.STEP_TASK)
    for t, (pp, gg, ii, mm, vv, nn) in zip(tasks, [(p, g, idx, mag, vm, n), (ps, gs, idxs, mags, vms, tail)]):
        t["p"], t["grad"], t["m_codebook"] = pp.data_ptr(), gg.data_ptr(), ii.data_ptr()
        t["m_magnitude"], t["vmean"] = mm.data_ptr(), vv.data_ptr()
        t["numel"], t["period"], t["period_one_divisor"] = nn, period, pod
        t["param_dtype"] = t["state_dtype"] = gu.CODE["bf16"]
        t["beta1"], t["beta2"], t["lr"], t["eps"], t["weight_decay"] = 0.9, 0.999, 1e-3, 1e-8, 0.01
    for step in (1, 2):
        tasks["bias_correction_1"] = 1 - 0.9 ** step
        tasks["bias_correction_2"] = 1 - 0.999 ** step
        _lib.check(lib.gefen_step_tasks(tasks.ctypes.data, 2, tables.data_ptr(), gu.stream()))
    torch.cuda.synchronize()
    assert torch.equal(p[-tail:].view(torch.int16), ps.view(torch.int16))
    assert torch.equal(idx[-tail:], idxs)
    assert torch.equal(mag[-(tail // blk):].view(torch.int16), mags.view(torch.int16))
    assert torch.equal(vm[-(tail // period):].view(torch.int16), vms.view(torch.int16))
    assert int(idxs.to(torch.int32).sum()) > 0  # the step did quantise something


def test_full_8b_step_equals_its_tensors_stepped_alone():
    """The Llama-3-8B-shaped step of bench.py at full size (291 tensors, 8.03e9
    bf16 elements, the optimizer's own periods and learned codebook) through the
    optimizer's batched, multi-launch, two-stream path: sampled tensors (the
    embedding, block-row and period-one projections, norms) must equal the same
    tensors stepped one at a time from a snapshot -- bit for bit."""
    import bench
    from gefen_amd.gefen import Gefen

    dev = torch.device("cuda:0")
    params = bench.build_problem(bench.CONFIGS["llama8b"], dev)
    print("8B problem built", flush=True)
    opt = Gefen(params)
    opt.step()  # periods, codebook, states
    torch.cuda.synchronize()
    sample = [0, 1, 2, 3, 4, 5, 6, 7, 8, 150, len(params) - 2, len(params) - 1]
    snap = []
    for i in sample:
        _, p = params[i]
        st = opt.state[p]
        snap.append({"p": p.detach().clone(), "idx": st["m_codebook"].clone(), "mag": st["m_magnitude"].clone(),
                     "v": st["vmean"].clone(), "period": st["automatic_period"],
                     "pod": st.get("period_one_divisor", 0), "step": st["step"]})
    opt.step()  # every tensor in one call of the step kernels
    tables = opt._codebook_tables()
    lib = _lib.load()
    kinds = set()
    for i, s in zip(sample, snap):
        _, p = params[i]
        st = opt.state[p]
        g = opt.param_groups[i]
        step = s["step"] + 1
        t = np.zeros(1, dtype=_lib.STEP_TASK)
        t["p"], t["grad"], t["m_codebook"] = s["p"].data_ptr(), p.grad.data_ptr(), s["idx"].data_ptr()
        t["m_magnitude"], t["vmean"] = s["mag"].data_ptr(), s["v"].data_ptr()
        t["numel"], t["period"] = p.numel(), s["period"]
        t["period_one_divisor"] = s["pod"] if s["period"] == 1 else 0
        t["param_dtype"] = t["state_dtype"] = gu.CODE["bf16"]
        t["beta1"], t["beta2"], t["lr"], t["eps"], t["weight_decay"] = (g["beta1"], g["beta2"], g["lr"], g["eps"],
                                                                         g["weight_decay"])
        t["bias_correction_1"] = 1 - g["beta1"] ** step
        t["bias_correction_2"] = 1 - g["beta2"] ** step
        _lib.check(lib.gefen_step_tasks(t.ctypes.data, 1, tables.data_ptr(), gu.stream()))
        torch.cuda.synchronize()
        print("tensor", i, params[i][0], p.numel(), "period", s["period"], flush=True)
        kinds.add("one" if s["period"] == 1 else ("small" if p.numel() < 2 ** 20 else "rows"))
        assert torch.equal(p.detach().view(torch.int16), s["p"].view(torch.int16))
        assert torch.equal(st["m_codebook"], s["idx"])
        assert torch.equal(st["m_magnitude"].view(torch.int16), s["mag"].view(torch.int16))
        assert torch.equal(st["vmean"].view(torch.int16), s["v"].view(torch.int16))
    assert kinds == {"one", "small", "rows"}, kinds


def test_full_qwen3_muon_momentum_equals_its_tensors_stepped_alone():
    """GefenMuon at bench.py's full Qwen3-1.7B shapes (196 matrices, cached plan,
    stacked Newton-Schulz): the quantised momentum state of sampled matrices after
    a step equals gefen_muon_tasks run on each of them alone from a snapshot, bit
    for bit."""
    import bench
    from gefen_amd.gefen import _DTYPE_CODE
    from gefen_amd.gefen_muon import GefenMuon

    dev = torch.device("cuda:0")
    params = bench.build_problem(bench.CONFIGS["muon"], dev)
    print("Qwen3 problem built", flush=True)
    opt = GefenMuon(params)
    opt.step()
    opt.step()  # the second step builds the cached plan
    torch.cuda.synchronize()
    sample = [0, 1, 2, 3, 4, 5, 6, len(params) - 1]
    snap = []
    for i in sample:
        _, p = params[i]
        st = opt.state[p]
        snap.append({"idx": st["m_codebook"].clone(), "mag": st["m_magnitude"].clone(),
                     "period": st["automatic_period"]})
    opt.step()  # through the cached plan
    tables = opt._codebook_tables()
    lib = _lib.load()
    periods = set()
    for i, s in zip(sample, snap):
        _, p = params[i]
        st = opt.state[p]
        g = opt.param_groups[i]
        flat = p.grad.reshape(-1)
        out = torch.empty_like(flat)
        t = np.zeros(1, dtype=_lib.MUON_TASK)
        t["grad"], t["m_codebook"], t["m_magnitude"], t["out"] = (flat.data_ptr(), s["idx"].data_ptr(),
                                                                   s["mag"].data_ptr(), out.data_ptr())
        t["numel"] = flat.numel()
        t["block"] = opt._period_one_divisor_from_state(st, flat.numel()) if s["period"] == 1 else s["period"]
        t["grad_dtype"], t["state_dtype"] = _DTYPE_CODE[flat.dtype], _DTYPE_CODE[st["m_magnitude"].dtype]
        t["momentum"], t["nesterov"] = g["momentum"], 1 if g["nesterov"] else 0
        _lib.check(lib.gefen_muon_tasks(t.ctypes.data, 1, tables.data_ptr(), gu.stream()))
        torch.cuda.synchronize()
        print("matrix", i, params[i][0], tuple(p.shape), "period", s["period"], flush=True)
        periods.add(s["period"] == 1)
        assert torch.equal(st["m_codebook"], s["idx"])
        assert torch.equal(st["m_magnitude"].view(torch.int16), s["mag"].view(torch.int16))
    assert periods == {True, False}, periods


def test_histogram_past_2_31_elements_is_the_sum_of_its_parts():
    """The first-step histogram normalises each row by its own absmax, so the
    counts of a tensor of more than 2^31 elements equal the counts of its first
    2^31 elements plus those of the rest, each taken as a tensor of its own."""
    print("large histogram", flush=True)
    n = 2048 * (2 ** 20 + 64)
    head = 2 ** 31
    g = torch.empty(n, dtype=torch.bfloat16, device="cuda:0")
    syn.fill_device(g, 41, 3, syn.KIND_ROW_SCALED, cols=2048, e_lo=-17, e_hi=-7)
    lib = _lib.load()
    counts = [torch.zeros(4096, dtype=torch.int64, device="cuda:0") for _ in range(3)]
    for c, (start, stop) in zip(counts, [(0, n), (0, head), (head, n)]):
        part = g[start:stop]
        _lib.check(lib.gefen_exact_histogram(part.data_ptr(), gu.CODE["bf16"], stop - start, 2048, c.data_ptr(),
                                             4096, gu.stream()))
    torch.cuda.synchronize()
    assert int(counts[0].sum()) == n
    assert torch.equal(counts[0], counts[1] + counts[2])

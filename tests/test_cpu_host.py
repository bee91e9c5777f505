"""CPU-side checks: the C-ABI library loads and exports every declared symbol,
the host logic of the drop-in (period selection, divisors, param groups,
argument validation) follows the reference."""

import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as orc

REPO = Path(__file__).resolve().parent.parent


def _declared(header):
    text = (REPO / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(gefen_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    from gefen_amd import _lib

    lib = _lib.load()
    names = _declared("gefen_hip.h")
    assert len(names) >= 20, names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)
    assert lib.gefen_struct_size(0) == _lib.STEP_TASK.itemsize
    assert lib.gefen_struct_size(1) == _lib.MUON_TASK.itemsize
    assert lib.gefen_struct_size(2) == _lib.MUON_APPLY_TASK.itemsize
    assert lib.gefen_abi_version() == 1


def test_entry_points_reject_invalid_arguments_without_a_device():
    from gefen_amd import _lib

    lib = _lib.load()
    with pytest.raises(ValueError, match="at most 256"):
        _lib.check(lib.gefen_prepare_codebook(1, 300, 1, None))
    with pytest.raises(ValueError, match="bins"):
        _lib.check(lib.gefen_exact_histogram(1, 0, 16, 4, 1, 5000, None))
    with pytest.raises(ValueError, match="divisible"):
        _lib.check(lib.gefen_exact_histogram(1, 0, 17, 4, 1, 4096, None))
    with pytest.raises(ValueError, match="vmean dtype"):
        _lib.check(lib.gefen_automatic_fused_update_from_vmean(1, 1, 0, 1, 1, 0, 1, 1, 1, 256, 1, 4, 4, 0.9, 1e-3,
                                                               0.5, 0.5, 1e-8, None))
    with pytest.raises(ValueError, match="beta2"):
        _lib.check(lib.gefen_automatic_vmean_update(1, 0, 1, 0, 4, 4, 1.5, None))
    assert lib.gefen_exact_dp_workspace_size(4096, 256) > 256 * 4097 * 12


def test_divisors_and_period_selection_match_the_oracle_restatement():
    from gefen_amd import partitioning as part

    for n in [1, 2, 7, 12, 48, 1031 * 3, 2 ** 10 * 3 * 167, 50257 * 768]:
        assert part.divisors(n) == orc.divisors(n)
        assert part.divisors(n, max_divisor=100) == orc.divisors(n, max_divisor=100)
    rng = np.random.default_rng(0)
    for _ in range(200):
        n = int(rng.choice([4096, 6144, 98304, 2304 * 12, 3072 * 40]))
        divs = part.candidate_divisors(n)
        scores = rng.random(len(divs)).tolist()
        pairs = list(zip(divs, scores))
        assert part._finalize_period_results(pairs, False, n, 0.25) == orc.finalize_period(pairs, n)


def test_period_selection_hand_built_cases():
    """partitioning.py:277-347 on score lists whose answer is known by hand."""
    from gefen_amd.partitioning import _finalize_period_results as fin

    n = 96 * 768
    divs = [p for p in orc.divisors(n) if n // p >= 4]
    flat = [(p, 1.0) for p in divs]
    assert fin(flat, False, n, 0.25) == 1                      # no strict local maximum
    peak = [(p, 2.0 if p == 768 else 1.0) for p in divs]
    assert fin(peak, False, n, 0.25) == 768
    small = [(p, 2.0 if p == 8 else 1.0) for p in divs]
    assert fin(small, False, n, 0.25) == 1                     # p <= 8 never wins
    two = [(p, 3.0 if p == 768 else 2.0 if p == 96 else 1.0) for p in divs]
    assert fin(two, False, n, 0.25) == 768                     # highest score wins
    # caps: best 2304 -> 1152, 3072 -> 1536, 4096 -> 2048
    for n, best, capped in [(2304 * 12, 2304, 1152), (3072 * 40, 3072, 1536), (4096 * 8, 4096, 2048)]:
        d = [p for p in orc.divisors(n) if n // p >= 4]
        s = [(p, 5.0 if p == best else 1.0) for p in d]
        assert fin(s, False, n, 0.25) == capped
    last = [(p, 2.0 if p == divs[-1] else 1.0) for p in divs]
    assert fin(last, False, 96 * 768, 0.25) == 1               # the last divisor is excluded


def test_param_group_flattening_matches_reference():
    from gefen_amd.gefen import Gefen

    a = torch.zeros(4, 3, requires_grad=True)
    b = torch.zeros(5, requires_grad=True)
    c = torch.zeros(2, requires_grad=False)
    d = torch.zeros(6, requires_grad=True)
    opt = Gefen([{"params": [("Alpha", a), b, c], "lr": 2e-3, "betas": (0.8, 0.95)}, ("Beta", d)], weight_decay=0.1)
    names = [g["name"] for g in opt.param_groups]
    assert names == ["alpha", "group_0_param_1", "beta"]
    g0 = opt.param_groups[0]
    assert (g0["lr"], g0["beta1"], g0["beta2"], g0["eps"], g0["weight_decay"]) == (2e-3, 0.8, 0.95, 1e-8, 0.1)
    assert set(g0.keys()) == {"name", "params", "lr", "beta1", "beta2", "eps", "weight_decay"}
    with pytest.raises(ValueError, match="Invalid beta parameter at index 0"):
        Gefen([a], betas=(1.0, 0.9))
    with pytest.raises(ValueError, match="missing the 'params' key"):
        Gefen([{"lr": 1.0}])
    with pytest.raises(TypeError, match="can only optimize Tensors"):
        Gefen([{"params": [1.0]}])


def test_muon_constructor_checks():
    from gefen_amd.gefen_muon import GefenMuon

    w = torch.zeros(4, 4, requires_grad=True)
    opt = GefenMuon([w])
    g = opt.param_groups[0]
    assert g["beta1"] == 0.95 and g["beta2"] == 0.0 and g["eps"] == 1e-7 and g["weight_decay"] == 0.1
    assert g["nesterov"] is True and g["ns_steps"] == 5
    with pytest.raises(ValueError, match="only supports 2D"):
        GefenMuon([torch.zeros(3, requires_grad=True)])
    with pytest.raises(ValueError, match="not supported"):
        GefenMuon([w], adjust_lr_fn="bogus")


def test_step_on_cpu_tensors_fails_loudly():
    from gefen_amd.gefen import Gefen

    w = torch.zeros(8, 8, requires_grad=True)
    w.grad = torch.ones(8, 8)
    opt = Gefen([w])
    with pytest.raises((RuntimeError, ValueError), match="HIP"):
        opt.step()

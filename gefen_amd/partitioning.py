"""Automatic period detection (reference: partitioning.py).

Scores are computed on the device by libgefen_hip.so (all divisors of one
gradient per call); the selection among divisors is host integer logic that
follows partitioning.py:277-347 step by step.
"""

from __future__ import annotations

import functools
import math
from typing import List, Optional, Sequence, Tuple

import torch

DMNB = 4


class ZeroBlockMeanError(ValueError):
    pass


@functools.lru_cache(maxsize=4096)
def _all_divisors(n: int) -> Tuple[int, ...]:
    """Every divisor of n > 0, ascending, from its prime factorisation (trial
    division stops at the square root of what is left, so the highly composite
    sizes of model tensors factor in a few steps)."""
    factors = []
    m, d = n, 2
    while d * d <= m:
        if m % d == 0:
            e = 0
            while m % d == 0:
                m //= d
                e += 1
            factors.append((d, e))
        d += 1 if d == 2 else 2
    if m > 1:
        factors.append((m, 1))
    divs = [1]
    for prime, e in factors:
        divs = [x * prime ** k for x in divs for k in range(e + 1)]
    return tuple(sorted(divs))


def divisors(n, max_divisor=None) -> List[int]:
    """Divisors of n in ascending order, n itself included for n > 1
    (partitioning.py:13-30); only those <= max_divisor when it is given."""
    if max_divisor is not None:
        max_divisor = int(max_divisor)
        if max_divisor < 1:
            raise ValueError("max_divisor must be positive, got {}.".format(max_divisor))
    n = int(n)
    if n <= 1:
        return []
    found = _all_divisors(n)
    if max_divisor is None:
        return list(found)
    return [d for d in found if d <= max_divisor]


def candidate_divisors(n: int, max_period: Optional[int] = None, min_num_blocks: int = DMNB) -> List[int]:
    """Divisors scored for a tensor of n elements (partitioning.py:147-151)."""
    return [p for p in divisors(n, max_divisor=max_period) if n // p >= min_num_blocks]


def _finalize_period_results(list_periods_and_scores: Sequence[Tuple[int, float]], print_results: bool,
                             flattened_length: int, threshold) -> int:
    """partitioning.py:277-347: the highest-scoring strict interior local maximum
    with p > 8 (1 if none), then capped to the smallest divisor of n in
    (1024, best] that divides best."""
    if len(list_periods_and_scores) == 0:
        raise ValueError("Expected at least one valid period candidate.")
    rows = []
    last = len(list_periods_and_scores) - 1
    for k, (p, score) in enumerate(list_periods_and_scores):
        if k == last:
            gap = 0.0
        else:
            nxt = list_periods_and_scores[k + 1][1]
            if nxt == 0.0:
                gap = 0.0 if score == 0.0 else float("inf")
            else:
                gap = score / nxt
        rows.append((p, score, gap))
    del threshold
    last_period = list_periods_and_scores[-1][0]
    candidates = []
    for k in range(1, len(list_periods_and_scores) - 1):
        p, score = list_periods_and_scores[k]
        if p <= 8 or p == last_period:
            continue
        if score <= list_periods_and_scores[k - 1][1] or score <= list_periods_and_scores[k + 1][1]:
            continue
        candidates.append((score, p))
    if not candidates:
        best_period = 1
    else:
        best_score, best_period = max(candidates)
        if not math.isfinite(best_score):
            raise ValueError("Expected finite best score, got {}.".format(best_score))
    cap = 1024
    if best_period > cap:
        best_period = min(p for p in divisors(flattened_length)
                          if p > cap and p <= best_period and best_period % p == 0)
    if print_results:
        print(f"Flattened length: {flattened_length}")
        for p, score, gap in rows:
            line = f"p={p} |  score={score:.10f} | score gap = {gap:.3f}"
            print(f"\033[92m{line}\033[0m" if p == best_period else line)
    return best_period


class PeriodScorer:
    """Scores the candidate divisors of many gradients with one host sync.

    add() enqueues the device scoring of one flat gradient; finish() copies all
    scores to the host once and returns the chosen period of each gradient."""

    def __init__(self, mode: int = 1, epsilon: float = 1e-12, min_num_blocks: int = DMNB):
        self.mode = mode
        self.epsilon = epsilon
        self.min_num_blocks = min_num_blocks
        self.items = []

    def add(self, flat: torch.Tensor, max_period: Optional[int] = None, print_results: bool = False):
        n = flat.numel()
        divs = candidate_divisors(n, max_period, self.min_num_blocks) if n > 1 else []
        self.items.append((flat, divs, print_results))
        return len(self.items) - 1

    def finish(self) -> List[int]:
        from gefen_amd.kernels.period_variance import period_scores_launch, period_scores_workspace_bytes

        work = [(i, f, d) for i, (f, d, _) in enumerate(self.items) if d]
        results: List[Optional[int]] = [None if d else 1 for (_, d, _) in self.items]
        if work:
            dev = work[0][1].device
            ws_bytes = max(period_scores_workspace_bytes(f.numel(), d) for _, f, d in work)
            workspace = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=dev)
            offsets = []
            total = 0
            for _, f, d in work:
                offsets.append(total)
                total += len(d) + 1
            scores = torch.empty(total, dtype=torch.float64, device=dev)
            keep = []
            for (i, f, d), off in zip(work, offsets):
                flat = f.detach().reshape(-1).contiguous()
                keep.append(flat)
                period_scores_launch(flat, d, self.mode, self.epsilon, scores[off:off + len(d) + 1], workspace)
            host = scores.cpu().tolist()  # the one synchronisation
            del keep, workspace
            for (i, f, d), off in zip(work, offsets):
                if host[off + len(d)] > 0:
                    raise ValueError("Expected values plus epsilon to be positive before log transform.")
                pairs = list(zip(d, host[off:off + len(d)]))
                results[i] = _finalize_period_results(pairs, self.items[i][2], f.numel(), 0.25)
        self.items = []
        return results  # type: ignore[return-value]


def find_period_by_block_variance(squared_grad_flattened_values, print_results=True, parameter_name=None,
                                  parameter_shape=None, backend="cpu", input_is_squared=True, max_period=None,
                                  threshold=0.25, epsilon=1e-12, min_num_blocks=DMNB):
    """partitioning.py:350-398 on a device tensor.  Every backend name is
    accepted and scored by the HIP kernels; input_is_squared=False squares in
    float64 as the reference's CPU scorer and CUDA kernel do."""
    if backend not in ("cpu", "gpu", "cuda_kernel"):
        raise ValueError("Unexpected backend: {}".format(backend))
    values = squared_grad_flattened_values
    if not isinstance(values, torch.Tensor) or values.device.type != "cuda":
        raise ValueError("gefen_amd scores periods on a HIP device tensor, got {}".format(
            type(values).__name__ if not isinstance(values, torch.Tensor) else values.device))
    scorer = PeriodScorer(mode=0 if input_is_squared else 2, epsilon=epsilon, min_num_blocks=min_num_blocks)
    scorer.add(values.detach().reshape(-1), max_period, print_results)
    return scorer.finish()[0]

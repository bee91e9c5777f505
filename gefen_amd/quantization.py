"""Codebook fitting (reference: quantization.py).

``exact_dp`` runs the exact dynamic programme of quantization.py:206-258 on the
device (gefen_exact_dp in libgefen_hip.so) over a power-of-two-bin histogram;
the padded small-histogram case (quantization.py:68-81) is handled there too.
"""

from __future__ import annotations

from pathlib import Path

import torch

from gefen_amd import _lib


def save_distribution_histogram_pt_from_counts(hist: torch.Tensor, prefix: str, suffix: str, num_samples: int,
                                               value_range=(-1.0, 1.0)) -> None:
    """Debug export of a histogram to ``<prefix>_<suffix>.pt`` (quantization.py:8-52)."""
    if prefix is None:
        raise ValueError("Cannot save gradient histogram because SAVE_CODEBOOK_PREFIX is None.")
    if hist.dim() != 1:
        raise ValueError("Expected 1D histogram counts, got dim={}.".format(hist.dim()))
    if hist.numel() <= 0:
        raise ValueError("Expected at least one histogram bin.")
    if num_samples < 0:
        raise ValueError("num_samples must be non-negative, got {}.".format(num_samples))
    prefix_path = Path(prefix).expanduser().resolve()
    prefix_path.parent.mkdir(parents=True, exist_ok=True)
    out = prefix_path.parent / "{}_{}.pt".format(prefix_path.stem, suffix)
    h = hist.detach().cpu().to(torch.float32)
    left, right = value_range
    edges = torch.linspace(float(left), float(right), steps=h.numel() + 1, dtype=torch.float32)
    torch.save({"hist": h, "bin_edges": edges, "bin_centers": 0.5 * (edges[:-1] + edges[1:]),
                "bin_width": float(right - left) / float(h.numel()), "range": (float(left), float(right)),
                "num_bins": h.numel(), "num_samples": int(num_samples)}, out)
    print("Saved distribution histogram data to {}".format(out))


def exact_dp_from_counts(bin_counts: torch.Tensor, num_codebooks: int, force_endpoints: bool = True) -> torch.Tensor:
    """Optimal num_codebooks-level quantiser of an fp32 histogram over [-1, 1]
    (bins a power of two); returns the sorted fp32 codebook on the counts' device."""
    if not isinstance(bin_counts, torch.Tensor) or bin_counts.device.type != "cuda":
        raise ValueError("exact_dp runs on a HIP device tensor of bin counts")
    counts = bin_counts.detach().to(torch.float32).contiguous()
    bins = counts.numel()
    lib = _lib.load()
    ws = torch.empty(int(lib.gefen_exact_dp_workspace_size(bins, num_codebooks)), dtype=torch.uint8,
                     device=counts.device)
    out = torch.empty(num_codebooks, dtype=torch.float32, device=counts.device)
    with torch.cuda.device(counts.device):
        rc = lib.gefen_exact_dp(counts.data_ptr(), bins, num_codebooks, int(bool(force_endpoints)), out.data_ptr(),
                                ws.data_ptr(), torch.cuda.current_stream(counts.device).cuda_stream)
    _lib.check(rc, "gefen_exact_dp")
    return out


def exact_dp(histogram_stats: dict, num_codebooks: int, force_endpoints: bool = True) -> torch.Tensor:
    """quantization.py:206-258 on the statistics dict built at gefen.py:373-387
    (uses its full ``bin_counts``)."""
    counts = histogram_stats["bin_counts"]
    active = histogram_stats.get("active_counts")
    if active is not None and active.numel() == 0:
        raise ValueError("Cannot run exact DP on an empty histogram.")
    if not isinstance(counts, torch.Tensor) or counts.device.type != "cuda":
        raise ValueError("exact_dp runs on a HIP device tensor of bin counts")
    return exact_dp_from_counts(counts, num_codebooks, force_endpoints)

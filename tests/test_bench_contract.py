"""bench.py's output contract: one JSON line with the driver's keys, a roofline
object and, for the default config, the other BASELINE configs under
other_configs; more than one GPU is refused before any device work."""

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
KEYS = {"metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
        "vs_baseline", "dtype", "data", "config", "roofline"}


def _run(args, timeout):
    return subprocess.run([sys.executable, str(REPO / "bench.py")] + args, capture_output=True, text=True,
                          timeout=timeout, cwd=str(REPO), env=dict(os.environ))


def test_more_than_one_gpu_is_refused():
    r = _run(["--gpus", "2"], 120)
    assert r.returncode == 2
    assert "Run with --gpus 1" in r.stderr
    assert r.stdout.strip() == ""


@pytest.mark.gpu
def test_bench_line_for_a_small_config():
    r = _run(["--config", "gpt2", "--steps", "3", "--warmup", "1", "--no-cpu-baseline"], 300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert len(lines) == 1
    out = json.loads(lines[0])
    assert KEYS <= set(out)
    assert out["n_gpus"] == 1 and out["steps"] == 3 and out["warmup"] == 1
    assert out["higher_is_better"] is False and out["unit"] == "ms" and out["dtype"] == "f32"
    assert out["value"] == out["ms_per_step"] > 0
    roof = out["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert 0 < roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"], abs=1e-4)
    assert out["config"]["tensors"] == 111 and sum(out["config"]["periods"].values()) == 111
    # the step's timing split: launches inside step(), host time, the C calls
    for key in ("kernel_ms_per_step", "step_frac", "frac_back_to_back", "copy_kernel_gbs", "host_ms_per_step",
                "gpu_ms_outside_launches", "host_ms_plan_run", "host_ms_step_tasks"):
        assert roof[key] > 0, key
    assert roof["kernel_ms_per_step"] < out["ms_per_step"]
    assert roof["step_frac"] == pytest.approx(roof["algorithmic_bytes_per_step"] / (out["ms_per_step"] * 1e-3) / 1e9
                                              / roof["peak"], abs=1e-3)

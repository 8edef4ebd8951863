"""bench.py's output line: the keys and meanings the driver reads.

The GPU cases run bench.py in a child process at the reference's small
configuration (C1, 256^3) and check its one JSON line; the CPU case checks
that more than one GPU is refused before anything touches a device.
"""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args, timeout=240):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                          stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                          timeout=timeout)


def test_bench_refuses_more_than_one_gpu():
    res = _run("--gpus", "2", timeout=120)
    assert res.returncode == 2
    assert "one GPU only" in res.stderr
    assert res.stdout.strip() == ""


@pytest.mark.gpu
@pytest.mark.parametrize("steps", [1, 4])
def test_bench_line_contract(gpu, steps):
    """One JSON line with the contract's keys; the roofline and split figures
    are positive and consistent with each other; with one timed step the
    events of all four phases are recorded in it, with more the even steps
    time the splits and the odd ones the cross-GEMM."""
    print(f"bench C1 steps={steps}", flush=True)
    res = _run("--config", "C1", "--no-cpu", "--steps", str(steps), "--warmup", "3")
    assert res.returncode == 0, res.stderr[-2000:]
    lines = [ln for ln in res.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, res.stdout
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
              "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
              "roofline", "split", "rel_err", "median_flushed"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == steps and d["warmup"] == 3
    assert d["unit"] == "TFLOP/s" and d["higher_is_better"] is True
    assert d["value"] > 0 and d["ms_per_step"] > 0
    cfg = d["config"]
    assert (cfg["M"], cfg["N"], cfg["K"], cfg["num_splits"]) == (256, 256, 256, 2)
    emu = 2.0 * 256 ** 3 / (d["ms_per_step"] * 1e-3) / 1e12
    assert abs(emu - d["value"]) <= 0.01 * d["value"] + 1e-3
    r = d["roofline"]
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["peak"] == 2500.0
    assert r["avg_ms"] > 0 and r["achieved"] > 0
    assert abs(r["frac"] - r["achieved"] / r["peak"]) < 1e-3
    assert r["kernel"].startswith("cross_gemm_") and r["kernel"].endswith("_kernel")
    s = d["split"]
    assert s["bound"] == "hbm" and s["ms_a"] > 0 and isinstance(s["one_launch"], bool)
    assert abs(s["frac"] - s["achieved"] / s["peak"]) < 1e-3
    assert 0 < d["rel_err"] < 1e-6

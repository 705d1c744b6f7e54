"""bench.py's output contract: one JSON line with the headline metric, its
roofline entry and the CPU baseline; one GPU only."""
import json
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(REPO, "bench.py")


def test_more_than_one_gpu_is_refused_with_a_message():
    proc = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True,
                          timeout=60, cwd=REPO)
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr
    assert proc.stdout == ""


@pytest.mark.gpu
def test_default_bench_line_has_the_contract_fields():
    proc = subprocess.run([sys.executable, BENCH, "--steps", "20", "--warmup", "5",
                           "--cpu-budget", "1"], capture_output=True, text=True, timeout=110,
                          cwd=REPO)
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = [ln for ln in proc.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, proc.stdout
    r = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in r, key
    assert r["n_gpus"] == 1 and r["steps"] == 20 and r["warmup"] == 5
    assert r["unit"] == "GB/s" and r["higher_is_better"] is True and r["dtype"] == "bf16"
    assert r["value"] > 0 and r["ms_per_step"] > 0
    assert "workload" in r["config"] and "model" not in r["config"]
    # value = algorithmic bytes / wall time per step
    algo = r["config"]["algorithmic_bytes_per_step"]
    assert r["value"] == pytest.approx(algo / (r["ms_per_step"] * 1e-3) / 1e9, rel=1e-6)
    roof = r["roofline"]
    assert set(roof) >= {"bound", "achieved", "peak", "unit", "frac", "traffic"}
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert 0 < roof["frac"] <= 1 and roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"])
    cpu = r["cpu_baseline"]
    assert set(cpu) >= {"value", "unit", "cores", "kind", "sample"}
    assert cpu["kind"] == "port" and cpu["value"] > 0 and cpu["cores"] >= 1

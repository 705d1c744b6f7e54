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
@pytest.mark.timeout(420)
def test_default_bench_line_has_the_contract_fields():
    """The default run: the headline (GQA Qwen2.5-7B decode) at the top, and
    every workload under "configs", each with its step time, HIP-event kernel
    times, a roofline entry (achieved <= peak) and a CPU baseline; the fp8-pool
    batch and the AttentionNode backend's calls beside them."""
    print("bench.py default run, --steps 10 --warmup 3 --cpu-budget 0.5", flush=True)
    proc = subprocess.run([sys.executable, BENCH, "--steps", "10", "--warmup", "3",
                           "--cpu-budget", "0.5"], capture_output=True, text=True, timeout=400,
                          cwd=REPO)
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = [ln for ln in proc.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, proc.stdout
    r = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline", "configs"):
        assert key in r, key
    assert r["n_gpus"] == 1 and r["steps"] == 10 and r["warmup"] == 3
    assert r["unit"] == "GB/s" and r["higher_is_better"] is True and r["dtype"] == "bf16"
    assert r["value"] > 0 and r["ms_per_step"] > 0
    assert "workload" in r["config"] and "model" not in r["config"]
    # value = algorithmic bytes / wall time per step
    algo = r["config"]["algorithmic_bytes_per_step"]
    assert r["value"] == pytest.approx(algo / (r["ms_per_step"] * 1e-3) / 1e9, rel=1e-6)
    extra = {"qwen7b_fp8", "node", "node_packed", "node_fp32"}
    assert set(r["configs"]) == {"opt125m", "llama7b", "long32k", "prefill", "qwen7b"} | extra
    # the fp8-pool batch: its own line, roofline and parity; the AttentionNode
    # backend's calls: wall time per call
    fp8 = r["configs"].pop("qwen7b_fp8")
    assert "error" not in fp8, fp8
    assert 0 < fp8["roofline"]["frac"] <= 1 and fp8["parity"]["within_bar"], fp8
    assert fp8["parity"]["rows"] == 128
    for name in ("node", "node_packed", "node_fp32"):
        e = r["configs"].pop(name)
        assert "error" not in e, (name, e)
        assert e["unit"] == "ms" and e["value"] > 0 and e["higher_is_better"] is False, name
    assert r["configs"]["qwen7b"]["value"] == r["value"]
    # OPT-125m: the step is the fused append + single-pass decode; the
    # two-launch form (reshape_and_cache, then the decode) is timed beside it
    assert "paged_decode_append" in r["configs"]["opt125m"]["kernels_us"]
    assert "reshape_and_cache" in r["configs"]["opt125m"]["two_launch"]["kernels_us"]
    assert "merge" in r["configs"]["long32k"]["kernels_us"]
    for name, e in r["configs"].items():
        roof = e["roofline"]
        assert set(roof) >= {"bound", "achieved", "peak", "unit", "frac", "traffic"}, name
        assert roof["bound"] == ("mfma" if name == "prefill" else "hbm"), name
        assert roof["peak"] == (2500.0 if name == "prefill" else 8000.0), name
        assert 0 < roof["frac"] <= 1, name
        assert roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"]), name
        assert 0 < e["value"] <= roof["peak"], name  # whole-step rate under the peak
        cpu = e["cpu_baseline"]
        assert set(cpu) >= {"value", "unit", "cores", "kind", "sample"}, name
        assert cpu["kind"] == "port" and cpu["value"] > 0 and cpu["cores"] >= 1, name
        assert cpu["unit"] == e["unit"], name
        # one timing rule: achieved = work per launch / back-to-back mean
        assert roof["kernel_us"] == pytest.approx(
            list(e["kernel_us_back_to_back"].values())[0]), name
        scale = 1e9 if roof["unit"] == "GB/s" else 1e12
        assert roof["achieved"] == pytest.approx(
            roof["work_per_launch"] / (roof["kernel_us"] * 1e-6) / scale), name
        # the timed launch's output against the oracle, every row
        par = e["parity"]
        assert par["within_bar"] and par["finite"], (name, par)
        assert par["max_abs"] <= 2e-3 and par["max_rel"] <= 1e-2, (name, par)
    assert r["parity"] == r["configs"]["qwen7b"]["parity"]
    assert r["configs"]["qwen7b"]["parity"]["rows"] == 128
    assert r["configs"]["llama7b"]["parity"]["rows"] == 64
    assert r["configs"]["long32k"]["parity"]["rows"] == 16
    assert r["configs"]["prefill"]["parity"]["rows"] == 8 * 512

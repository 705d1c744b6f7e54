"""The launches bench.py times, checked at the workloads' full sizes.

Each test builds a workload with bench.py's own seeded builder, runs bench.py's
measurement function on it (its schedule, wave count, partition size and
pool rotation, a few steps), and compares the output of the last timed
launch, every row, with the fp32 oracle through the literal parity bar:
max-abs 2e-3, max-rel 1e-2 where |ref| >= 0.2. Reference semantics:
src/core/attention_backend.py:116-118 (decode), :105-118 applied per query
token (chunked prefill)."""
import argparse

import pytest
import torch

import bench
from oracle import attention as oa
from tests.helpers import assert_parity_bar

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(240)]


def _args():
    return argparse.Namespace(steps=2, warmup=1, settle=0.0, waves=0, partition=None)


@pytest.mark.parametrize("name,schedule,rows", [
    ("opt125m", "single", 8),      # fused append + single pass, 8 x 128, fp32
    ("llama7b", "balanced", 64),   # 64 x 2048, 32 heads, fp16
    ("long32k", "split", 16),      # 16 x 32768, 32 q / 8 kv heads, fp16, partition 512
    ("qwen7b", "balanced", 128),   # 128 x U[256, 8192], 28 q / 4 kv heads, bf16 (headline)
])
def test_bench_decode_launch_full_batch(name, schedule, rows):
    print(f"bench launch {name}: full batch, schedule {schedule}", flush=True)
    entry, host = bench.measure_decode(_args(), name)
    assert entry["schedule"] == schedule
    if name == "long32k":
        assert entry["partition_size"] == 512
    assert len(host["seqs"]) == rows == entry["num_seqs"]
    ref = torch.stack([oa.attend(q, kk, vv, host["scale"]) for q, kk, vv in host["seqs"]])
    assert_parity_bar(host["out"], ref, f"{name}: bench launch, all {rows} sequences")
    # bench.py's own parity leg reads the same figures
    rec = bench.parity_decode(host, name)
    assert rec["within_bar"] and rec["rows"] == rows


def test_bench_prefill_launch_full_batch():
    """8 x (4096 cached + 512 new), 32 q / 8 kv heads, bf16: the append and
    the prefill as timed, all 4096 query rows against the causal-masked
    contraction of the oracle."""
    print("bench launch prefill: 8 x (4096 + 512)", flush=True)
    entry, host = bench.measure_prefill(_args())
    ref = torch.stack([oa.chunked_prefill_masked(host["q"][s], host["keys"][s],
                                                 host["values"][s], host["scale"])
                       for s in range(8)])
    assert_parity_bar(host["out"], ref, "prefill: bench launch, 8 x 512 query rows")
    assert bench.parity_prefill(host, "prefill")["within_bar"]


def test_bench_fp8_launch_full_batch():
    """The GQA Qwen2.5-7B batch over fp8 (e4m3) pools as bench.py times it
    (--config qwen7b_fp8): the parity entry covers all 128 sequences."""
    print("bench launch qwen7b_fp8: full batch", flush=True)
    res = bench.bench_decode_fp8(_args())
    par = res["parity"]
    assert par["rows"] == 128 and par["within_bar"], par

"""KVCacheManager bookkeeping (CPU): bit-exact against the oracle's
restatement of src/core/memory_manager.py:55-173 and the reference tests'
known answers. The data path (attention, KV writes) needs the HIP device
and is covered by the gpu tests; here it must refuse to run."""
import json
import os
import random

import pytest
import torch

from cloverinfer_amd.memory_manager import KVCacheManager
from oracle.blocks import BlockBookkeeping

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def _mgr(nb, bs, h=2, d=8, **kw):
    return KVCacheManager(nb, bs, h, d, device="cpu", **kw)


def test_reference_kat_append():
    kat = KATS["test_kernels_append"]
    m = _mgr(kat["num_blocks"], kat["block_size"], kat["num_heads"], kat["head_dim"])
    m.allocate("req_1", seq_len=0)
    for _ in range(5):
        m.append_slot("req_1")
    assert m.context_lens["req_1"] == kat["context_len"]
    assert m.block_tables["req_1"] == kat["block_table"]
    assert m.k_cache.shape == (16, 4, 2, 8)


def test_reference_kat_50_appends():
    kat = KATS["verify_attention_kernel_vs_ref"]
    m = _mgr(kat["num_blocks"], kat["block_size"], 4, 32, dtype=torch.float16)
    m.allocate("r", 0)
    for _ in range(50):
        m.append_slot("r")
    assert m.block_tables["r"] == kat["block_table"]
    assert m.context_lens["r"] == kat["context_len"]


def test_random_op_sequences_match_oracle():
    rng = random.Random(0)
    for trial in range(30):
        nb, bs = rng.choice([(8, 4), (32, 16), (64, 2), (5, 1)])
        m, o = _mgr(nb, bs), BlockBookkeeping(nb, bs)
        live = []
        for step in range(200):
            op = rng.random()
            try:
                if op < 0.3:
                    rid, n = f"r{step}", rng.randrange(0, 3 * bs)
                    try:
                        o.allocate(rid, n)
                    except Exception as e:  # the product must raise the same class
                        with pytest.raises(type(e), match=str(e)):
                            m.allocate(rid, n)
                        continue
                    m.allocate(rid, n)
                    live.append(rid)
                elif op < 0.8 and live:
                    rid = rng.choice(live)
                    try:
                        exp = o.append_slot(rid)
                    except Exception as e:
                        with pytest.raises(type(e), match=str(e)):
                            m.append_slot(rid)
                        continue
                    assert m.append_slot(rid) == exp
                elif live:
                    rid = live.pop(rng.randrange(len(live)))
                    o.free(rid)
                    m.free(rid)
            finally:
                assert m.free_blocks == o.free_blocks
                assert m.block_tables == o.block_tables
                assert m.context_lens == o.context_lens
        if live:
            bt, ctx, mx = m.get_kernel_inputs(live)
            tables, lens, omx = o.kernel_inputs(live)
            assert bt.dtype == torch.int32 and ctx.dtype == torch.int32
            assert bt.tolist() == tables and ctx.tolist() == lens and mx == omx


def test_duplicate_and_oom_errors():
    m = _mgr(2, 4)
    m.allocate("a", 3)  # ceil(4/4) = 1 block
    with pytest.raises(ValueError, match="already exists"):
        m.allocate("a")
    m.allocate("b", 0)
    with pytest.raises(RuntimeError, match="OOM: Not enough blocks"):
        m.allocate("c")
    m.append_slot("a")  # 3 -> 4 fills block
    with pytest.raises(RuntimeError, match="OOM during append"):
        m.append_slot("a")
    m.free("missing")  # no-op


def test_slot_mapping():
    m = _mgr(8, 4)
    m.allocate("a", 9)  # ceil(10/4) = 3 blocks: [7, 6, 5]
    assert m.slot_mapping("a", [0, 3, 4, 9]) == [28, 31, 24, 21]


def test_gqa_pool_shape_and_defaults():
    m = KVCacheManager(4, 16, 28, 128, dtype=torch.bfloat16, device="cpu", num_kv_heads=4)
    assert m.k_cache.shape == (4, 16, 4, 128) and m.k_cache.dtype == torch.bfloat16
    assert m.scale == pytest.approx(128 ** -0.5)
    with pytest.raises(ValueError):
        KVCacheManager(4, 16, 6, 64, device="cpu", num_kv_heads=4)


def test_data_path_refuses_cpu():
    m = _mgr(4, 4)
    m.allocate("a", 0)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        m.attention(torch.randn(1, 2, 8), ["a"])
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        m.write_new_kv("a", torch.randn(2, 8), torch.randn(2, 8))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        m.load_initial_kv("b", torch.randn(3, 2, 8), torch.randn(3, 2, 8))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        m._paged_attention_ref(torch.randn(1, 2, 8), ["a"])


def test_batch_append_block_count():
    """write_new_kv_batch counts the blocks a batch takes before appending
    anything (all or nothing): a request listed twice takes a block for the
    token that crosses its border only, and the count equals what the same
    appends one by one take from the free list."""
    for lens, order in (([3, 4, 0], ["a", "b", "c"]), ([3, 3], ["a", "a", "b", "a"]),
                        ([7, 8], ["b", "b", "b", "b", "b"])):
        m = _mgr(64, 4)
        for rid, T in zip("abc", lens):
            m.allocate(rid, T)
        need = m._blocks_needed(order)
        free0 = len(m.free_blocks)
        for rid in order:
            m.append_slot(rid)
        assert free0 - len(m.free_blocks) == need
    m = _mgr(3, 4)
    for rid in "ab":
        m.allocate(rid, 3)  # one block each
        m.append_slot(rid)  # now full
    assert m._blocks_needed(["a", "b"]) == 2 > len(m.free_blocks) == 1
    with pytest.raises(KeyError):
        m._blocks_needed(["zz"])

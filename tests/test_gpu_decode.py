"""Paged decode on the GPU against the fp32 CPU oracle, through the C ABI.

Oracle-sized cases compare every output element; full-size configurations
are checked on sampled sequences plus split-K == single-pass."""
import math

import pytest
import torch

from cloverinfer_amd import kernels
from cloverinfer_amd.memory_manager import KVCacheManager
from oracle import attention as oa
from tests.helpers import (assert_attention_close, assert_parity_bar, make_paged_kv,
                           padded_tables)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def run_decode(q, k, v, tables, ctx, scale, partition_size=None, width=None, num_waves=0):
    qg = q.to(DEV)
    out = torch.full_like(qg, float("nan"))  # a row the kernels leave unwritten shows as NaN
    bt = padded_tables(tables, width).to(DEV)
    cl = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    kernels.paged_attention(out, qg, k.to(DEV), v.to(DEV), bt, cl, k.shape[1], max(ctx),
                            scale=scale, partition_size=partition_size, num_waves=num_waves)
    torch.cuda.synchronize()
    return out.cpu()


def case(seed, ctx, hq, hkv, d, bs, dtype, scale=None, value_scale=1.0):
    k, v, tables = make_paged_kv(seed, ctx, hkv, d, bs, dtype, value_scale, spare_blocks=3)
    g = torch.Generator().manual_seed(seed + 1)
    q = (torch.randn(len(ctx), hq, d, generator=g) * value_scale).to(dtype)
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    return q, k, v, tables, scale


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hq,hkv,d", [(8, 8, 128), (28, 4, 128), (32, 8, 64), (16, 1, 128),
                                      (32, 1, 64), (6, 2, 256), (4, 4, 32), (128, 4, 128),
                                      (96, 8, 64), (24, 12, 128),
                                      # VALU head dims with more than four query heads per
                                      # kv head (the kernel's 16-row query-head chunk)
                                      (16, 2, 256), (28, 4, 32)])
@pytest.mark.parametrize("partition", [None, 0, 32, 512])
def test_decode_matches_oracle(dtype, hq, hkv, d, partition):
    ctx = [1, 17, 31, 32, 33, 100, 511, 513, 1000, 0]
    print(f"decode dtype={dtype} hq={hq} hkv={hkv} d={d} P={partition}", flush=True)
    q, k, v, tables, scale = case(hq * 7 + d, ctx, hq, hkv, d, 16, dtype)
    got = run_decode(q, k, v, tables, ctx, scale, partition_size=partition)
    ref = oa.paged_decode(q, k, v, tables, ctx, scale)
    assert_attention_close(got, ref, what=f"{dtype} {hq}/{hkv} d{d} P{partition}")
    assert torch.equal(got[-1].float(), torch.zeros(hq, d))  # empty context -> zeros


@pytest.mark.parametrize("bs", [4, 8, 32, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_block_sizes(bs, dtype):
    ctx = [5, 64, 129, 300]
    q, k, v, tables, scale = case(bs, ctx, 14, 2, 128, bs, dtype)
    for partition in (None, 0, 64):
        width = max(len(t) for t in tables) + 3  # extra -1 padding columns
        got = run_decode(q, k, v, tables, ctx, scale, partition_size=partition, width=width)
        ref = oa.paged_decode(q, k, v, tables, ctx, scale)
        assert_attention_close(got, ref, what=f"bs{bs} {dtype} P{partition}")


@pytest.mark.parametrize("num_waves", [1, 3, 7, 64, 1000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_balanced_decode_wave_counts(num_waves, dtype):
    """The balanced decode splits the batch's steps over any number of waves;
    spans cross sequence and kv-head borders and skip empty contexts."""
    ctx = [0, 1, 16, 17, 300, 0, 1000, 33, 2050]
    print(f"balanced waves={num_waves} dtype={dtype}", flush=True)
    q, k, v, tables, scale = case(num_waves + 3, ctx, 28, 4, 128, 16, dtype)
    got = run_decode(q, k, v, tables, ctx, scale, partition_size=None, num_waves=num_waves)
    ref = oa.paged_decode(q, k, v, tables, ctx, scale)
    assert_attention_close(got, ref, what=f"balanced W={num_waves}")
    assert torch.equal(got[0].float(), torch.zeros(28, 128))


@pytest.mark.parametrize("ctx", [
    [0, 3000, 17, 811, 0, 4096, 256, 1500, 33, 2222] * 4,  # every piece long
    [480] * 10,     # 340 steps: pieces held at one step per group
    [200] * 10,     # 170 steps: fewer than the first piece's groups, even split
], ids=["ragged", "clamped", "even"])
@pytest.mark.parametrize("slots", [2, 3])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_balanced_decode_workgroups_per_cu(ctx, slots, dtype):
    """At two or three workgroups per compute unit the balanced decode splits
    the steps in one piece per dispatch slot (the older slots take more);
    the merge must find every segment's partials under that split."""
    waves = slots * kernels._native.load().clv_default_num_waves()
    print(f"balanced slots={slots} waves={waves} dtype={dtype} nseq={len(ctx)}", flush=True)
    q, k, v, tables, scale = case(len(ctx) + 5, ctx, 28, 4, 128, 16, dtype)
    got = run_decode(q, k, v, tables, ctx, scale, partition_size=None, num_waves=waves)
    ref = oa.paged_decode(q, k, v, tables, ctx, scale)
    assert_attention_close(got, ref, what=f"balanced W={waves}")


@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 1), (32, 32)])  # head groups 2, 1, 2
@pytest.mark.parametrize("slots", [2, 3])
def test_balanced_decode_workgroups_per_cu_head_groups(hq, hkv, slots):
    """The per-slot split with head groups of two and one (the pieces hold
    4 * CUs / head_group groups each) on a ragged batch long enough for every
    piece."""
    waves = slots * kernels._native.load().clv_default_num_waves()
    ctx = [int(c) for c in torch.randint(0, 3000, (24,),
                                          generator=torch.Generator().manual_seed(hkv + slots))]
    print(f"balanced slots={slots} hq={hq} hkv={hkv} waves={waves}", flush=True)
    q, k, v, tables, scale = case(hkv * 10 + slots, ctx, hq, hkv, 128, 16, torch.bfloat16)
    got = run_decode(q, k, v, tables, ctx, scale, partition_size=None, num_waves=waves)
    ref = oa.paged_decode(q, k, v, tables, ctx, scale)
    assert_attention_close(got, ref, what=f"balanced {hq}/{hkv} W={waves}")


@pytest.mark.parametrize("d,bs", [(128, 16), (64, 16), (128, 8), (64, 4)])
def test_fp32_balanced_decode_is_fp32_exact(d, bs):
    """fp32 pools on the fp32 MFMA wave: nothing is rounded below fp32, so
    the result agrees with the float64 brute force to fp32 accuracy (a bar
    100x tighter than the 16-bit one)."""
    ctx = [0, 1, 15, 16, 17, 250, 1031]
    q, k, v, tables, scale = case(d + bs, ctx, 28, 4, d, bs, torch.float32)
    got = run_decode(q, k, v, tables, ctx, scale, partition_size=None)
    for s, c in enumerate(ctx):
        if c == 0:
            assert torch.equal(got[s], torch.zeros(28, d))
            continue
        kk, vv = oa.gather_context(k, v, tables[s], c)
        # float64 attention with the h // G grouping (oa.attend's, in float64)
        qf = q[s].double().view(4, 7, d)
        w = torch.softmax(torch.einsum("kgd,lkd->kgl", qf, kk.double()) * scale, dim=-1)
        want = torch.einsum("kgl,lkd->kgd", w, vv.double()).reshape(28, d)
        err = (got[s].double() - want).abs().max().item()
        assert err < 2e-5, (s, c, err)


def test_balanced_decode_many_segments():
    """4096 (sequence, kv head) segments: the largest count the balanced
    decode holds (asked for by a wave count); one more sequence falls back to
    the schedule chosen without it."""
    for nseq in (1024, 1025):
        ctx = [int(x) for x in torch.randint(0, 70, (nseq,),
                                              generator=torch.Generator().manual_seed(nseq))]
        q, k, v, tables, scale = case(nseq, ctx, 8, 4, 64, 16, torch.float16)
        got = run_decode(q, k, v, tables, ctx, scale, num_waves=1024)
        ref = oa.paged_decode(q, k, v, tables, ctx, scale)
        assert_attention_close(got, ref, what=f"{nseq} seqs")


def test_decode_strided_query_and_output():
    ctx = [40, 200, 77]
    q, k, v, tables, scale = case(11, ctx, 8, 2, 128, 16, torch.float16)
    qkv = torch.randn(3, 12, 128).half().to(DEV)
    qkv[:, :8] = q.to(DEV)
    qv = qkv[:, :8]          # strided view (seq stride 12*128)
    outbuf = torch.zeros(3, 10, 128, dtype=torch.float16, device=DEV)
    out = outbuf[:, 1:9]
    kernels.paged_attention(out, qv, k.to(DEV), v.to(DEV), padded_tables(tables).to(DEV),
                            torch.tensor(ctx, dtype=torch.int32, device=DEV), 16, max(ctx),
                            scale=scale)
    torch.cuda.synchronize()
    assert_attention_close(out.cpu(), oa.paged_decode(q, k, v, tables, ctx, scale))
    assert torch.equal(outbuf[:, 0].cpu(), torch.zeros(3, 128, dtype=torch.float16))
    assert torch.equal(outbuf[:, 9].cpu(), torch.zeros(3, 128, dtype=torch.float16))


def test_decode_large_scores_and_one_hot():
    # Peaked softmax: one key aligned with q at a large score.
    ctx = [700]
    q, k, v, tables, _ = case(12, ctx, 4, 4, 128, 16, torch.bfloat16)
    t = 555
    b, o = tables[0][t // 16], t % 16
    k[b, o] = (q[0].float() * 4).to(torch.bfloat16)
    got = run_decode(q, k, v, tables, ctx, 1.0 / math.sqrt(128), partition_size=64)
    ref = oa.paged_decode(q, k, v, tables, ctx, 1.0 / math.sqrt(128))
    assert_attention_close(got, ref)
    assert torch.allclose(got[0].float(), v[b, o].float(), atol=2e-2)


def test_reference_kat_test_kernels_on_gpu():
    """tests/test_kernels.py:14-63 through the manager: every output element is
    sum_t t e^{2 sqrt(2) t} / sum_t e^{2 sqrt(2) t} = 3.93718491..."""
    import json, os
    kat = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                      "reference_kats.json")))["test_kernels_append"]
    m = KVCacheManager(16, 4, 2, 8, device=DEV)
    m.allocate("req_1", seq_len=0)
    for _ in range(5):
        m.append_slot("req_1")
    blocks = m.block_tables["req_1"]
    for i in range(4):
        m.k_cache[blocks[0], i] = i
        m.v_cache[blocks[0], i] = i
    m.k_cache[blocks[1], 0] = 4
    m.v_cache[blocks[1], 0] = 4
    out = m.attention(torch.ones(1, 2, 8, device=DEV), ["req_1"])
    torch.cuda.synchronize()
    assert out.shape == (1, 2, 8)
    assert torch.allclose(out.cpu(), torch.full((1, 2, 8), kat["expected_output_every_element"]),
                          atol=1e-5, rtol=0)


def test_reference_kat_identical_rows_on_gpu():
    """tests/verify_attention.py:88-136 asserted: 50 copies of one (k, v) give v."""
    m = KVCacheManager(100, 16, 4, 32, dtype=torch.float16, device=DEV)
    m.allocate("r", seq_len=0)
    g = torch.Generator().manual_seed(9)
    k = torch.randn(4, 32, generator=g).half().to(DEV)
    v = torch.randn(4, 32, generator=g).half().to(DEV)
    for _ in range(50):
        m.write_new_kv("r", k, v)
    assert m.block_tables["r"] == [99, 98, 97, 96]
    q = torch.randn(1, 4, 32, generator=g).half().to(DEV)
    out = m.attention(q, ["r"])
    torch.cuda.synchronize()
    assert torch.allclose(out[0].float().cpu(), v.float().cpu(), atol=1e-2, rtol=1e-2)


def test_reference_check_kernel_vs_reference_flow():
    """tests/verify_attention.py:88-136 as the reference runs it against the
    drop-in: attention() (the kernel) and _paged_attention_ref() (an
    independent plain-torch gather + softmax) agree to allclose(atol=1e-2,
    rtol=1e-2), both
    return tensors like q, and both equal the oracle. A query in another dtype
    than the pool comes back in its own dtype."""
    m = KVCacheManager(100, 16, 4, 32, dtype=torch.float16, device=DEV)
    m.allocate("req_test_kernel", seq_len=0)
    g = torch.Generator().manual_seed(10)
    k = torch.randn(4, 32, generator=g).half().to(DEV)
    v = torch.randn(4, 32, generator=g).half().to(DEV)
    for _ in range(50):
        m.write_new_kv("req_test_kernel", k, v)
    q = torch.randn(1, 4, 32, generator=g).half().to(DEV)
    out_kernel = m.attention(q, ["req_test_kernel"])
    out_ref = m._paged_attention_ref(q, ["req_test_kernel"])
    torch.cuda.synchronize()
    for o in (out_kernel, out_ref):
        assert o.shape == q.shape and o.dtype == q.dtype and o.device == q.device
    assert torch.allclose(out_kernel, out_ref, atol=1e-2, rtol=1e-2)
    ref = oa.attend(q[0].cpu(), k.cpu().expand(50, 4, 32), v.cpu().expand(50, 4, 32), 32 ** -0.5)
    assert_attention_close(out_ref[0], ref, what="plain-torch reference path")
    assert_attention_close(out_kernel[0], ref, what="kernel")
    q32 = q.float()
    o32 = m.attention(q32, ["req_test_kernel"])
    assert o32.dtype == torch.float32 and o32.device == q32.device
    assert_attention_close(o32[0], ref, what="fp32 query over an fp16 pool")


def test_paged_attention_ref_is_independent_and_gqa():
    """_paged_attention_ref (plain torch gather + softmax, the reference's
    memory_manager.py:192-239 with the repeat_kv grouping) equals the oracle
    on a GQA pool with ragged contexts spanning several blocks, as does
    attention() over the same requests."""
    m = KVCacheManager(64, 16, 28, 128, dtype=torch.bfloat16, device=DEV, num_kv_heads=4)
    g = torch.Generator().manual_seed(21)
    rids, kv = ["a", "b", "c"], {}
    for rid, n in zip(rids, (1, 37, 300)):
        kd = torch.randn(n, 4, 128, generator=g).to(torch.bfloat16)
        vd = torch.randn(n, 4, 128, generator=g).to(torch.bfloat16)
        kv[rid] = (kd, vd)
        m.load_initial_kv(rid, kd.to(DEV), vd.to(DEV))
    q = torch.randn(3, 28, 128, generator=g).to(torch.bfloat16)
    ref = torch.stack([oa.attend(q[i], kv[r][0], kv[r][1], 128 ** -0.5)
                       for i, r in enumerate(rids)])
    out_ref = m._paged_attention_ref(q.to(DEV), rids)
    out = m.attention(q.to(DEV), rids)
    torch.cuda.synchronize()
    assert out_ref.dtype == torch.bfloat16
    assert_attention_close(out_ref.cpu(), ref, what="_paged_attention_ref, GQA")
    assert_attention_close(out.cpu(), ref, what="attention, GQA")


# ---------------------------------------------------------------- configs
def test_config_opt125m_fp32_with_append():
    """8 seqs, 12 heads, D 64, fp32, 64-block pool in random order: 127 tokens
    prefilled, one appended through reshape_and_cache -> context 128."""
    g = torch.Generator().manual_seed(1001)
    m = KVCacheManager(64, 16, 12, 64, dtype=torch.float32, device=DEV)
    m.free_blocks = torch.randperm(64, generator=g).tolist()
    rids = [f"s{i}" for i in range(8)]
    kv = {}
    for rid in rids:
        kd, vd = torch.randn(128, 12, 64, generator=g), torch.randn(128, 12, 64, generator=g)
        kv[rid] = (kd, vd)
        m.load_initial_kv(rid, kd[:127].to(DEV), vd[:127].to(DEV))
    m.write_new_kv_batch(rids, torch.stack([kv[r][0][127] for r in rids]).to(DEV),
                         torch.stack([kv[r][1][127] for r in rids]).to(DEV))
    q = torch.randn(8, 12, 64, generator=g)
    out = m.attention(q.to(DEV), rids)
    torch.cuda.synchronize()
    ref = torch.stack([oa.attend(q[i], kv[r][0], kv[r][1], 1 / 8) for i, r in enumerate(rids)])
    assert_attention_close(out.cpu(), ref, atol=1e-4, rtol=1e-4)
    assert_parity_bar(out, ref, "opt125m fp32, 8 x 128 (full config)")


@pytest.mark.parametrize("nseq", [8])
def test_config_llama7b_mha_fp16(nseq):
    ctx = [2048] * nseq
    q, k, v, tables, scale = case(1002, ctx, 32, 32, 128, 16, torch.float16, value_scale=0.5)
    ref = oa.paged_decode(q, k, v, tables, ctx, scale)
    for partition in (None, 0, 512):
        got = run_decode(q, k, v, tables, ctx, scale, partition_size=partition)
        assert_attention_close(got, ref, what=f"llama7b P{partition}")
        assert_parity_bar(got, ref, f"llama7b fp16, {nseq} x 2048, partition {partition}")


def test_config_qwen7b_gqa_bf16_ragged():
    ctx = [int(torch.randint(256, 8193, (1,), generator=torch.Generator().manual_seed(1003000 + i)))
           for i in range(16)]
    q, k, v, tables, scale = case(1003, ctx, 28, 4, 128, 16, torch.bfloat16)
    ref = oa.paged_decode(q, k, v, tables, ctx, scale)
    for partition in (None, 0, 256, 512):
        got = run_decode(q, k, v, tables, ctx, scale, partition_size=partition)
        assert_attention_close(got, ref, what=f"qwen7b P{partition}")
        assert_parity_bar(got, ref, f"qwen7b bf16, 16 seqs U[256,8192], partition {partition}")
    got = run_decode(q, k, v, tables, ctx, scale, num_waves=37)
    assert_attention_close(got, ref, what="qwen7b balanced W=37")
    assert_parity_bar(got, ref, "qwen7b bf16, 16 seqs, balanced W=37")


def test_config_long_context_splitk_fp16():
    ctx = [32768, 32768]
    q, k, v, tables, scale = case(1004, ctx, 32, 8, 128, 16, torch.float16)
    ref = oa.paged_decode(q, k, v, tables, ctx, scale)
    for partition in (512, None):
        got = run_decode(q, k, v, tables, ctx, scale, partition_size=partition)
        assert_attention_close(got, ref, what=f"long-context P{partition}")
        assert_parity_bar(got, ref, f"long32k fp16, 2 x 32768, partition {partition}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,d,max_ctx", [(32, 8, 128, 4096), (32, 8, 64, 4096),
                                              (32, 1, 128, 8192)])
def test_splitk_batch_equals_single_sequence_launches(dtype, hq, hkv, d, max_ctx):
    """Split-K partials depend on nothing but their own (sequence, kv head,
    partition): a batch of 16 ragged sequences (a grid of up to 16K
    workgroups) and the same sequences launched one at a time give bitwise
    equal outputs. Ragged contexts end on partial partitions, leave
    workgroups past a short context idle and include an empty sequence; the
    first rows are also checked against the oracle."""
    ctx = [max_ctx, max_ctx - 1, max_ctx - 31, 3000, 33, 0, 1, max_ctx] * 2
    print(f"split-K batch vs alone {dtype} hq={hq} hkv={hkv} d={d} max_ctx={max_ctx}", flush=True)
    q, k, v, tables, scale = case(1100 + d + hkv, ctx, hq, hkv, d, 16, dtype)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    bt = padded_tables(tables).to(DEV)
    cl = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    batch = torch.full_like(qg, float("nan"))
    kernels.paged_attention(batch, qg, kg, vg, bt, cl, 16, max_ctx, scale=scale, partition_size=32)
    alone = torch.full_like(qg, float("nan"))
    for s in range(len(ctx)):
        kernels.paged_attention(alone[s:s + 1], qg[s:s + 1], kg, vg, bt[s:s + 1], cl[s:s + 1], 16,
                                max_ctx, scale=scale, partition_size=32)
    torch.cuda.synchronize()
    assert torch.equal(batch.view(torch.int16), alone.view(torch.int16))
    ref = oa.paged_decode(q[:2], k, v, tables[:2], ctx[:2], scale)
    assert_attention_close(batch[:2].cpu(), ref, what="split-K batch vs oracle")


def test_decode_repeated_calls_shared_workspace():
    """Ten calls of changing shapes, wave counts and dtypes on the same cached
    workspace, with split-K calls in between on the same stream: every result
    matches the oracle (nothing a call leaves in the workspace leaks into the
    next one), empty contexts give zero rows."""
    shapes = [([300, 1, 0, 4097, 77], 28, 4, 128, 0), ([5, 900, 17], 12, 12, 64, 37),
              ([2050, 2050], 8, 2, 128, 1000), ([16, 33, 600, 1200, 3], 16, 1, 128, 7),
              ([700] * 6, 32, 8, 128, 0)]
    for rep in range(2):
        for idx, (ctx, hq, hkv, d, w) in enumerate(shapes):
            dtype = (torch.bfloat16, torch.float16, torch.float32)[(rep + idx) % 3]
            print(f"repeated balanced rep {rep} shape {idx} {dtype} W={w}", flush=True)
            q, k, v, tables, scale = case(500 + 10 * rep + idx, ctx, hq, hkv, d, 16, dtype)
            got = run_decode(q, k, v, tables, ctx, scale, num_waves=w or 1024)
            ref = oa.paged_decode(q, k, v, tables, ctx, scale)
            assert_attention_close(got, ref, what=f"rep {rep} shape {idx}")
            for s, c in enumerate(ctx):
                if c == 0:
                    assert torch.equal(got[s].float(), torch.zeros(hq, d))
            split = run_decode(q, k, v, tables, ctx, scale, partition_size=64)
            assert_attention_close(split, ref, what=f"split-K between balanced calls {idx}")

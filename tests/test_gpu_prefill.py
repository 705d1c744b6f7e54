"""Chunked prefill over paged KV on the GPU: against the oracle (row i ==
the i-th successive append-then-attend decode step) and, at the full
8 x (4096 cached + 512 new) shape, against the GPU decode kernel run with
each row's causal context length."""
import math

import pytest
import torch

from cloverinfer_amd import kernels
from oracle import attention as oa
from tests.helpers import (assert_attention_close, assert_parity_bar, make_paged_kv,
                           padded_tables)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def build(seed, cached, new, hq, hkv, d, bs, dtype):
    ctx = [c + n for c, n in zip(cached, new)]
    k, v, tables = make_paged_kv(seed, ctx, hkv, d, bs, dtype, spare_blocks=2)
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(sum(new), hq, d, generator=g).to(dtype)
    qsl = [0]
    for n in new:
        qsl.append(qsl[-1] + n)
    return q, k, v, tables, ctx, qsl


def run_prefill(q, k, v, tables, ctx, qsl, scale):
    qg = q.to(DEV)
    out = torch.full_like(qg, float("nan"))
    kernels.chunked_prefill(out, qg, k.to(DEV), v.to(DEV), padded_tables(tables).to(DEV),
                            torch.tensor(ctx, dtype=torch.int32, device=DEV),
                            torch.tensor(qsl, dtype=torch.int32, device=DEV),
                            max(b - a for a, b in zip(qsl, qsl[1:])), scale=scale)
    torch.cuda.synchronize()
    return out.cpu()


def oracle_prefill(q, k, v, tables, ctx, qsl, scale):
    outs = []
    for s in range(len(ctx)):
        kk, vv = oa.gather_context(k, v, tables[s], ctx[s])
        outs.append(oa.chunked_prefill(q[qsl[s]:qsl[s + 1]], kk, vv, scale))
    return torch.cat(outs)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 64), (28, 4, 128), (4, 2, 32)])
def test_prefill_matches_oracle(dtype, hq, hkv, d):
    print(f"prefill dtype={dtype} hq={hq} hkv={hkv} d={d}", flush=True)
    cached = [0, 5, 130, 300, 64]
    new = [7, 64, 1, 100, 129]
    q, k, v, tables, ctx, qsl = build(hq + d, cached, new, hq, hkv, d, 16, dtype)
    scale = 1.0 / math.sqrt(d)
    got = run_prefill(q, k, v, tables, ctx, qsl, scale)
    ref = oracle_prefill(q, k, v, tables, ctx, qsl, scale)
    assert_attention_close(got, ref, what=f"prefill {dtype} {hq}/{hkv} d{d}")


def test_prefill_reduced_chunk_config():
    """2 sequences of the chunked-prefill config (4096 cached + 512 new)."""
    cached, new = [4096, 4096], [512, 512]
    q, k, v, tables, ctx, qsl = build(1005, cached, new, 32, 8, 128, 16, torch.bfloat16)
    scale = 1.0 / math.sqrt(128)
    got = run_prefill(q, k, v, tables, ctx, qsl, scale)
    ref = oracle_prefill(q, k, v, tables, ctx, qsl, scale)
    assert_attention_close(got, ref, what="chunked prefill 4096+512")
    assert_parity_bar(got, ref, "prefill bf16, 2 x (4096 + 512), successive-step oracle")


def test_prefill_full_config_against_masked_oracle():
    """All 8 sequences of the chunked-prefill config (4096 cached + 512 new,
    32 q / 8 kv heads, bf16) against the oracle's causal-masked contraction
    (pinned against the successive decode steps and float64 brute force)."""
    cached, new = [4096] * 8, [512] * 8
    q, k, v, tables, ctx, qsl = build(1005, cached, new, 32, 8, 128, 16, torch.bfloat16)
    scale = 1.0 / math.sqrt(128)
    got = run_prefill(q, k, v, tables, ctx, qsl, scale)
    refs = []
    for s in range(8):
        kk, vv = oa.gather_context(k, v, tables[s], ctx[s])
        refs.append(oa.chunked_prefill_masked(q[qsl[s]:qsl[s + 1]], kk, vv, scale))
    ref = torch.cat(refs)
    assert_attention_close(got, ref, what="chunked prefill 8 x (4096+512)")
    assert_parity_bar(got, ref, "prefill bf16, 8 x (4096 + 512) (full config)")


def test_prefill_rows_equal_decode_steps_full_config():
    """8 x (4096 + 512), bf16: every query row equals the decode kernel over
    that row's causal context (the same K/V, a per-row context length)."""
    cached, new = [4096] * 8, [512] * 8
    q, k, v, tables, ctx, qsl = build(1006, cached, new, 32, 8, 128, 16, torch.bfloat16)
    scale = 1.0 / math.sqrt(128)
    got = run_prefill(q, k, v, tables, ctx, qsl, scale)
    # Decode view: one "sequence" per query row, sharing its sequence's table.
    rows_tables, rows_ctx = [], []
    for s in range(8):
        for i in range(512):
            rows_tables.append(tables[s])
            rows_ctx.append(cached[s] + i + 1)
    kg, vg = k.to(DEV), v.to(DEV)
    out = torch.empty(q.shape, dtype=q.dtype, device=DEV)
    kernels.paged_attention(out, q.to(DEV), kg, vg, padded_tables(rows_tables).to(DEV),
                            torch.tensor(rows_ctx, dtype=torch.int32, device=DEV), 16,
                            max(rows_ctx), scale=scale, partition_size=0)
    torch.cuda.synchronize()
    assert_attention_close(got, out.cpu(), what="prefill rows vs decode")


@pytest.mark.parametrize("bs", [4, 8, 32, 64])
def test_prefill_block_sizes(bs):
    cached, new = [0, 33, 200], [70, 5, 64]
    q, k, v, tables, ctx, qsl = build(300 + bs, cached, new, 16, 4, 128, bs, torch.bfloat16)
    scale = 1.0 / math.sqrt(128)
    got = run_prefill(q, k, v, tables, ctx, qsl, scale)
    ref = oracle_prefill(q, k, v, tables, ctx, qsl, scale)
    assert_attention_close(got, ref, what=f"prefill bs{bs}")


@pytest.mark.parametrize("scale", [-0.125, 0.0, 0.02])
def test_prefill_scales(scale):
    """Negative scales (applied as a sign flip of q), zero (uniform weights)
    and a small positive scale."""
    cached, new = [90, 0], [40, 130]
    q, k, v, tables, ctx, qsl = build(41, cached, new, 8, 2, 64, 16, torch.float16)
    got = run_prefill(q, k, v, tables, ctx, qsl, scale)
    ref = oracle_prefill(q, k, v, tables, ctx, qsl, scale)
    assert_attention_close(got, ref, what=f"prefill scale {scale}")


def test_prefill_bf16_values_beyond_fp16_range():
    """bf16 V values of magnitude >= 2^16 do not fit the fp16 P.V path: the
    workgroups that see them take the exact bf16 pass. Large scores too, so
    that the running maximum is raised several times."""
    cached, new = [300, 1000], [200, 300]
    q, k, v, tables, ctx, qsl = build(57, cached, new, 32, 8, 128, 16, torch.bfloat16)
    # A few huge V values in the context of sequence 1 only (sequence 0 keeps
    # the fast pass), plus a scaled-up stretch of keys.
    blk = tables[1][3]
    v[blk, 2, 5, :] = 3.0e5
    v[blk, 7, 0, 17] = -1.0e30
    k[tables[1][10], :, :, :] *= 6
    scale = 1.0 / math.sqrt(128)
    got = run_prefill(q, k, v, tables, ctx, qsl, scale)
    ref = oracle_prefill(q, k, v, tables, ctx, qsl, scale)
    assert_attention_close(got, ref, what="prefill bf16 beyond fp16 range")


def test_prefill_every_workgroup_takes_the_exact_pass():
    """Every workgroup meets a bf16 V value beyond fp16's range in its first
    tile (token 0 of every sequence and kv head, which every query row sees)
    and reruns its rows in the exact pass, all at once. The overflow flag is
    read by every wave after the fast pass; the exact pass must not clear it
    while another wave may still be reading it (waves that disagreed on taking
    the exact pass would wait at different barriers)."""
    cached, new = [512, 700, 256, 1000], [512, 300, 700, 128]
    q, k, v, tables, ctx, qsl = build(91, cached, new, 32, 8, 128, 16, torch.bfloat16)
    for s in range(len(cached)):
        v[tables[s][0], 0, :, 3] = 2.0e5
    scale = 1.0 / math.sqrt(128)
    got = run_prefill(q, k, v, tables, ctx, qsl, scale)
    assert torch.isfinite(got.float()).all()
    ref = oracle_prefill(q, k, v, tables, ctx, qsl, scale)
    assert_attention_close(got, ref, what="prefill, exact pass in every workgroup")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])  # MFMA and VALU kernels
def test_prefill_max_query_len_none_and_too_small(dtype):
    """max_query_len=None is computed from query_start_loc; a value below the
    longest chunk makes that chunk's rows at or past it NaN (a loud error, not
    stale memory), and the other rows stay exact, in both kernel forms."""
    cached, new = [30, 200], [300, 40]
    q, k, v, tables, ctx, qsl = build(77, cached, new, 16, 4, 128, 16, dtype)
    scale = 1.0 / math.sqrt(128)
    ref = oracle_prefill(q, k, v, tables, ctx, qsl, scale)
    kg, vg, bt = k.to(DEV), v.to(DEV), padded_tables(tables).to(DEV)
    cl = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    qs = torch.tensor(qsl, dtype=torch.int32, device=DEV)
    out = torch.full((q.shape[0], 16, 128), 7.0, dtype=dtype, device=DEV)
    kernels.chunked_prefill(out, q.to(DEV), kg, vg, bt, cl, qs, None, scale=scale)
    torch.cuda.synchronize()
    assert_attention_close(out.cpu(), ref, what="max_query_len=None")
    out.fill_(7.0)
    kernels.chunked_prefill(out, q.to(DEV), kg, vg, bt, cl, qs, 40, scale=scale)
    torch.cuda.synchronize()
    got = out.cpu().float()
    assert_attention_close(got[:40], ref[:40], what="rows below max_query_len")
    assert torch.isnan(got[40:300]).all(), "rows at or past max_query_len must come out as NaN"
    assert_attention_close(got[300:], ref[300:], what="the second, shorter chunk")

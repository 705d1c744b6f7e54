"""fp8 (OCP e4m3) KV pools on the GPU: the quantising append bit for bit
against the oracle's definition (clamp(x / scale) rounded to nearest even),
the balanced decode against the fp32 oracle on the dequantised pools, and
the gpu backend with kv_dtype="fp8" against the restated CpuAttentionBackend
fed the dequantised values."""
import math

import pytest
import torch

from cloverinfer_amd import kernels
from cloverinfer_amd.attention_backend import GpuAttentionBackend
from oracle import attention as oa
from oracle.attention import CpuAttentionOracle
from tests.helpers import assert_attention_close, padded_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"
FP8 = torch.float8_e4m3fn


@pytest.mark.parametrize("src", [torch.float32, torch.float16, torch.bfloat16])
def test_fp8_append_bit_exact(src):
    g = torch.Generator().manual_seed(61)
    T, H, D, NB, bs = 40, 4, 128, 8, 16
    scale_k = torch.tensor([0.5, 2.0, 0.03, 7.0])
    scale_v = torch.tensor([1.0, 0.25, 3.0, 0.01])
    k = torch.randn(T, H, D, generator=g) * torch.tensor([1.0, 100.0, 0.01, 1000.0]).view(1, H, 1)
    v = torch.randn(T, H, D, generator=g) * 3
    special = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0, 1e-8, 1e6, -3e4])
    k[0, 0, :8] = special
    v[1, 2, :8] = special
    k, v = k.to(src), v.to(src)
    slots = torch.randperm(NB * bs, generator=g)[:T].to(torch.int64)
    slots[3] = -1          # skipped
    slots[5] = NB * bs     # out of range: skipped
    kc = torch.full((NB, bs, H, D), 0x55, dtype=torch.uint8).view(FP8)
    vc = kc.clone()
    kg, vg = kc.to(DEV), vc.to(DEV)
    kernels.reshape_and_cache(k.to(DEV), v.to(DEV), kg, vg, slots.to(DEV),
                              k_scale=scale_k, v_scale=scale_v)
    torch.cuda.synchronize()
    for i, sl in enumerate(slots.tolist()):
        if 0 <= sl < NB * bs:
            kc[sl // bs, sl % bs] = oa.quantize_fp8(k[i], scale_k)
            vc[sl // bs, sl % bs] = oa.quantize_fp8(v[i], scale_v)
    assert torch.equal(kg.cpu().view(torch.uint8), kc.view(torch.uint8))
    assert torch.equal(vg.cpu().view(torch.uint8), vc.view(torch.uint8))


def _fp8_pools(seed, ctx, hkv, d, bs, ks, vs):
    """Random fp8 pools (codes of N(0,1) data at the given scales); unused
    slots hold the NaN code."""
    g = torch.Generator().manual_seed(seed)
    need = [max(1, math.ceil(c / bs)) for c in ctx]
    nb = sum(need) + 2
    perm = torch.randperm(nb, generator=g).tolist()
    tables, pos = [], 0
    for n in need:
        tables.append(perm[pos:pos + n])
        pos += n
    kc = torch.full((nb, bs, hkv, d), 0x7F, dtype=torch.uint8).view(FP8)
    vc = kc.clone()
    for t, c in zip(tables, ctx):
        for p in range(c):
            kc[t[p // bs], p % bs] = oa.quantize_fp8(torch.randn(hkv, d, generator=g) * ks.view(-1, 1), ks)
            vc[t[p // bs], p % bs] = oa.quantize_fp8(torch.randn(hkv, d, generator=g) * vs.view(-1, 1), vs)
    return kc, vc, tables


@pytest.mark.parametrize("hq,hkv,bs,qdt", [(28, 4, 16, torch.bfloat16), (32, 8, 32, torch.float16),
                                           (8, 8, 16, torch.bfloat16), (32, 1, 16, torch.float16)])
def test_fp8_decode_matches_oracle(hq, hkv, bs, qdt):
    d = 128
    ctx = [1, 15, 16, 17, 0, 300, 1000, 33]
    ks = torch.linspace(0.05, 3.0, hkv)
    vs = torch.linspace(2.0, 0.1, hkv)
    print(f"fp8 decode hq={hq} hkv={hkv} bs={bs} {qdt}", flush=True)
    kc, vc, tables = _fp8_pools(hq + bs, ctx, hkv, d, bs, ks, vs)
    q = torch.randn(len(ctx), hq, d, generator=torch.Generator().manual_seed(9)).to(qdt)
    out = torch.empty(q.shape, dtype=qdt, device=DEV)
    scale = 1.0 / math.sqrt(d)
    kernels.paged_attention(out, q.to(DEV), kc.to(DEV), vc.to(DEV), padded_tables(tables).to(DEV),
                            torch.tensor(ctx, dtype=torch.int32, device=DEV), bs, max(ctx),
                            scale=scale, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    kf = kc.float() * ks.view(1, 1, -1, 1)
    vf = vc.float() * vs.view(1, 1, -1, 1)
    ref = oa.paged_decode(q, kf, vf, tables, ctx, scale)
    assert_attention_close(out.cpu(), ref, what=f"fp8 {hq}/{hkv} bs{bs}")
    assert torch.equal(out[4].float().cpu(), torch.zeros(hq, d))


@pytest.mark.parametrize("slots", [2, 3])
def test_fp8_decode_workgroups_per_cu(slots):
    """fp8 pools at two (the default) and three workgroups per compute unit,
    with enough steps that the balanced split comes in one piece per
    dispatch slot (ragged contexts, about 2,000 steps over 512 or 768
    four-wave groups)."""
    hq, hkv, d, bs, qdt = 28, 4, 128, 16, torch.bfloat16
    ctx = [int(c) for c in torch.randint(0, 4097, (20,),
                                          generator=torch.Generator().manual_seed(slots))]
    ctx[3], ctx[7] = 0, 1
    ks = torch.linspace(0.05, 3.0, hkv)
    vs = torch.linspace(2.0, 0.1, hkv)
    waves = slots * kernels._native.load().clv_default_num_waves()
    print(f"fp8 decode slots={slots} waves={waves}", flush=True)
    kc, vc, tables = _fp8_pools(100 + slots, ctx, hkv, d, bs, ks, vs)
    q = torch.randn(len(ctx), hq, d, generator=torch.Generator().manual_seed(19)).to(qdt)
    out = torch.empty(q.shape, dtype=qdt, device=DEV)
    scale = 1.0 / math.sqrt(d)
    kernels.paged_attention(out, q.to(DEV), kc.to(DEV), vc.to(DEV), padded_tables(tables).to(DEV),
                            torch.tensor(ctx, dtype=torch.int32, device=DEV), bs, max(ctx),
                            scale=scale, num_waves=waves, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    kf = kc.float() * ks.view(1, 1, -1, 1)
    vf = vc.float() * vs.view(1, 1, -1, 1)
    ref = oa.paged_decode(q, kf, vf, tables, ctx, scale)
    assert_attention_close(out.cpu(), ref, what=f"fp8, {slots} slots")


def test_fp8_backend_steps():
    """kv_dtype="fp8" with a per-head kv_scale: fp32 and bf16 payloads, three
    decode steps on two layers, against the restated CpuAttentionBackend fed
    the values the pools hold (queries rounded to the compute dtype)."""
    g = torch.Generator().manual_seed(71)
    hq, hkv, d, layers = 14, 2, 128, 2
    scale = torch.tensor([0.02, 0.05])
    gpu = GpuAttentionBackend(num_blocks=64, block_size=16, kv_dtype="fp8", kv_scale=scale.tolist())
    cpu = CpuAttentionOracle()
    q8 = lambda t: oa.dequantize_fp8(oa.quantize_fp8(t.float(), scale), scale)
    kv = [{"key": torch.randn(29, hkv, d, generator=g), "value": torch.randn(29, hkv, d, generator=g)}
          for _ in range(layers)]
    assert gpu.init_request("r", kv) == 29
    cpu.init_request("r", [{"key": q8(x["key"]), "value": q8(x["value"])} for x in kv])
    for step in range(3):
        for layer in range(layers):
            dt = torch.float32 if step % 2 == 0 else torch.bfloat16
            it = {"request_id": "r", "layer_idx": layer,
                  "query": torch.randn(1, hq, d, generator=g).to(dt),
                  "key": torch.randn(1, hkv, d, generator=g).to(dt),
                  "value": torch.randn(1, hkv, d, generator=g).to(dt), "score_scale": d ** -0.5}
            got = gpu.decode_layer_batch([it])[0]
            ref = cpu.decode_layer_batch([{**it, "query": it["query"].to(torch.bfloat16).float(),
                                           "key": q8(it["key"]), "value": q8(it["value"])}])[0]
            assert got.dtype == dt
            assert_attention_close(got, ref, what=f"step {step} layer {layer}")
    assert gpu.get_context_len("r") == cpu.get_context_len("r") == 32


def test_fp8_partials_then_reduce_equal_the_one_call():
    """clv_paged_decode_fp8_partials followed by clv_balanced_reduce (same
    workspace and wave count) writes exactly what clv_paged_decode_fp8 writes."""
    hq, hkv, d, bs = 28, 4, 128, 16
    ctx = [1, 15, 16, 17, 0, 300, 1000, 33]
    ks = torch.linspace(0.05, 3.0, hkv)
    vs = torch.linspace(2.0, 0.1, hkv)
    kc, vc, tables = _fp8_pools(hq + bs, ctx, hkv, d, bs, ks, vs)
    q = torch.randn(len(ctx), hq, d, generator=torch.Generator().manual_seed(11)).to(torch.bfloat16)
    q, kc, vc = q.to(DEV), kc.to(DEV), vc.to(DEV)
    bt = padded_tables(tables).to(DEV)
    lens = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    ksd, vsd = ks.to(DEV), vs.to(DEV)
    lib = kernels._native.load()
    waves = lib.clv_default_num_waves_fp8()
    outs = []
    for split in (False, True):
        out = torch.full(q.shape, float("nan"), dtype=q.dtype, device=DEV)
        a = kernels.decode_args(out, q, kc, vc, bt, lens, bs, max(ctx))
        ws = torch.empty(kernels.balanced_workspace_bytes(a, waves), dtype=torch.uint8, device=DEV)
        stream = torch.cuda.current_stream().cuda_stream
        if split:
            kernels._native.check(lib.clv_paged_decode_fp8_partials(
                a, ksd.data_ptr(), vsd.data_ptr(), waves, ws.data_ptr(), ws.numel(), stream),
                "clv_paged_decode_fp8_partials")
            kernels._native.check(lib.clv_balanced_reduce(a, waves, ws.data_ptr(), ws.numel(),
                                                          stream), "clv_balanced_reduce")
        else:
            kernels._native.check(lib.clv_paged_decode_fp8(
                a, ksd.data_ptr(), vsd.data_ptr(), waves, ws.data_ptr(), ws.numel(), stream),
                "clv_paged_decode_fp8")
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1])
    assert torch.isfinite(outs[0].float()).all()

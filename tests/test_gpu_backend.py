"""The "gpu" AttentionNode backend against the CPU oracle of
CpuAttentionBackend, step by step, with the node's payload shapes."""
import math

import pytest
import torch

from cloverinfer_amd.attention_backend import GpuAttentionBackend, create_attention_backend
from oracle import attention as oa
from oracle.attention import CpuAttentionOracle
from tests.helpers import assert_attention_close

pytestmark = pytest.mark.gpu


def _drive(layers, hq, hkv, d, dtype, prompt_lens, steps, scale, seed, batch=True,
           reserve=0, block_size=16):
    g = torch.Generator().manual_seed(seed)
    gpu = create_attention_backend("gpu", {"num_blocks": 512, "block_size": block_size})
    cpu = CpuAttentionOracle()
    rids = [f"req{i}" for i in range(len(prompt_lens))]
    for rid, T in zip(rids, prompt_lens):
        kv = [{"key": torch.randn(T, hkv, d, generator=g).to(dtype),
               "value": torch.randn(T, hkv, d, generator=g).to(dtype)} for _ in range(layers)]
        assert gpu.init_request(rid, kv, decode_reserve_tokens=reserve) == T
        assert cpu.init_request(rid, kv) == T
    for step in range(steps):
        for layer in range(layers):
            items = [{"request_id": rid, "layer_idx": layer,
                      "query": torch.randn(1, hq, d, generator=g).to(dtype),
                      "key": torch.randn(hkv, d, generator=g).to(dtype),
                      "value": torch.randn(1, hkv, d, generator=g).to(dtype),
                      "score_scale": scale} for rid in rids]
            if batch:
                got = gpu.decode_layer_batch(items)
            else:
                got = [gpu.decode_layer(it["request_id"], it["layer_idx"], it["query"],
                                        it["key"], it["value"], it["score_scale"]) for it in items]
            ref = cpu.decode_layer_batch(items)
            for a, b in zip(got, ref):
                assert a.shape == b.shape and a.dtype == b.dtype and a.device == b.device
                assert_attention_close(a, b, what=f"step {step} layer {layer}")
        for rid in rids:
            assert gpu.get_context_len(rid) == cpu.get_context_len(rid)
    return gpu, rids


def test_opt125m_shape_fp16():
    # OPT pre-scales q and sends score_scale 1.0 (src/core/model_adapter.py:373,386).
    _drive(layers=12, hq=12, hkv=12, d=64, dtype=torch.float16, prompt_lens=[5, 17, 40],
           steps=3, scale=1.0, seed=21)


def test_qwen_gqa_shape_bf16_single_items():
    _drive(layers=2, hq=28, hkv=4, d=128, dtype=torch.bfloat16, prompt_lens=[15, 16, 300],
           steps=3, scale=1 / math.sqrt(128), seed=22, batch=False, block_size=8)


def test_fp32_reserve_and_free():
    gpu, rids = _drive(layers=2, hq=4, hkv=4, d=64, dtype=torch.float32, prompt_lens=[0, 31],
                       steps=2, scale=0.125, seed=23, reserve=64)
    info = gpu.get_debug_info()
    assert info["requests"] == 2 and info["backend"] == "gpu"
    before = info["free_blocks"]
    gpu.free_request(rids[1])
    gpu.free_request(rids[1])
    assert gpu.get_debug_info()["free_blocks"] > before


def test_protocol_errors():
    gpu = GpuAttentionBackend(num_blocks=4, block_size=16)
    kv = [{"key": torch.randn(3, 2, 64), "value": torch.randn(3, 2, 64)}]
    gpu.init_request("a", kv)
    with pytest.raises(ValueError):
        gpu.init_request("a", kv)
    with pytest.raises(KeyError):
        gpu.decode_layer("b", 0, torch.randn(2, 64), torch.randn(2, 64), torch.randn(2, 64))
    with pytest.raises(RuntimeError, match="OOM"):
        gpu.init_request("big", [{"key": torch.randn(200, 2, 64), "value": torch.randn(200, 2, 64)}])
    with pytest.raises(ValueError):
        create_attention_backend("cpu")


def test_row_reuse_and_shuffled_batches():
    """Requests freed and re-created (their device-table rows are reused),
    batches in shuffled order (the table is gathered, not sliced), contexts
    growing across block borders; every step against the restated
    CpuAttentionBackend."""
    g = torch.Generator().manual_seed(31)
    hq, hkv, d, dtype = 8, 2, 64, torch.bfloat16
    gpu = GpuAttentionBackend(num_blocks=256, block_size=16)
    cpu = CpuAttentionOracle()
    live = []
    next_id = 0

    def new_request(T):
        nonlocal next_id
        rid = f"r{next_id}"
        next_id += 1
        kv = [{"key": torch.randn(T, hkv, d, generator=g).to(dtype),
               "value": torch.randn(T, hkv, d, generator=g).to(dtype)}]
        assert gpu.init_request(rid, kv) == cpu.init_request(rid, kv) == T
        live.append(rid)

    for T in (3, 15, 16, 40, 0, 70):
        new_request(T)
    for step in range(40):
        if step % 9 == 4:  # free two requests, start three (rows reused)
            for rid in (live[1], live[3]):
                gpu.free_request(rid)
                cpu.free_request(rid)
                live.remove(rid)
            for T in (1, 33, 17):
                new_request(T)
        order = torch.randperm(len(live), generator=g).tolist()
        items = [{"request_id": live[i], "layer_idx": 0,
                  "query": torch.randn(1, hq, d, generator=g).to(dtype),
                  "key": torch.randn(1, hkv, d, generator=g).to(dtype),
                  "value": torch.randn(1, hkv, d, generator=g).to(dtype),
                  "score_scale": d ** -0.5} for i in order]
        for a, b in zip(gpu.decode_layer_batch(items), cpu.decode_layer_batch(items)):
            assert_attention_close(a, b, what=f"step {step}")
    for rid in live:
        assert gpu.get_context_len(rid) == cpu.get_context_len(rid)


class _LayerCache:
    """Stands in for one layer of a Hugging Face cache object."""

    def __init__(self, k, v):
        self.key_cache, self.value_cache = k, v


@pytest.mark.parametrize("layout", ["bhtd", "bthd"])
def test_init_from_hf_cache_matches_normalised_ingest(layout):
    """HF caches ingested in place (strided views, on the device) give the
    same pools, bit for bit, as the reference's normalised [T, H, D] path, and
    the same decode outputs as the restated CpuAttentionBackend."""
    g = torch.Generator().manual_seed(41)
    layers, B, hq, hkv, d, T_pad, T = 3, 2, 8, 2, 64, 37, 29
    dtype = torch.float16
    shape = (B, hkv, T_pad, d) if layout == "bhtd" else (B, T_pad, hkv, d)
    cache = [(torch.randn(shape, generator=g).to(dtype).cuda(),
              torch.randn(shape, generator=g).to(dtype).cuda()) for _ in range(layers)]
    hf = [_LayerCache(k, v) for k, v in cache[:2]] + [cache[2]]  # both entry forms

    def normalised(t):  # the reference's _normalize_*_cache for sequence 1
        t = t[1] if layout == "bthd" else t[1].permute(1, 0, 2)
        return t[:T].contiguous().cpu()

    initial = [{"key": normalised(k), "value": normalised(v)} for k, v in cache]
    a = GpuAttentionBackend(num_blocks=64, block_size=16)
    b = GpuAttentionBackend(num_blocks=64, block_size=16)
    cpu = CpuAttentionOracle()
    assert a.init_request_from_hf("r", hf, layout=layout, batch_index=1, seq_len=T) == T
    assert b.init_request("r", initial) == T
    assert cpu.init_request("r", initial) == T
    assert torch.equal(a.k_pools, b.k_pools) and torch.equal(a.v_pools, b.v_pools)
    for layer in range(layers):
        it = [{"request_id": "r", "layer_idx": layer,
               "query": torch.randn(1, hq, d, generator=g).to(dtype),
               "key": torch.randn(1, hkv, d, generator=g).to(dtype),
               "value": torch.randn(1, hkv, d, generator=g).to(dtype), "score_scale": 0.125}]
        assert_attention_close(a.decode_layer_batch(it)[0], cpu.decode_layer_batch(it)[0],
                               what=f"layer {layer}")
    assert a.get_context_len("r") == cpu.get_context_len("r") == T + 1


@pytest.mark.parametrize("knob", [{"resident_kv_dtype": "fp16"}, {"kv_dtype": "bf16"}])
def test_resident_kv_dtype_knob(knob):
    """fp32 payloads with the pools in fp16 / bf16 (the reference's
    resident_kv_dtype knob): outputs in fp32, equal to the restated
    CpuAttentionBackend fed the same values rounded to the pool dtype (the
    backend converts q, k and v to the pool dtype)."""
    g = torch.Generator().manual_seed(51)
    pool_dt = torch.float16 if "resident_kv_dtype" in knob else torch.bfloat16
    rnd = lambda t: t.to(pool_dt).float()
    hq, hkv, d, layers = 8, 2, 64, 2
    gpu = create_attention_backend("gpu", {"num_blocks": 64, "block_size": 16, **knob})
    cpu = CpuAttentionOracle()
    kv = [{"key": torch.randn(37, hkv, d, generator=g), "value": torch.randn(37, hkv, d, generator=g)}
          for _ in range(layers)]
    assert gpu.init_request("r", kv) == 37
    cpu.init_request("r", [{"key": rnd(x["key"]), "value": rnd(x["value"])} for x in kv])
    assert gpu.get_debug_info()["kv_dtype"] == str(pool_dt)
    for layer in range(layers):
        it = {"request_id": "r", "layer_idx": layer, "query": torch.randn(1, hq, d, generator=g),
              "key": torch.randn(1, hkv, d, generator=g), "value": torch.randn(1, hkv, d, generator=g),
              "score_scale": 0.125}
        got = gpu.decode_layer_batch([it])[0]
        ref = cpu.decode_layer_batch([{**it, "query": rnd(it["query"]), "key": rnd(it["key"]),
                                       "value": rnd(it["value"])}])[0]
        assert got.dtype == torch.float32
        assert_attention_close(got, ref, what=f"layer {layer}")


def test_many_requests_long_rows_mixed_batches():
    """More requests than the initial table rows (64) and rows wider than its
    initial width (64 blocks), so the device table and the host state grow;
    batches that mix layers and repeat a request (split into several
    launches, in order); payloads on the device in some steps."""
    g = torch.Generator().manual_seed(41)
    hq, hkv, d, dtype, layers = 8, 2, 64, torch.float16, 2
    gpu = GpuAttentionBackend(num_blocks=4096, block_size=16)
    cpu = CpuAttentionOracle()
    lens = [int(x) for x in torch.randint(0, 120, (80,), generator=g)]
    lens[3], lens[70] = 1100, 1023  # 69 and 64 blocks: past the initial width
    rids = [f"m{i}" for i in range(len(lens))]
    for rid, T in zip(rids, lens):
        kv = [{"key": torch.randn(T, hkv, d, generator=g).to(dtype),
               "value": torch.randn(T, hkv, d, generator=g).to(dtype)} for _ in range(layers)]
        assert gpu.init_request(rid, kv) == cpu.init_request(rid, kv) == T

    def item(rid, layer, dev):
        return {"request_id": rid, "layer_idx": layer,
                "query": torch.randn(1, hq, d, generator=g).to(dtype).to(dev),
                "key": torch.randn(1, hkv, d, generator=g).to(dtype).to(dev),
                "value": torch.randn(1, hkv, d, generator=g).to(dtype).to(dev),
                "score_scale": d ** -0.5}

    for step in range(18):
        dev = "cuda" if step % 4 == 1 else "cpu"
        if step % 3 == 2:
            # one call: layer 0 for all, a request repeated, then layer 1 for all
            items = [item(r, 0, dev) for r in rids] + [item(rids[5], 1, dev), item(rids[5], 1, dev)]
            items += [item(r, 1, dev) for r in rids if r != rids[5]]
            calls = [items]
        else:
            calls = [[item(r, layer, dev) for r in rids] for layer in range(layers)]
        for items in calls:
            got = gpu.decode_layer_batch(items)
            ref = cpu.decode_layer_batch([{k: (v.cpu() if torch.is_tensor(v) else v)
                                           for k, v in it.items()} for it in items])
            for a, b in zip(got, ref):
                assert a.device.type == dev.split(":")[0]
                assert_attention_close(a.cpu(), b, what=f"step {step}")
    for rid in rids:
        assert gpu.get_context_len(rid) == cpu.get_context_len(rid)
    assert gpu.tables.table.shape[0] >= 80 and gpu.tables.width >= 70


@pytest.mark.parametrize("kv_dtype,dtype", [(None, torch.bfloat16), ("fp32", torch.float32),
                                            ("fp8", torch.bfloat16)])
def test_packed_batch_equals_item_batch(kv_dtype, dtype):
    """decode_layer_packed (stacked payloads, host or device) returns exactly
    the rows decode_layer_batch returns for the same items, and leaves the
    pools, tables and context lengths in the same state."""
    g = torch.Generator().manual_seed(53)
    hq, hkv, d, layers, bs = 28, 4, 128, 2, 16
    kw = {"num_blocks": 512, "block_size": bs}
    if kv_dtype:
        kw["kv_dtype"] = kv_dtype
    a, b = GpuAttentionBackend(**kw), GpuAttentionBackend(**kw)
    lens = [0, 1, 15, 16, 17, 200, 513, 96]
    rids = [f"p{i}" for i in range(len(lens))]
    for rid, T in zip(rids, lens):
        kv = [{"key": torch.randn(T, hkv, d, generator=g).to(dtype),
               "value": torch.randn(T, hkv, d, generator=g).to(dtype)} for _ in range(layers)]
        assert a.init_request(rid, kv) == b.init_request(rid, kv) == T
    for step in range(3):
        dev = "cuda" if step == 1 else "cpu"
        order = rids[step:] + rids[:step]  # a different row order per step
        for layer in range(layers):
            q = torch.randn(len(order), hq, d, generator=g).to(dtype).to(dev)
            k = torch.randn(len(order), hkv, d, generator=g).to(dtype).to(dev)
            v = torch.randn(len(order), hkv, d, generator=g).to(dtype).to(dev)
            items = [{"request_id": r, "layer_idx": layer, "query": q[i:i + 1],
                      "key": k[i:i + 1], "value": v[i:i + 1], "score_scale": d ** -0.5}
                     for i, r in enumerate(order)]
            ref = a.decode_layer_batch(items)
            got = b.decode_layer_packed(order, layer, q, k, v, d ** -0.5)
            assert got.shape == (len(order), 1, hq, d) and got.dtype == dtype
            assert got.device.type == dev
            assert torch.equal(got, torch.stack(ref)), f"step {step} layer {layer}"
    assert torch.equal(a.k_pools, b.k_pools) and torch.equal(a.v_pools, b.v_pools)
    assert [a.get_context_len(r) for r in rids] == [b.get_context_len(r) for r in rids]
    assert all(a.get_context_len(r) == T + 3 for r, T in zip(rids, lens))
    with pytest.raises(ValueError, match="at most once"):
        b.decode_layer_packed([rids[0], rids[0]], 0, q[:2], k[:2], v[:2])
    with pytest.raises(KeyError):
        b.decode_layer_packed(["nope"], 0, q[:1], k[:1], v[:1])
    with pytest.raises(ValueError, match="one row per request"):
        b.decode_layer_packed(rids[:2], 0, q[:3], k[:2], v[:2])


@pytest.mark.parametrize("lens", [[15, 16, 31], [527, 528, 543]], ids=["fused", "split"])
def test_malformed_payload_leaves_state_unchanged(lens):
    """A decode call with a malformed payload (wrong kv-head count, a query
    whose heads are no multiple of the kv heads, a short key) raises and
    changes nothing: later valid steps, including ones that cross a block
    border and take a new block, still match the restated
    CpuAttentionBackend, and the context lengths agree. Contexts past 512
    tokens take the split decode, whose decode over the cached tokens is
    already queued when a key or value is found malformed."""
    g = torch.Generator().manual_seed(61)
    hq, hkv, d, dtype, bs = 8, 2, 64, torch.bfloat16, 16
    gpu = GpuAttentionBackend(num_blocks=128, block_size=bs)
    cpu = CpuAttentionOracle()
    # each request's next token opens a new block within two steps
    rids = [f"x{i}" for i in range(len(lens))]
    for rid, T in zip(rids, lens):
        kv = [{"key": torch.randn(T, hkv, d, generator=g).to(dtype),
               "value": torch.randn(T, hkv, d, generator=g).to(dtype)}]
        assert gpu.init_request(rid, kv) == cpu.init_request(rid, kv) == T

    def items(bad=None):
        out = []
        for i, rid in enumerate(rids):
            it = {"request_id": rid, "layer_idx": 0,
                  "query": torch.randn(1, hq, d, generator=g).to(dtype),
                  "key": torch.randn(1, hkv, d, generator=g).to(dtype),
                  "value": torch.randn(1, hkv, d, generator=g).to(dtype), "score_scale": 0.125}
            if bad is not None and i == len(rids) - 1:
                it[bad[0]] = bad[1]
            out.append(it)
        return out

    free0 = len(gpu.free_blocks)
    for bad in (("key", torch.randn(1, hkv + 1, d).to(dtype)),
                ("value", torch.randn(hkv, d - 8).to(dtype)),
                ("query", torch.randn(1, hq + 1, d).to(dtype))):
        with pytest.raises((ValueError, RuntimeError)):
            gpu.decode_layer_batch(items(bad))
        packed = {"query": torch.randn(len(rids), hq, d).to(dtype),
                  "key": torch.randn(len(rids), hkv, d).to(dtype),
                  "value": torch.randn(len(rids), hkv, d).to(dtype)}
        packed[bad[0]] = {"key": torch.randn(len(rids), hkv + 1, d),
                          "value": torch.randn(len(rids), hkv, d - 8),
                          "query": torch.randn(len(rids), hq + 1, d)}[bad[0]].to(dtype)
        with pytest.raises((ValueError, RuntimeError)):
            gpu.decode_layer_packed(rids, 0, packed["query"], packed["key"], packed["value"],
                                    0.125)
    assert len(gpu.free_blocks) == free0
    assert [gpu.get_context_len(r) for r in rids] == lens
    for step in range(3):
        it = items()
        for a, b in zip(gpu.decode_layer_batch(it), cpu.decode_layer_batch(it)):
            assert_attention_close(a, b, what=f"step {step} after the refused calls")
    assert [gpu.get_context_len(r) for r in rids] == [cpu.get_context_len(r) for r in rids]


def test_packed_strided_device_payloads():
    """Stacked device payloads that are strided views (a transposed buffer,
    head_dim not contiguous until copied) give the same rows as the
    contiguous ones."""
    g = torch.Generator().manual_seed(62)
    hq, hkv, d, dtype = 8, 2, 128, torch.float16
    a = GpuAttentionBackend(num_blocks=64, block_size=16)
    b = GpuAttentionBackend(num_blocks=64, block_size=16)
    for be in (a, b):
        g2 = torch.Generator().manual_seed(63)
        for i, T in enumerate((5, 40)):
            be.init_request(f"s{i}", [{"key": torch.randn(T, hkv, d, generator=g2).to(dtype),
                                       "value": torch.randn(T, hkv, d, generator=g2).to(dtype)}])
    rids = ["s0", "s1"]
    q = torch.randn(2, hq, d, generator=g).to(dtype).cuda()
    k = torch.randn(2, hkv, d, generator=g).to(dtype).cuda()
    v = torch.randn(2, hkv, d, generator=g).to(dtype).cuda()
    qt = q.permute(2, 0, 1).contiguous().permute(1, 2, 0)  # same values, stride(2) != 1
    kt = k.permute(2, 0, 1).contiguous().permute(1, 2, 0)
    vt = v.permute(2, 0, 1).contiguous().permute(1, 2, 0)
    assert qt.stride(2) != 1 and torch.equal(qt, q)
    ref = a.decode_layer_packed(rids, 0, q, k, v, 0.1)
    got = b.decode_layer_packed(rids, 0, qt, kt, vt, 0.1)
    assert torch.equal(got, ref)
    assert torch.equal(a.k_pools, b.k_pools) and torch.equal(a.v_pools, b.v_pools)


@pytest.mark.parametrize("pool", ["bf16", "fp16"])
def test_fp32_queries_over_16bit_pools_unrounded_oracle(pool):
    """fp32 payloads over 16-bit pools: the backend computes with q rounded to
    the pool dtype and rounds the output to it before returning fp32. Checked
    against the oracle fed the fp32 query unrounded and the K/V values the
    pool holds (rounded, as any 16-bit resident KV is), output unrounded: the
    deviation stays inside the parity bar."""
    g = torch.Generator().manual_seed(64)
    pool_dt = {"bf16": torch.bfloat16, "fp16": torch.float16}[pool]
    rnd = lambda t: t.to(pool_dt).float()
    hq, hkv, d, T = 28, 4, 128, 300
    gpu = GpuAttentionBackend(num_blocks=64, block_size=16, kv_dtype=pool)
    kv = [{"key": torch.randn(T, hkv, d, generator=g), "value": torch.randn(T, hkv, d, generator=g)}]
    gpu.init_request("r", kv)
    keys, vals = rnd(kv[0]["key"]), rnd(kv[0]["value"])
    worst = 0.0
    for step in range(4):
        q = torch.randn(1, hq, d, generator=g)
        kn, vn = torch.randn(1, hkv, d, generator=g), torch.randn(1, hkv, d, generator=g)
        got = gpu.decode_layer("r", 0, q, kn, vn, d ** -0.5)
        keys, vals = torch.cat([keys, rnd(kn)]), torch.cat([vals, rnd(vn)])
        ref = oa.attend(q[0], keys, vals, d ** -0.5).unsqueeze(0)  # fp32 q, fp32 output
        assert got.dtype == torch.float32
        assert_attention_close(got, ref, what=f"{pool} pool step {step}")
        worst = max(worst, (got - ref).abs().max().item())
    print(f"fp32 queries over {pool} pools: max-abs vs the unrounded oracle {worst:.3e}")

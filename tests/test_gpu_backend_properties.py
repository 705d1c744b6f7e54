"""Property test of the "gpu" AttentionNode backend (hypothesis, GPU): random
batches of requests driven step by step beside the restated
CpuAttentionBackend. Prompt lengths straddle the 512-token switch between
the fused append + decode and the split decode (partials over the cached
tokens, then the merge that takes the new token), requests cross block
borders and take new blocks mid-run (with and without reserved tokens),
items arrive in random order, as host items, as a stacked host batch or as
device items, over fp32, fp16 and bf16 pools. Every output is compared with
the oracle's within the parity bar and every context length must agree."""
import pytest
import torch
from hypothesis import given, settings, strategies as st

from cloverinfer_amd.attention_backend import GpuAttentionBackend
from oracle.attention import CpuAttentionOracle
from tests.helpers import assert_attention_close

pytestmark = pytest.mark.gpu


@st.composite
def run(draw):
    hkv = draw(st.sampled_from([1, 2, 4]))
    g = draw(st.sampled_from([1, 4, 7]))
    d = draw(st.sampled_from([64, 128]))
    bs = draw(st.sampled_from([8, 16]))
    dtype = draw(st.sampled_from([torch.float32, torch.float16, torch.bfloat16]))
    lens = draw(st.lists(st.one_of(st.integers(0, 40), st.integers(500, 530),
                                   st.integers(531, 900)), min_size=1, max_size=5))
    layers = draw(st.integers(1, 2))
    steps = draw(st.integers(2, 4))
    reserve = draw(st.sampled_from([0, 3]))
    form = draw(st.sampled_from(["items", "packed", "device"]))
    seed = draw(st.integers(0, 10 ** 6))
    return hkv, g, d, bs, dtype, lens, layers, steps, reserve, form, seed


@settings(max_examples=30, deadline=None, derandomize=True)
@given(run())
def test_backend_random_runs_against_the_oracle(c):
    hkv, g, d, bs, dtype, lens, layers, steps, reserve, form, seed = c
    hq = hkv * g
    print(f"backend run hkv={hkv} g={g} d={d} bs={bs} {dtype} lens={lens} layers={layers} "
          f"steps={steps} reserve={reserve} form={form} seed={seed}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    nb = sum(-(-(T + steps + reserve + 1) // bs) + 1 for T in lens) + 4
    gpu = GpuAttentionBackend(num_blocks=nb, block_size=bs)
    cpu = CpuAttentionOracle()
    rids = [f"r{i}" for i in range(len(lens))]
    for rid, T in zip(rids, lens):
        kv = [{"key": torch.randn(T, hkv, d, generator=gen).to(dtype),
               "value": torch.randn(T, hkv, d, generator=gen).to(dtype)} for _ in range(layers)]
        assert gpu.init_request(rid, kv, decode_reserve_tokens=reserve) == T
        assert cpu.init_request(rid, kv) == T
    scale = d ** -0.5
    for step in range(steps):
        for layer in range(layers):
            order = torch.randperm(len(rids), generator=gen).tolist()
            items = [{"request_id": rids[i], "layer_idx": layer,
                      "query": torch.randn(1, hq, d, generator=gen).to(dtype),
                      "key": torch.randn(1, hkv, d, generator=gen).to(dtype),
                      "value": torch.randn(1, hkv, d, generator=gen).to(dtype),
                      "score_scale": scale} for i in order]
            ref = cpu.decode_layer_batch(items)
            if form == "packed":
                out = gpu.decode_layer_packed([it["request_id"] for it in items], layer,
                                              torch.cat([it["query"] for it in items]),
                                              torch.cat([it["key"] for it in items]),
                                              torch.cat([it["value"] for it in items]), scale)
                got = list(out.unbind(0))
            elif form == "device":
                dev = [{**it, "query": it["query"].cuda(), "key": it["key"].cuda(),
                        "value": it["value"].cuda()} for it in items]
                got = gpu.decode_layer_batch(dev)
            else:
                got = gpu.decode_layer_batch(items)
            for it, a, b in zip(items, got, ref):
                assert a.dtype == b.dtype, (a.dtype, b.dtype)
                assert_attention_close(a.cpu(), b, what=f"step {step} layer {layer} "
                                                       f"{it['request_id']}")
        assert [gpu.get_context_len(r) for r in rids] == [cpu.get_context_len(r) for r in rids]

"""Pins the CPU oracle: reference-test known answers, closed forms, float64
brute force and invariants. None of these checks retypes the oracle's
formula; each is chosen so that a dropped scale, a wrong head mapping, a
transposed operand or a wrong merge weight fails at least one of them."""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle.blocks import BlockBookkeeping

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def _pools(nb, bs, h, d, dtype=torch.float32):
    return torch.zeros(nb, bs, h, d, dtype=dtype), torch.zeros(nb, bs, h, d, dtype=dtype)


def test_kat_test_kernels_append_then_closed_form():
    kat = KATS["test_kernels_append"]
    bk = BlockBookkeeping(kat["num_blocks"], kat["block_size"])
    bk.allocate("req_1", 0)
    for _ in range(5):
        bk.append_slot("req_1")
    assert bk.context_lens["req_1"] == kat["context_len"]
    assert bk.block_tables["req_1"] == kat["block_table"]
    k, v = _pools(kat["num_blocks"], kat["block_size"], kat["num_heads"], kat["head_dim"])
    tbl = bk.block_tables["req_1"]
    for t in range(5):
        k[tbl[t // 4], t % 4] = t
        v[tbl[t // 4], t % 4] = t
    q = torch.ones(1, kat["num_heads"], kat["head_dim"])
    out = oa.paged_decode(q, k, v, [tbl], [5], kat["scale"])
    assert torch.allclose(out, torch.full_like(out, kat["expected_output_every_element"]),
                          rtol=0, atol=2e-6)


def test_kat_verify_attention_block_tables():
    kat = KATS["verify_attention_load_initial_kv"]
    bk = BlockBookkeeping(kat["num_blocks"], kat["block_size"])
    slots = bk.load_initial_kv("req_1", 5)
    assert bk.block_tables["req_1"] == kat["block_table_after_load"]
    assert bk.context_lens["req_1"] == kat["context_len_after_load"]
    assert slots == [9 * 4 + 0, 9 * 4 + 1, 9 * 4 + 2, 9 * 4 + 3, 8 * 4 + 0]
    bk.append_slot("req_1")
    assert bk.context_lens["req_1"] == kat["context_len_after_append"]
    assert bk.block_tables["req_1"] == kat["block_table_after_append"]


def test_kat_identical_rows_give_v():
    kat = KATS["verify_attention_kernel_vs_ref"]
    bk = BlockBookkeeping(kat["num_blocks"], kat["block_size"])
    bk.allocate("r", 0)
    g = torch.Generator().manual_seed(7)
    kk = torch.randn(4, 32, generator=g).half()
    vv = torch.randn(4, 32, generator=g).half()
    k, v = _pools(kat["num_blocks"], kat["block_size"], 4, 32, torch.float16)
    for _ in range(50):
        b, o = bk.append_slot("r")
        k[b, o] = kk
        v[b, o] = vv
    assert bk.block_tables["r"] == kat["block_table"]
    q = torch.randn(1, 4, 32, generator=g).half()
    out = oa.paged_decode(q, k, v, [bk.block_tables["r"]], [50], 1 / math.sqrt(32))
    assert torch.allclose(out[0], vv.float(), atol=1e-6, rtol=0)


def test_uniform_keys_give_mean_of_values():
    g = torch.Generator().manual_seed(1)
    L, hkv, G, d = 37, 3, 2, 16
    keys = torch.randn(1, hkv, d, generator=g).expand(L, hkv, d).contiguous()
    values = torch.randn(L, hkv, d, generator=g)
    q = torch.randn(hkv * G, d, generator=g)
    out = oa.attend(q, keys, values, 0.7)
    mean = values.double().mean(dim=0)  # [hkv, d]
    expect = mean.repeat_interleave(G, dim=0)
    assert torch.allclose(out.double(), expect, atol=1e-6)


def test_one_hot_score_selects_that_row():
    g = torch.Generator().manual_seed(2)
    L, h, d = 20, 2, 8
    q = torch.zeros(h, d)
    q[:, 0] = 1.0
    keys = torch.zeros(L, h, d)
    keys[13, :, 0] = 200.0  # score 200*scale dominates every other (0)
    values = torch.randn(L, h, d, generator=g)
    out = oa.attend(q, keys, values, 0.5)
    assert torch.allclose(out, values[13], atol=1e-6)


@pytest.mark.parametrize("hq,hkv,d,L", [(1, 1, 4, 1), (2, 2, 4, 5), (4, 2, 8, 9), (6, 2, 4, 7),
                                         (8, 1, 8, 3)])
def test_brute_force_fp64(hq, hkv, d, L):
    g = torch.Generator().manual_seed(hq * 100 + L)
    q = torch.randn(hq, d, generator=g)
    k = torch.randn(L, hkv, d, generator=g)
    v = torch.randn(L, hkv, d, generator=g)
    scale = 1.0 / math.sqrt(d)
    ref = oa.brute_attention_fp64(q.numpy(), k.numpy(), v.numpy(), scale)
    assert np.allclose(oa.attend(q, k, v, scale).numpy(), ref, atol=2e-6)
    assert np.allclose(oa.attend_repeat_kv(q, k, v, scale).numpy(), ref, atol=2e-6)


def test_gqa_head_mapping_is_h_div_group():
    # kv head 0 holds V = +1, kv head 1 holds V = -1: q heads 0,1 -> +1; 2,3 -> -1.
    L, d = 5, 4
    k = torch.randn(L, 2, d)
    v = torch.stack([torch.ones(L, d), -torch.ones(L, d)], dim=1)
    q = torch.randn(4, d)
    out = oa.attend(q, k, v, 1.0)
    assert torch.allclose(out[:2], torch.ones(2, d))
    assert torch.allclose(out[2:], -torch.ones(2, d))


@pytest.mark.parametrize("P", [1, 3, 16, 50, 64])
def test_split_merge_equals_single_pass(P):
    g = torch.Generator().manual_seed(P)
    L, hkv, G, d = 50, 2, 3, 8
    q = torch.randn(hkv * G, d, generator=g)
    k = torch.randn(L, hkv, d, generator=g) * 2
    v = torch.randn(L, hkv, d, generator=g)
    single = oa.attend(q, k, v, 0.9)
    assert torch.allclose(oa.split_attend(q, k, v, 0.9, P), single, atol=2e-6)


def test_partials_report_max_and_sum():
    q = torch.tensor([[1.0, 0.0]])
    k = torch.tensor([[[0.0, 0.0]], [[2.0, 0.0]]])  # scores 0, 2 (scale 1)
    v = torch.tensor([[[1.0, 3.0]], [[5.0, 7.0]]])
    ctx, m, l = oa.partial_attend(q, k, v, 1.0)
    assert m.item() == pytest.approx(2.0)
    assert l.item() == pytest.approx(1.0 + math.exp(-2.0))
    w0 = math.exp(-2.0) / (1 + math.exp(-2.0))
    assert ctx[0, 0].item() == pytest.approx(w0 * 1 + (1 - w0) * 5)


def test_chunked_prefill_equals_successive_decode_steps():
    g = torch.Generator().manual_seed(3)
    cached, new, hkv, G, d = 11, 6, 2, 2, 8
    k = torch.randn(cached + new, hkv, d, generator=g)
    v = torch.randn(cached + new, hkv, d, generator=g)
    q = torch.randn(new, hkv * G, d, generator=g)
    chunk = oa.chunked_prefill(q, k, v, 0.4)
    cpu = oa.CpuAttentionOracle()
    cpu.init_request("r", [{"key": k[:cached], "value": v[:cached]}])
    for i in range(new):
        step = cpu.decode_layer("r", 0, q[i], k[cached + i], v[cached + i], 0.4)
        assert torch.allclose(step[0], chunk[i], atol=1e-6)
    assert cpu.get_context_len("r") == cached + new


@pytest.mark.parametrize("cached,new,hkv,G,d", [(11, 6, 2, 2, 8), (0, 5, 1, 3, 4), (30, 1, 2, 1, 16)])
def test_masked_prefill_equals_successive_steps_and_fp64(cached, new, hkv, G, d):
    """The dense causal-masked formulation (the CPU baseline of chunked
    prefill) equals the successive decode steps and, row by row, the float64
    brute force over exactly the visible keys: a mask off by one (a row seeing
    its successor's key, or not its own) or a wrong head regrouping fails."""
    g = torch.Generator().manual_seed(cached + new)
    k = torch.randn(cached + new, hkv, d, generator=g)
    v = torch.randn(cached + new, hkv, d, generator=g)
    q = torch.randn(new, hkv * G, d, generator=g)
    dense = oa.chunked_prefill_masked(q, k, v, 0.3)
    assert torch.allclose(dense, oa.chunked_prefill(q, k, v, 0.3), atol=1e-5)
    for i in range(new):
        lim = cached + i + 1
        ref = oa.brute_attention_fp64(q[i].double().numpy(), k[:lim].double().numpy(),
                                      v[:lim].double().numpy(), 0.3)
        assert np.allclose(dense[i].double().numpy(), ref, atol=1e-5)


def test_cpu_oracle_protocol_semantics():
    cpu = oa.CpuAttentionOracle()
    kv = [{"key": torch.randn(3, 2, 4), "value": torch.randn(3, 2, 4)} for _ in range(2)]
    assert cpu.init_request("a", kv, decode_reserve_tokens=8) == 3
    with pytest.raises(ValueError):
        cpu.init_request("a", kv)
    with pytest.raises(KeyError):
        cpu.decode_layer("zz", 0, torch.randn(2, 4), torch.randn(2, 4), torch.randn(2, 4))
    q = torch.randn(1, 2, 4, dtype=torch.float16)
    out = cpu.decode_layer("a", 0, q, torch.randn(2, 4), torch.randn(2, 4), 0.5)
    assert out.shape == (1, 2, 4) and out.dtype == torch.float16
    assert cpu.get_context_len("a") == 3  # not the last layer yet
    cpu.decode_layer("a", 1, q, torch.randn(2, 4), torch.randn(2, 4), 0.5)
    assert cpu.get_context_len("a") == 4
    cpu.free_request("a")
    cpu.free_request("a")  # idempotent


def test_paged_gather_matches_contiguous():
    g = torch.Generator().manual_seed(4)
    bs, hkv, d, ctx = 4, 2, 8, 13
    table = [5, 0, 7, 2]
    contig_k = torch.randn(ctx, hkv, d, generator=g)
    contig_v = torch.randn(ctx, hkv, d, generator=g)
    k = torch.full((8, bs, hkv, d), float("nan"))
    v = torch.full((8, bs, hkv, d), float("nan"))
    for t in range(ctx):  # explicit scatter: slot of token t
        k[table[t // bs], t % bs] = contig_k[t]
        v[table[t // bs], t % bs] = contig_v[t]
    gk, gv = oa.gather_context(k, v, table, ctx)
    assert torch.equal(gk, contig_k) and torch.equal(gv, contig_v)
    q = torch.randn(1, hkv, d, generator=g)
    out = oa.paged_decode(q, k, v, [table], [ctx], 0.3)
    assert torch.isfinite(out).all()
    assert torch.allclose(out[0], oa.attend(q[0], contig_k, contig_v, 0.3))


def test_empty_context_gives_zeros():
    k, v = _pools(2, 4, 1, 8)
    out = oa.paged_decode(torch.randn(1, 1, 8), k, v, [[0]], [0], 1.0)
    assert torch.equal(out, torch.zeros(1, 1, 8))


def test_block_bookkeeping_errors_and_free_order():
    bk = BlockBookkeeping(4, 2)
    bk.allocate("a", 3)  # ceil(4/2) = 2 blocks
    assert bk.block_tables["a"] == [3, 2]
    with pytest.raises(ValueError):
        bk.allocate("a", 0)
    bk.allocate("b", 2)
    assert bk.block_tables["b"] == [1, 0]
    with pytest.raises(RuntimeError, match="OOM: Not enough blocks"):
        bk.allocate("c", 0)
    assert bk.append_slot("b") == (0, 0)  # position 2 -> block table[1], offset 0
    assert bk.append_slot("b") == (0, 1)
    with pytest.raises(RuntimeError, match="OOM during append"):
        bk.append_slot("b")
    bk.free("a")
    assert bk.free_blocks == [3, 2]
    bk.free("nope")
    tables, lens, mx = bk.kernel_inputs(["b"])
    assert tables == [[1, 0]] and lens == [4] and mx == 4


def test_fp8_codes_and_rounding_pinned():
    """The fp8 pool definition: torch's float8_e4m3fn decode equals the e4m3
    field formula on all 256 codes, and its encode (after the clamp) equals
    the brute-force nearest-even search on values that include every
    representable value, every midpoint between neighbours, signed zeros,
    subnormals, values that round to zero and out-of-range magnitudes."""
    import math
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    for c in range(256):
        want = oa.e4m3_value(c)
        assert (math.isnan(want) and math.isnan(codes[c].item())) or codes[c].item() == want
    finite = sorted({oa.e4m3_value(c) for c in range(256) if not math.isnan(oa.e4m3_value(c))})
    mids = [(a + b) / 2 for a, b in zip(finite, finite[1:])]
    g = torch.Generator().manual_seed(5)
    rand = (torch.randn(400, generator=g) * torch.tensor([0.003, 0.1, 3.0, 300.0]).repeat(100)).tolist()
    vals = finite + mids + [-0.0, 0.0, 2.0 ** -10, -2.0 ** -10, 3 * 2.0 ** -11, 500.0, -1e6] + rand
    x = torch.tensor(vals, dtype=torch.float32)
    got = oa.quantize_fp8(x.view(-1, 1, 1), torch.ones(1)).view(torch.uint8).flatten().tolist()
    for v, c in zip(vals, got):
        assert c == oa.e4m3_round(max(-448.0, min(448.0, v))), (v, hex(c))
    # scales divide, per kv head; NaN becomes code 0x7f; dequantize inverts exact codes
    s = torch.tensor([0.5, 4.0])
    q = oa.quantize_fp8(torch.tensor([[[1.0, float("nan")], [6.0, -1e9]]]), s)
    assert q.float()[0, 0, 0].item() == 2.0 and q.view(torch.uint8)[0, 0, 1].item() == 0x7F
    neg_nan = oa.quantize_fp8(-torch.tensor([[[float("nan")]]]), torch.ones(1))
    assert neg_nan.view(torch.uint8).item() == 0x7F
    assert q.float()[0, 1].tolist() == [1.5, -448.0]
    assert torch.equal(oa.dequantize_fp8(q[:, :, :1], s), torch.tensor([[[1.0], [6.0]]]))

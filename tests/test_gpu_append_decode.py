"""Fused append + decode (clv_paged_decode_append) against the two-call form
(reshape_and_cache with the same slots, then the decode schedule the fused
call runs: the single pass for contexts of at most 512 tokens and at most 16
query heads per kv head, the balanced decode otherwise) and the fp32 oracle:
pools bit for bit, outputs equal to the two-call result and within the
parity bar of the oracle. Three consecutive steps per case, so contexts
cross block borders; every slot not yet written holds NaN, so a read of a
stale new-token slot shows up in the output."""
import math

import pytest
import torch

from cloverinfer_amd import kernels
from oracle import attention as oa
from tests.helpers import assert_attention_close, make_paged_kv, padded_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _same_bits(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def _fused_schedule(hq, hkv, max_len):
    """paged_attention keyword arguments of the schedule the fused call runs."""
    if max_len <= 512 and hq // hkv <= 16:
        return {"partition_size": 0}
    return {"num_waves": kernels._native.load().clv_default_num_waves()}


@pytest.mark.parametrize("hq,hkv,d,bs,dtype", [
    (28, 4, 128, 16, torch.bfloat16),   # written inside the decode kernel
    (32, 8, 128, 32, torch.float16),    # idem, larger blocks
    (8, 8, 128, 16, torch.bfloat16),    # idem, one query head per kv head
    (32, 1, 128, 16, torch.bfloat16),   # 32 query heads per kv head: append kernel first
    (16, 2, 64, 16, torch.float16),     # head_dim 64: append kernel first
    (14, 2, 128, 8, torch.bfloat16),    # block_size 8: append kernel first
    (28, 4, 128, 16, torch.float32),    # fp32 pools: append kernel (4-byte rows), fp32 MFMA wave
    (16, 2, 64, 8, torch.float32),      # idem, head_dim 64, block_size 8
])
@pytest.mark.parametrize("long", [False, True], ids=["single-pass", "balanced"])
def test_fused_append_decode(hq, hkv, d, bs, dtype, long):
    # 0: no new token, zero output, pool untouched; 600: past the single
    # pass's range, so the call takes the balanced decode
    ctx0 = [1, 15, 16, 31, 600 if long else 100, 0, 47]
    steps = 3
    print(f"append+decode hq={hq} hkv={hkv} d={d} bs={bs} {dtype} long={long}", flush=True)
    cap = [c + steps for c in ctx0]
    k, v, tables = make_paged_kv(hq + d + bs, cap, hkv, d, bs, dtype, spare_blocks=2)
    # positions >= the starting context hold stale NaN until appended
    for t, c, n in zip(tables, ctx0, cap):
        for pos in range(c, n):
            blk, off = t[pos // bs], pos % bs
            k[blk, off] = float("nan")
            v[blk, off] = float("nan")
    kf, vf = k.to(DEV), v.to(DEV)          # fused
    ku, vu = k.clone().to(DEV), v.clone().to(DEV)  # two-call form
    bt = padded_tables(tables).to(DEV)
    g = torch.Generator().manual_seed(7)
    scale = 1.0 / math.sqrt(d)
    ctx = list(ctx0)
    for step in range(steps):
        grow = [c + 1 if c0 > 0 else 0 for c, c0 in zip(ctx, ctx0)]
        q = torch.randn(len(ctx), hq, d, generator=g).to(dtype).to(DEV)
        kn = torch.randn(len(ctx), hkv, d, generator=g).to(dtype).to(DEV)
        vn = torch.randn(len(ctx), hkv, d, generator=g).to(dtype).to(DEV)
        lens = torch.tensor(grow, dtype=torch.int32, device=DEV)
        out_f = torch.empty_like(q)
        kernels.paged_attention_append(out_f, q, kf, vf, bt, lens, bs, max(grow), kn, vn,
                                       scale=scale)
        slots = [t[(c - 1) // bs] * bs + (c - 1) % bs if c > 0 else -1
                 for t, c in zip(tables, grow)]
        kernels.reshape_and_cache(kn, vn, ku, vu, torch.tensor(slots, dtype=torch.int64, device=DEV))
        out_u = torch.empty_like(q)
        kernels.paged_attention(out_u, q, ku, vu, bt, lens, bs, max(grow), scale=scale,
                                **_fused_schedule(hq, hkv, max(grow)))
        torch.cuda.synchronize()
        assert _same_bits(kf, ku) and _same_bits(vf, vu), f"pools differ at step {step}"
        assert torch.equal(out_f, out_u), f"fused output differs from the two-call form, step {step}"
        ref = oa.paged_decode(q.cpu(), ku.cpu(), vu.cpu(), tables, grow, scale)
        assert_attention_close(out_f.cpu(), ref, what=f"step {step}")
        assert torch.equal(out_f[5].float().cpu(), torch.zeros(hq, d))
        ctx = grow


@pytest.mark.parametrize("num_waves", [0, 1024], ids=["single-pass", "balanced"])
def test_fused_append_out_of_range_positions(num_waves):
    """Contexts past max_context_len and block-table entries outside the pool
    append nothing (as the slot form with a skipped slot would), in the
    single-pass and the balanced form of the call."""
    hq, hkv, d, bs, dtype = 8, 2, 128, 16, torch.bfloat16
    k, v, tables = make_paged_kv(3, [40, 40], hkv, d, bs, dtype, spare_blocks=1)
    tables[1][2] = 10_000  # position 32.. of sequence 1 maps outside the pool
    kf, vf = k.clone().to(DEV), v.clone().to(DEV)
    bt = padded_tables(tables).to(DEV)
    q = torch.randn(2, hq, d).to(dtype).to(DEV)
    kn = torch.randn(2, hkv, d).to(dtype).to(DEV)
    vn = torch.randn(2, hkv, d).to(dtype).to(DEV)
    lens = torch.tensor([40, 40], dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    kernels.paged_attention_append(out, q, kf, vf, bt, lens, bs, 39, kn, vn,  # 40 > max_context_len
                                   num_waves=num_waves)
    kernels.paged_attention_append(out, q, kf, vf, bt, torch.tensor([0, 35], dtype=torch.int32,
                                                                     device=DEV), bs, 40, kn, vn,
                                   num_waves=num_waves)
    torch.cuda.synchronize()
    assert _same_bits(kf.cpu(), k) and _same_bits(vf.cpu(), v)


@pytest.mark.parametrize("long", [False, True], ids=["single-pass", "balanced"])
def test_fused_append_strided_new_rows_and_reused_launch(long):
    """New K/V rows given as transposed views (head-major storage) and with
    different strides for key and value: the launch copies them to
    contiguous rows and holds the copies until its kernels have read them.
    The same launch, re-pointed with update() and replayed through bind(),
    writes the next step's rows; pools and outputs equal the two-call form."""
    hq, hkv, d, bs, dtype = 28, 4, 128, 16, torch.bfloat16
    ctx0 = [40, 700 if long else 90, 17]
    cap = [c + 2 for c in ctx0]
    k, v, tables = make_paged_kv(91, cap, hkv, d, bs, dtype, spare_blocks=2)
    kf, vf = k.to(DEV), v.to(DEV)
    ku, vu = k.clone().to(DEV), v.clone().to(DEV)
    bt = padded_tables(tables).to(DEV)
    g = torch.Generator().manual_seed(92)
    scale = d ** -0.5
    launch = None
    for step in range(2):
        lens_h = [c + step for c in ctx0]
        lens = torch.tensor(lens_h, dtype=torch.int32, device=DEV)
        q = torch.randn(3, hq, d, generator=g).to(dtype).to(DEV)
        # key: [hkv, S, d] storage seen as [S, hkv, d]; value contiguous
        kn = torch.randn(hkv, 3, d, generator=g).to(dtype).to(DEV).transpose(0, 1)
        vn = torch.randn(3, hkv, d, generator=g).to(dtype).to(DEV)
        assert kn.stride() != vn.stride()
        out_f = torch.empty_like(q)
        if launch is None:
            launch = kernels.AppendDecodeLaunch(out_f, q, kf, vf, bt, lens, bs, max(lens_h), kn,
                                                vn, scale=scale)
            launch.launch()
        else:
            launch.update(out_f, q, bt, lens, max(lens_h), kn, vn)
            call = launch.bind()
            del kn, vn  # the launch holds the contiguous copies it reads
            junk = torch.full((64, hkv, d), float("nan"), dtype=dtype, device=DEV)
            kernels._native.check(call(), "clv_paged_decode_append")
            del junk
        slots = [t[(c - 1) // bs] * bs + (c - 1) % bs for t, c in zip(tables, lens_h)]
        knc = launch._key_new
        vnc = launch._value_new
        kernels.reshape_and_cache(knc, vnc, ku, vu,
                                  torch.tensor(slots, dtype=torch.int64, device=DEV))
        out_u = torch.empty_like(q)
        kernels.paged_attention(out_u, q, ku, vu, bt, lens, bs, max(lens_h), scale=scale,
                                **_fused_schedule(hq, hkv, max(lens_h)))
        torch.cuda.synchronize()
        assert _same_bits(kf, ku) and _same_bits(vf, vu), f"pools differ at step {step}"
        assert torch.equal(out_f, out_u), f"step {step}"
        ref = oa.paged_decode(q.cpu(), ku.cpu(), vu.cpu(), tables, lens_h, scale)
        assert_attention_close(out_f.cpu(), ref, what=f"strided rows, step {step}")

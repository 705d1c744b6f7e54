"""The split decode step (clv_balanced_partials over the cached tokens, then
clv_balanced_reduce_append merging in each sequence's new token and writing
its rows at the given slots) against the fused append + decode
(clv_paged_decode_append, balanced form) and the fp32 oracle: pools bit for
bit, outputs within the parity bar of both. Three consecutive steps per case,
so contexts cross block borders; every slot not yet written holds NaN, so a
read past the cached tokens shows up in the output."""
import math

import pytest
import torch

from cloverinfer_amd import kernels
from oracle import attention as oa
from tests.helpers import assert_attention_close, make_paged_kv, padded_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _same_bits(a, b):
    return torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("hq,hkv,d,bs,dtype", [
    (28, 4, 128, 16, torch.bfloat16),   # the GQA-7B node's shape
    (32, 8, 128, 32, torch.float16),
    (8, 8, 128, 16, torch.bfloat16),    # one query head per kv head
    (32, 1, 128, 16, torch.bfloat16),   # 32 query heads per kv head: two chunks
    (16, 2, 64, 16, torch.float16),     # head_dim 64
    (14, 2, 128, 8, torch.bfloat16),    # block_size 8
    (28, 4, 128, 16, torch.float32),    # fp32 pools
    (16, 2, 64, 8, torch.float32),
])
def test_split_append_decode(hq, hkv, d, bs, dtype):
    # 0: the new token alone; 600: past the single pass's range
    ctx0 = [1, 15, 16, 31, 600, 0, 47]
    steps = 3
    print(f"split append+decode hq={hq} hkv={hkv} d={d} bs={bs} {dtype}", flush=True)
    cap = [c + steps for c in ctx0]
    k, v, tables = make_paged_kv(hq + d + bs + 5, cap, hkv, d, bs, dtype, spare_blocks=2)
    for t, c, n in zip(tables, ctx0, cap):  # not yet written: NaN
        for pos in range(c, n):
            blk, off = t[pos // bs], pos % bs
            k[blk, off] = float("nan")
            v[blk, off] = float("nan")
    ks, vs = k.to(DEV), v.to(DEV)                   # split form
    kf, vf = k.clone().to(DEV), v.clone().to(DEV)   # fused form
    bt = padded_tables(tables).to(DEV)
    g = torch.Generator().manual_seed(11)
    scale = 1.0 / math.sqrt(d)
    waves = kernels._native.load().clv_default_num_waves()
    ctx = list(ctx0)
    launch = None
    for step in range(steps):
        new = [c + 1 for c in ctx]
        q = torch.randn(len(ctx), hq, d, generator=g).to(dtype).to(DEV)
        kn = torch.randn(len(ctx), hkv, d, generator=g).to(dtype).to(DEV)
        vn = torch.randn(len(ctx), hkv, d, generator=g).to(dtype).to(DEV)
        old_lens = torch.tensor(ctx, dtype=torch.int32, device=DEV)
        slots = torch.tensor([t[c // bs] * bs + c % bs for t, c in zip(tables, ctx)],
                             dtype=torch.int64, device=DEV)
        out_s = torch.empty_like(q)
        if launch is None:
            launch = kernels.SplitAppendDecode(out_s, q, ks, vs, bt, old_lens, bs, max(ctx),
                                               scale=scale)
        else:  # the same launch, re-pointed
            launch.update(out_s, q, bt, old_lens, max(ctx))
        launch.partials()
        launch.reduce(kn, vn, slots)
        out_f = torch.empty_like(q)
        kernels.paged_attention_append(out_f, q, kf, vf, bt,
                                       torch.tensor(new, dtype=torch.int32, device=DEV), bs,
                                       max(new), kn, vn, scale=scale, num_waves=waves)
        torch.cuda.synchronize()
        assert _same_bits(ks, kf) and _same_bits(vs, vf), f"pools differ at step {step}"
        ref = oa.paged_decode(q.cpu(), ks.cpu(), vs.cpu(), tables, new, scale)
        assert_attention_close(out_s.cpu(), ref, what=f"split, step {step}")
        assert_attention_close(out_s.cpu(), out_f.cpu(), what=f"split against fused, step {step}")
        if step == 0:  # a sequence with no cached token: its new value row
            g_ = hq // hkv
            assert torch.equal(out_s[5].cpu(), vn[5].repeat_interleave(g_, 0).cpu())
        ctx = new


def test_split_append_skipped_slots_and_strided_rows():
    """A negative slot or one past the pools writes nothing, the new token is
    attended all the same; new rows given as transposed (head-major) views
    are read through a contiguous copy the call holds until its kernel ran."""
    hq, hkv, d, bs, dtype = 28, 4, 128, 16, torch.bfloat16
    ctx = [700, 40, 300]
    k, v, tables = make_paged_kv(5, [c + 1 for c in ctx], hkv, d, bs, dtype, spare_blocks=1)
    kd, vd = k.clone().to(DEV), v.clone().to(DEV)
    bt = padded_tables(tables).to(DEV)
    g = torch.Generator().manual_seed(12)
    q = torch.randn(3, hq, d, generator=g).to(dtype).to(DEV)
    kn = torch.randn(hkv, 3, d, generator=g).to(dtype).to(DEV).transpose(0, 1)
    vn = torch.randn(hkv, 3, d, generator=g).to(dtype).to(DEV).transpose(0, 1)
    nslots = k.shape[0] * bs
    good = tables[2][ctx[2] // bs] * bs + ctx[2] % bs
    slots = torch.tensor([-1, nslots, good], dtype=torch.int64, device=DEV)
    out = torch.empty_like(q)
    sp = kernels.SplitAppendDecode(out, q, kd, vd, bt, torch.tensor(ctx, dtype=torch.int32,
                                                                    device=DEV), bs, max(ctx))
    with pytest.raises(RuntimeError):
        sp.reduce(kn, vn, slots)  # no partials yet
    sp.partials()
    with pytest.raises(ValueError):
        sp.reduce(kn.float(), vn.float(), slots)
    with pytest.raises(ValueError):
        sp.reduce(kn, vn, slots.to(torch.int32))
    sp.reduce(kn, vn, slots)
    torch.cuda.synchronize()
    kc, vc = kd.cpu(), vd.cpu()
    blk, off = divmod(good, bs)
    assert torch.equal(kc[blk, off], kn[2].cpu()) and torch.equal(vc[blk, off], vn[2].cpu())
    kc[blk, off], vc[blk, off] = k[blk, off], v[blk, off]
    assert _same_bits(kc, k) and _same_bits(vc, v), "a skipped slot was written"
    # the oracle over the cached tokens plus the new one, appended where the
    # skipped sequences would have had it
    kr, vr = k.clone(), v.clone()
    for s in range(3):
        b, o = divmod(tables[s][ctx[s] // bs] * bs + ctx[s] % bs, bs)
        kr[b, o], vr[b, o] = kn[s].cpu(), vn[s].cpu()
    ref = oa.paged_decode(q.cpu(), kr, vr, tables, [c + 1 for c in ctx], 1.0 / math.sqrt(d))
    assert_attention_close(out.cpu(), ref, what="skipped slots")


def test_mapped_device_address_and_direct_results():
    """Pinned host memory has a device address (the zero-copy result of the
    node backend's split decode relies on it), pageable memory has none, and
    the refused query leaves no error behind for the next launch's check."""
    from cloverinfer_amd import _native
    pinned = torch.empty(4096, dtype=torch.uint8, pin_memory=True)
    assert _native.mapped_device_address(pinned.data_ptr()) is not None
    pageable = torch.empty(4096, dtype=torch.uint8)
    assert _native.mapped_device_address(pageable.data_ptr()) is None
    # a reduce straight into pinned host memory, right after the refused query
    hq, hkv, d, bs, dtype = 28, 4, 128, 16, torch.bfloat16
    ctx = [700, 600]
    k, v, tables = make_paged_kv(21, [c + 1 for c in ctx], hkv, d, bs, dtype)
    kd, vd = k.to(DEV), v.to(DEV)
    bt = padded_tables(tables).to(DEV)
    q = torch.randn(2, hq, d).to(dtype).to(DEV)
    kn = torch.randn(2, hkv, d).to(dtype).to(DEV)
    vn = torch.randn(2, hkv, d).to(dtype).to(DEV)
    slots = torch.tensor([t[c // bs] * bs + c % bs for t, c in zip(tables, ctx)],
                         dtype=torch.int64, device=DEV)
    out = torch.empty_like(q)
    sp = kernels.SplitAppendDecode(out, q, kd, vd, bt, torch.tensor(ctx, dtype=torch.int32,
                                                                    device=DEV), bs, max(ctx))
    host = torch.full((2, hq, d), float("nan"), dtype=dtype, pin_memory=True)
    sp.partials()
    sp.reduce(kn, vn, slots, out_address=_native.mapped_device_address(host.data_ptr()))
    torch.cuda.synchronize()
    ref = oa.paged_decode(q.cpu(), kd.cpu(), vd.cpu(), tables, [c + 1 for c in ctx],
                          1.0 / math.sqrt(d))
    assert_attention_close(host, ref, what="merge into pinned host memory")


@pytest.mark.parametrize("slots", [2, 3])
def test_split_append_workgroups_per_cu(slots):
    """The split step at two or three workgroups per compute unit, where the
    balanced decode splits its steps in one piece per dispatch slot: the
    merge with the new token must find every segment's partials under that
    split (against the fused step at the same wave count and the oracle)."""
    hq, hkv, d, bs, dtype = 28, 4, 128, 16, torch.bfloat16
    ctx = [3000, 17, 811, 0, 4096, 256, 1500, 33] * 3
    waves = slots * kernels._native.load().clv_default_num_waves()
    print(f"split append slots={slots} waves={waves}", flush=True)
    k, v, tables = make_paged_kv(31, [c + 1 for c in ctx], hkv, d, bs, dtype)
    ks, vs = k.to(DEV), v.to(DEV)
    kf, vf = k.clone().to(DEV), v.clone().to(DEV)
    bt = padded_tables(tables).to(DEV)
    g = torch.Generator().manual_seed(13)
    q = torch.randn(len(ctx), hq, d, generator=g).to(dtype).to(DEV)
    kn = torch.randn(len(ctx), hkv, d, generator=g).to(dtype).to(DEV)
    vn = torch.randn(len(ctx), hkv, d, generator=g).to(dtype).to(DEV)
    slots = torch.tensor([t[c // bs] * bs + c % bs for t, c in zip(tables, ctx)],
                         dtype=torch.int64, device=DEV)
    new = [c + 1 for c in ctx]
    scale = 1.0 / math.sqrt(d)
    out_s = torch.empty_like(q)
    sp = kernels.SplitAppendDecode(out_s, q, ks, vs, bt, torch.tensor(ctx, dtype=torch.int32,
                                                                      device=DEV),
                                   bs, max(ctx), scale=scale, num_waves=waves)
    sp.partials()
    sp.reduce(kn, vn, slots)
    out_f = torch.empty_like(q)
    kernels.paged_attention_append(out_f, q, kf, vf, bt,
                                   torch.tensor(new, dtype=torch.int32, device=DEV), bs,
                                   max(new), kn, vn, scale=scale, num_waves=waves)
    torch.cuda.synchronize()
    assert _same_bits(ks, kf) and _same_bits(vs, vf)
    ref = oa.paged_decode(q.cpu(), ks.cpu(), vs.cpu(), tables, new, scale)
    assert_attention_close(out_s.cpu(), ref, what=f"split, {slots} slots")
    assert_attention_close(out_f.cpu(), ref, what=f"fused, {slots} slots")


def test_split_append_workspace_taken_in_between():
    """The partials live in the stream's workspace until the merge: another
    decode on the same stream in between makes reduce() raise instead of
    merging overwritten partials; a decode on another stream, or partials()
    run again, do not."""
    hq, hkv, d, bs, dtype = 28, 4, 128, 16, torch.bfloat16
    ctx = [700, 600, 900]
    k, v, tables = make_paged_kv(41, [c + 1 for c in ctx], hkv, d, bs, dtype)
    kd, vd = k.to(DEV), v.to(DEV)
    bt = padded_tables(tables).to(DEV)
    lens = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    q = torch.randn(3, hq, d).to(dtype).to(DEV)
    kn = torch.randn(3, hkv, d).to(dtype).to(DEV)
    vn = torch.randn(3, hkv, d).to(dtype).to(DEV)
    slots = torch.tensor([t[c // bs] * bs + c % bs for t, c in zip(tables, ctx)],
                         dtype=torch.int64, device=DEV)
    out = torch.empty_like(q)
    other = torch.empty_like(q)
    sp = kernels.SplitAppendDecode(out, q, kd, vd, bt, lens, bs, max(ctx))
    sp.partials()
    kernels.paged_attention(other, q, kd, vd, bt, lens, bs, max(ctx), num_waves=1024)
    with pytest.raises(RuntimeError, match="workspace"):
        sp.reduce(kn, vn, slots)
    sp.partials()  # again: its own lease
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # another stream has its own workspace
        kernels.paged_attention(other, q, kd, vd, bt, lens, bs, max(ctx), num_waves=1024)
    torch.cuda.current_stream().wait_stream(side)
    sp.reduce(kn, vn, slots)
    torch.cuda.synchronize()
    ref = oa.paged_decode(q.cpu(), kd.cpu(), vd.cpu(), tables, [c + 1 for c in ctx],
                          1.0 / math.sqrt(d))
    assert_attention_close(out.cpu(), ref, what="merge after a decode on another stream")

"""Slot-protocol oracle pins and the server's host side (message parsing,
validation, replies that need no kernel). No GPU needed."""
import io
import math
import struct

import numpy as np
import pytest
import torch

from cloverinfer_amd import kv_slot_server as ks
from oracle import attention as oa
from oracle import kvslot as ok


def _server():
    return ks.KVSlotServer(num_dpus=2, device="cpu")


# -- oracle pins ----------------------------------------------------------------

def test_message_bytes_follow_the_helper_structs():
    # kvslot_io_header_t + kvslot_slot_args_t (src/pim/upmem_kvslot/common.h:37-50):
    # little-endian u32 fields, magic 0x4B56534C ("LSVK" in memory), then the payload.
    k = torch.tensor([[[1.0, -2.0]]])
    v = torch.tensor([[[0.5, 4.0]]])
    msg = ok.msg_allocate(7, 16, k, v, 1)
    want = bytes.fromhex(
        "4c53564b" "01000000" "07000000" "00000000"                    # magic, ALLOCATE, slot 7, 0
        "10000000" "01000000" "01000000" "02000000" "01000000"         # cap 16, len 1, 1 head, dim 2, fp16
        "003c" "00c0"                                                  # K: 1.0, -2.0 as fp16
        "0038" "0044")                                                 # V: 0.5, 4.0 as fp16
    assert msg == want
    q = torch.tensor([[1.0, 0.0]])
    att = ok.msg_attention([(3, [0], 5, q, 0.5)], partial=True)
    assert att[:32] == struct.pack("<IIIIIIII", ok.MAGIC, 12, 0, 0, 1, 0, 0, 0)
    assert att[32:52] == struct.pack("<I", 3) + struct.pack("<IIIf", 1, 5, 2, 0.5)
    assert att[52:] == struct.pack("<I", 0) + struct.pack("<2f", 1.0, 0.0)


def test_row_attention_identity_is_the_backend_math():
    g = torch.Generator().manual_seed(5)
    keys = torch.randn(37, 4, 64, generator=g)
    values = torch.randn(37, 4, 64, generator=g)
    q = torch.randn(4, 64, generator=g)
    ctx, m, s = ok.row_attention(keys, values, range(4), q, 0.125)
    ref = oa.attend(q, keys, values, 0.125)
    assert np.allclose(ctx, ref.numpy(), atol=1e-6)
    brute = oa.brute_attention_fp64(q.double().numpy(), keys.double().numpy(),
                                    values.double().numpy(), 0.125)
    assert np.allclose(ctx, brute, atol=1e-5)


def test_row_attention_local_heads_pick_k_and_v():
    g = torch.Generator().manual_seed(6)
    keys = torch.randn(20, 3, 16, generator=g)
    values = torch.randn(20, 3, 16, generator=g)
    q = torch.randn(3, 16, generator=g)
    local = [2, 2, 0]
    ctx, _, _ = ok.row_attention(keys, values, local, q, 0.3)
    for r, h in enumerate(local):
        one = oa.brute_attention_fp64(q[r:r + 1].double().numpy(),
                                      keys[:, h:h + 1].double().numpy(),
                                      values[:, h:h + 1].double().numpy(), 0.3)
        assert np.allclose(ctx[r], one[0], atol=1e-5)


def test_row_stats_closed_forms():
    # Equal keys: every score is scale * q.k, so the row sum is the length and
    # the row max that score; one dominant key: the row sum tends to 1.
    q = torch.tensor([[1.0, 2.0]])
    keys = torch.tensor([[[0.5, 0.25]]]).repeat(9, 1, 1)
    values = torch.arange(18.0).view(9, 1, 2)
    ctx, m, s = ok.row_attention(keys, values, [0], q, 2.0)
    assert s[0] == pytest.approx(9.0, abs=1e-5)
    assert m[0] == pytest.approx(2.0 * (0.5 + 0.5), abs=1e-6)
    assert np.allclose(ctx[0], values[:, 0].mean(0).numpy(), atol=1e-5)
    keys2 = torch.zeros(9, 1, 2)
    keys2[4, 0] = torch.tensor([30.0, 0.0])
    ctx2, m2, s2 = ok.row_attention(keys2, values, [0], q, 1.0)
    assert m2[0] == pytest.approx(30.0)
    assert s2[0] == pytest.approx(1.0, abs=1e-6)
    assert np.allclose(ctx2[0], values[4, 0].numpy(), atol=1e-5)


def test_partials_merge_to_the_whole_slot():
    g = torch.Generator().manual_seed(7)
    keys = torch.randn(90, 2, 32, generator=g)
    values = torch.randn(90, 2, 32, generator=g)
    q = torch.randn(2, 32, generator=g)
    whole, _, _ = ok.row_attention(keys, values, [0, 1], q, 0.2)
    parts = [ok.row_attention(keys[a:b], values[a:b], [0, 1], q, 0.2)
             for a, b in ((0, 40), (40, 41), (41, 90))]
    assert np.allclose(ok.merge_partials(parts), whole, atol=1e-5)


def test_oracle_helper_validation():
    o = ok.SlotHelperOracle(num_dpus=1)
    k = torch.zeros(3, 2, 8)
    with pytest.raises(ok.OracleProtocolError):
        o.allocate(256, 4, k, k, 0)          # slot id beyond 1 unit
    with pytest.raises(ok.OracleProtocolError):
        o.allocate(0, 2, k, k, 0)            # 3 tokens > capacity 2
    assert o.allocate(0, 4, k, k, 0) == (4, 3, 2, 8, 0)
    assert o.append(0, k[:1], k[:1], 0) == (4, 4, 2, 8, 0)
    with pytest.raises(ok.OracleProtocolError):
        o.append(0, k[:1], k[:1], 0)         # full
    with pytest.raises(ok.OracleProtocolError):
        o.attention([(0, [0, 1], 2, torch.zeros(2, 8), 1.0)], False)   # window short of the slot


# -- server host side -------------------------------------------------------------

def _err(server, payload, match):
    with pytest.raises(ks.KVSlotProtocolError, match=match):
        server.request(payload)


def test_server_rejects_what_the_helper_rejects():
    s = _server()
    hdr = lambda cmd, sid=0: struct.pack("<IIII", ok.MAGIC, cmd, sid, 0)
    _err(s, struct.pack("<IIII", 0x1234, 1, 0, 0), "magic")
    for cmd in (6, 7, 8, 9, 10, 15, 99):
        _err(s, hdr(cmd), f"Unknown kvslot command {cmd}")
    k0 = torch.zeros(0, 2, 8)
    _err(s, ok.msg_allocate(512, 4, k0, k0, 0), "Invalid slot id 512")
    for cap, heads, dim in ((0, 2, 8), (257, 2, 8), (4, 0, 8), (4, 33, 8), (4, 2, 0), (4, 2, 129)):
        kk = torch.zeros(0, max(heads, 1), max(dim, 1))
        msg = (hdr(1) + struct.pack("<IIIII", cap, 0, heads, dim, 0))
        _err(s, msg, "Invalid slot shape")
    k5 = torch.zeros(5, 2, 8)
    _err(s, ok.msg_allocate(1, 4, k5, k5, 0), "Initial seq_len exceeds capacity")
    _err(s, ok.msg_append(3, k5[:1], k5[:1], 0), "Append on uninitialized slot 3")
    _err(s, ok.msg_simple(3, 9), "Readback on uninitialized slot 9")
    # an empty slot accepts no mismatched append
    s.request(ok.msg_allocate(4, 8, k0, k0, 1))
    _err(s, ok.msg_append(4, k5[:2], k5[:2], 1), "Append args mismatch")
    _err(s, ok.msg_append(4, torch.zeros(1, 3, 8), torch.zeros(1, 3, 8), 1), "Append args mismatch")
    _err(s, ok.msg_append(4, k5[:1], k5[:1], 0), "Append args mismatch")
    # attention batches
    q = torch.zeros(2, 8)
    _err(s, hdr(11) + struct.pack("<IIII", 0, 0, 0, 0), "num_slots=0")
    _err(s, hdr(11) + struct.pack("<IIII", 33, 0, 0, 0), "num_slots=33")
    _err(s, ok.msg_attention([(5, [0, 1], 0, q, 1.0)], False), "uninitialized slot 5")
    _err(s, ok.msg_attention([(4, [0, 1, 1], 0, torch.zeros(3, 8), 1.0)], False), "num_heads=3")
    _err(s, ok.msg_attention([(4, [0, 1], 0, torch.zeros(2, 9), 1.0)], False), "head_dim=9")
    _err(s, ok.msg_attention([(4, [0, 2], 0, q, 1.0)], False), "local head idx 2 for slot 4 at row 1")
    _err(s, ok.msg_attention([(4, [0], 0, q[:1], 1.0)], False), "shape mismatch at item 0")
    # a message cut short
    _err(s, ok.msg_allocate(6, 4, k5[:2], k5[:2], 0)[:-3], "Failed to read allocate payload")


def test_server_replies_without_kernels():
    s = _server()
    k0 = torch.zeros(0, 3, 80)
    assert s.request(ok.msg_allocate(1, 40, k0, k0, 1)) == struct.pack("<IIIII", 40, 0, 3, 80, 1)
    assert s.request(ok.msg_allocate(2, 256, torch.zeros(0, 32, 128), torch.zeros(0, 32, 128), 0)) \
        == struct.pack("<IIIII", 256, 0, 32, 128, 0)
    # pools: head_dim 80 pads to 128; 3 heads x ceil(40/16) blocks + 32 x 16 blocks
    assert s.slots[1].pool.head_dim == 128 and s.slots[1].blocks.shape == (3, 3)
    assert s.slots[2].blocks.shape == (32, 16)
    assert s.request(ok.msg_simple(3, 1)) == struct.pack("<IIIII", 40, 0, 3, 80, 1)
    stats = s.request(ok.msg_simple(5))
    rows = [struct.unpack_from("<IIIIII", stats, 24 * u) for u in range(2)]
    assert len(stats) == 48
    assert rows[0] == (0, 0, 0, 0, 1, 256 * 32 * 128)          # slot 2 on unit 0
    assert rows[1] == (0, 0, 0, 0, 1, (40 * 3 * 80 + 1) // 2)  # slot 1 on unit 1, fp16 packed
    topo = s.request(ok.msg_simple(14))
    assert struct.unpack_from("<IIII", topo) == (2, 1, 0, 0) and len(topo) == 16 + 2 * 16
    assert struct.unpack_from("<IIII", topo, 32) == (1, 0, 0, 0)
    # empty slots attend to nothing: zero context, row max -inf, row sum 0
    q = torch.ones(3, 80)
    reply = s.request(ok.msg_attention([(1, [0, 1, 2], 7, q, 0.5)], True))
    head, items = ok.parse_attention_reply(reply, [(3, 80)], True)
    assert head == (1, 0, 0, 0)
    args, ctx, m, sm = items[0]
    assert args == (40, 0, 3, 80, 1) and not ctx.any()
    assert np.isneginf(m).all() and not sm.any()
    prof = struct.unpack("<32Q", s.request(ok.msg_simple(13)))
    assert prof[0] == prof[8] == 1 and prof[3] == prof[11] == 1
    # free: 20 zero bytes, also for a slot that never existed
    assert s.request(ok.msg_simple(4, 1) + ok.msg_simple(4, 300)) == bytes(40)
    assert 1 not in s.slots
    # slot 1's blocks are back; slot 2 (32 heads x 16 blocks) still holds its own
    assert s.pools[128].num_blocks == 1024 and len(s.pools[128].free) == 1024 - 32 * 16


def test_serve_loop_status_and_stderr():
    s = _server()
    k0 = torch.zeros(0, 1, 8)
    out, err = io.BytesIO(), io.StringIO()
    rc = s.serve(io.BytesIO(ok.msg_allocate(0, 4, k0, k0, 0) + ok.msg_simple(4, 0)), out, err)
    assert rc == 0 and out.getvalue() == struct.pack("<IIIII", 4, 0, 1, 8, 0) + bytes(20)
    out, err = io.BytesIO(), io.StringIO()
    rc = s.serve(io.BytesIO(ok.msg_simple(3, 2) + ok.msg_simple(4, 0)), out, err)
    assert rc == 1 and out.getvalue() == b"" and "Readback on uninitialized slot 2" in err.getvalue()
    assert ks.main([]) == 1          # the helper's usage error without --stdio


def test_pool_head_dims():
    assert [ks.pool_head_dim(d) for d in (1, 8, 9, 64, 80, 96, 127, 128)] == \
        [8, 8, 16, 64, 128, 128, 128, 128]

"""The slot-protocol server on the GPU against the slot-helper oracle.

Readbacks are byte-exact (the pools hold the wire values exactly); contexts,
row maxima and row sums meet |got - ref| <= 2e-3 + 1e-2 |ref|.
"""
import os
import struct
import subprocess
import sys

import numpy as np
import pytest
import torch

from cloverinfer_amd import kv_slot_server as ks
from oracle import kvslot as ok

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _close(got, ref):
    got, ref = np.asarray(got, dtype=np.float64), np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape
    same = got == ref          # also equal infinities (row max of an empty slot)
    with np.errstate(invalid="ignore"):
        err = np.where(same, 0.0, np.abs(got - ref))
    assert (same | (err <= ATOL + RTOL * np.abs(ref))).all(), float(err.max())


class Session:
    """Drives the server and the oracle with the same messages."""

    def __init__(self, num_dpus=4):
        self.server = ks.KVSlotServer(num_dpus=num_dpus, device="cuda")
        self.oracle = ok.SlotHelperOracle(num_dpus=num_dpus)

    def allocate(self, sid, cap, k, v, code):
        got = self.server.request(ok.msg_allocate(sid, cap, k, v, code))
        assert struct.unpack("<IIIII", got) == self.oracle.allocate(sid, cap, k, v, code)

    def append(self, sid, k, v, code):
        got = self.server.request(ok.msg_append(sid, k, v, code))
        assert struct.unpack("<IIIII", got) == self.oracle.append(sid, k, v, code)

    def readback(self, sid):
        got = self.server.request(ok.msg_simple(3, sid))
        args, data = self.oracle.readback(sid)
        assert struct.unpack_from("<IIIII", got) == args
        assert got[20:] == data

    def attention(self, items, partial):
        reply = self.server.request(ok.msg_attention(items, partial))
        metas = [(q.shape[0], q.shape[1]) for _, _, _, q, _ in items]
        head, got = ok.parse_attention_reply(reply, metas, partial)
        assert head == (len(items), 0, 0, 0)
        ref = self.oracle.attention(items, partial)
        for (args, ctx, m, s), (rc, rm, rs), item in zip(got, ref, items):
            assert args == self.oracle.slots[item[0]].args()
            _close(ctx, rc)
            if partial:
                _close(m, rm)
                _close(s, rs)
        return got


def _kv(g, n, heads, dim, scale=1.0):
    return (torch.randn(n, heads, dim, generator=g) * scale,
            torch.randn(n, heads, dim, generator=g) * scale)


@pytest.mark.parametrize("code", [0, 1])
@pytest.mark.parametrize("heads,dim", [(1, 128), (4, 64), (7, 128), (32, 128), (3, 80), (2, 8), (5, 1)])
def test_allocate_append_readback_attend(code, heads, dim):
    g = torch.Generator().manual_seed(100 + heads * 7 + dim + code)
    s = Session()
    k, v = _kv(g, 37, heads, dim)
    s.allocate(5, 64, k, v, code)
    s.readback(5)
    for _ in range(3):
        s.append(5, *_kv(g, 1, heads, dim), code)
    s.readback(5)
    q = torch.randn(heads, dim, generator=g)
    scale = dim ** -0.5
    for partial in (False, True):
        s.attention([(5, list(range(heads)), 40, q, scale)], partial)


def test_full_slot_and_capacity_error():
    g = torch.Generator().manual_seed(3)
    s = Session(num_dpus=1)
    k, v = _kv(g, 255, 8, 128)
    s.allocate(255, 256, k, v, 1)
    s.append(255, *_kv(g, 1, 8, 128), 1)
    s.readback(255)
    with pytest.raises(ks.KVSlotProtocolError, match="capacity exceeded"):
        s.server.request(ok.msg_append(255, *_kv(g, 1, 8, 128), 1))
    q = torch.randn(8, 128, generator=g)
    s.attention([(255, list(range(8)), 256, q, 0.09)], True)


def test_batch_of_slots_across_pools_and_local_heads():
    """32 items over fp16 and fp32 pools and two head dims, windows larger
    than the slot, permuted and repeated local heads, a query shorter than
    the slot's head_dim, and slots at every length from 0 to 256."""
    g = torch.Generator().manual_seed(11)
    s = Session(num_dpus=8)
    items = []
    for i in range(32):
        code = i % 2
        heads = 1 + (i * 5) % 12
        dim = (64, 128, 96)[i % 3]
        n = (0, 1, 15, 16, 17, 100, 255, 256)[i % 8]
        sid = 7 * i + 3
        k, v = _kv(g, n, heads, dim, scale=1.5)
        s.allocate(sid, 256, k, v, code)
        local = [(h * 3 + i) % heads for h in range(heads)]
        qdim = dim if i % 5 else dim // 2
        q = torch.randn(heads, qdim, generator=g)
        items.append((sid, local, n + (i % 3) * 50, q, 0.1 + 0.01 * i))
    got = s.attention(items, True)
    assert len(got) == 32
    s.attention(items[:16], False)


def test_blocked_partials_merge_like_one_slot():
    """The reference splits a long context into 256-token block slots and
    merges their partials on the host; merged, they equal one attention."""
    g = torch.Generator().manual_seed(17)
    s = Session(num_dpus=2)
    heads, dim = 4, 128
    k, v = _kv(g, 700, heads, dim)
    bounds = [(0, 256), (256, 512), (512, 700)]
    for j, (a, b) in enumerate(bounds):
        s.allocate(10 + j, 256, k[a:b], v[a:b], 1)
    q = torch.randn(heads, dim, generator=g)
    items = [(10 + j, list(range(heads)), b - a, q, dim ** -0.5) for j, (a, b) in enumerate(bounds)]
    got = s.attention(items, True)
    merged = ok.merge_partials([(c, m, sm) for _, c, m, sm in got])
    whole, _, _ = ok.row_attention(k.half(), v.half(), range(heads), q, dim ** -0.5)
    _close(merged, whole)


def test_reallocate_and_free_recycle_blocks():
    g = torch.Generator().manual_seed(23)
    s = Session(num_dpus=1)
    for rnd in range(3):
        for sid in range(40):
            s.allocate(sid, 200, *_kv(g, 50 + sid, 6, 64), rnd % 2)
        for sid in range(0, 40, 3):
            s.readback(sid)
        for sid in range(40):
            s.server.request(ok.msg_simple(4, sid))
            s.oracle.free(sid)
    pool_sizes = {key: p.num_blocks for key, p in s.server.pools.items()}
    assert all(len(p.free) == p.num_blocks for p in s.server.pools.values()), pool_sizes


def test_helper_stand_in_over_pipes():
    """Started as the resident store starts its helper
    (src/core/resident_kv_store.py:203-210): the launcher script, --stdio,
    --num-dpus, binary messages over the pipes."""
    exe = os.path.join(REPO, "cloverinfer_amd", "kvslot", "build", "host_kvslot")
    g = torch.Generator().manual_seed(29)
    k, v = _kv(g, 30, 4, 128)
    q = torch.randn(4, 128, generator=g)
    msgs = (ok.msg_simple(14) + ok.msg_allocate(9, 64, k, v, 1)
            + ok.msg_append(9, *_kv(g, 1, 4, 128), 1)
            + ok.msg_attention([(9, [0, 1, 2, 3], 31, q, 0.088)], True)
            + ok.msg_simple(4, 9))
    env = dict(os.environ, PYTHON=sys.executable)
    proc = subprocess.run([exe, "--stdio", "--num-dpus", "2"], input=msgs, capture_output=True,
                          timeout=120, env=env)
    assert proc.returncode == 0, proc.stderr.decode()[-2000:]
    local = ks.KVSlotServer(num_dpus=2, device="cuda").request(msgs)
    out = proc.stdout
    assert len(out) == len(local)
    n_topo = 16 + 2 * 16
    assert out[:n_topo] == local[:n_topo]
    assert out[n_topo:n_topo + 40] == local[n_topo:n_topo + 40]    # allocate + append replies
    tail = n_topo + 40
    _, a = ok.parse_attention_reply(out[tail:-20], [(4, 128)], True)
    _, b = ok.parse_attention_reply(local[tail:-20], [(4, 128)], True)
    for x, y in zip(a[0][1:], b[0][1:]):
        assert np.array_equal(x, y)
    assert out[-20:] == bytes(20)
    bad = subprocess.run([exe, "--stdio"], input=ok.msg_simple(3, 0), capture_output=True,
                         timeout=120, env=env)
    assert bad.returncode == 1 and b"Readback on uninitialized slot 0" in bad.stderr

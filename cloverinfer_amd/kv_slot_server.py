"""The resident-KV slot protocol served from paged device pools.

The reference's UPMEM resident store keeps each KV slot (one request's K/V
for a group of heads of one layer, at most 256 tokens) in a helper process
that it drives over stdin/stdout with little-endian binary messages:

* client side: src/core/resident_kv_store.py:97-137 (commands, limits),
  :238-347 (slot commands), :348-427 (stats, profile, topology), :649-783
  (fused attention batches), :189-213 (how the helper is started);
* message structs: src/pim/upmem_kvslot/common.h:6-102;
* helper side: src/pim/upmem_kvslot/host_kvslot.c:812-839 (slot shape
  limits), :1140-1372 (allocate, append, readback, free), :1374-1425 (stats,
  profile, topology), :1780-1876 and :3332-3592 (attention batches),
  :3766-3844 (message loop, command line).

:class:`KVSlotServer` answers the same messages with every slot head kept as
its own list of blocks in paged device pools, and the attention batches run
on this library's decode kernel (split-K partials with one partition per
query row, so each row's softmax statistics come out with its context). The
store can start it in place of the helper binary, with the helper's command
line (a two-line launcher script is shown in the integration notes):

    python -m cloverinfer_amd.kv_slot_server --stdio --num-dpus N

Served commands: ALLOCATE, APPEND, READBACK, FREE, GET_STATS, GET_PROFILE,
GET_TOPOLOGY, QK_SOFTMAX_AV_BATCH, QK_SOFTMAX_AV_PARTIAL_BATCH. The unfused
PIM steps (QK_BATCH, AV, AV_BATCH, QK_SLOT_BATCH, SOFTMAX_AV_BATCH) end the
session the way the helper ends it on an unknown command. As in the helper,
any invalid message ends the session: the message goes to stderr and the
process exits with status 1, so the client sees its pipe close.

Numerics: a query row ``r`` with local head ``h = local_head_indices[r]``
attends to all ``seq_len`` tokens of slot head ``h`` (the helper requires
the window to cover the whole slot), ``softmax(score_scale * K_h q_r) V_h``
in fp32 as the reference's host slot store defines it
(src/core/resident_kv_store.py:1057-1094); the partial variant also returns
the row max (natural-log domain) and row sum the reference's merge consumes
(src/core/resident_kv_store.py:2486-2509). A query shorter than the slot's
head_dim uses the slot's leading dimensions, as there; the context keeps the
slot's head_dim. Slots of both wire dtypes live in fp32 pools (fp16 converts
to fp32 exactly and back on readback), so the attention runs on fp32
queries as the reference's host store computes it; head dims that the
kernels do not take (not a power of two) live in pools padded with zero
columns to the next power of two >= 8.
"""
from __future__ import annotations

import argparse
import io
import struct
import sys
import time
from dataclasses import dataclass
from typing import BinaryIO, Dict, List, Optional, Tuple

import numpy as np
import torch

MAGIC = 0x4B56534C
CMD_ALLOCATE = 1
CMD_APPEND = 2
CMD_READBACK = 3
CMD_FREE = 4
CMD_GET_STATS = 5
CMD_QK_BATCH = 6
CMD_AV = 7
CMD_AV_BATCH = 8
CMD_QK_SLOT_BATCH = 9
CMD_SOFTMAX_AV_BATCH = 10
CMD_QK_SOFTMAX_AV_BATCH = 11
CMD_QK_SOFTMAX_AV_PARTIAL_BATCH = 12
CMD_GET_PROFILE = 13
CMD_GET_TOPOLOGY = 14

DTYPE_FP32 = 0
DTYPE_FP16 = 1

# Slot shape limits of the helper (src/pim/upmem_kvslot/common.h:7-10).
MAX_HEADS = 32
MAX_HEAD_DIM = 128
MAX_CAPACITY = 256
MAX_SLOTS_PER_DPU = 256

HEADER = struct.Struct("<IIII")       # magic, command, slot_id, reserved
SLOT_ARGS = struct.Struct("<IIIII")   # capacity, seq_len, group_heads, head_dim, dtype_code
BATCH_ARGS = struct.Struct("<IIII")   # num_slots, reserved x3
ITEM_ARGS = struct.Struct("<IIIf")    # num_heads, window, head_dim, score_scale
STATS = struct.Struct("<IIIIII")
TOPOLOGY_ITEM = struct.Struct("<IIII")
PROFILE = struct.Struct("<32Q")

# Profile counter positions (src/core/resident_kv_store.py:371-404).
_P_QK_ROUNDS, _P_QK_BATCHED, _P_QK_ITEMS, _P_QK_BATCHED_ITEMS, _P_QK_MAX = 0, 1, 3, 4, 6
_P_AV_ROUNDS, _P_AV_BATCHED, _P_AV_ITEMS, _P_AV_BATCHED_ITEMS, _P_AV_MAX = 8, 9, 11, 12, 14
_P_QK_BATCHED_NS, _P_AV_BATCHED_NS = 16, 24


class KVSlotProtocolError(RuntimeError):
    """An invalid message: the helper would print it and exit with status 1."""


def elem_format(dtype_code: int) -> Tuple[int, torch.dtype]:
    """Bytes per element and element type of a slot's dtype code: fp16 for
    code 1, fp32 for every other code (host_kvslot.c:828-831)."""
    return (2, torch.float16) if dtype_code == DTYPE_FP16 else (4, torch.float32)


def packed_elems(logical: int, dtype_code: int) -> int:
    """Elements in the helper's 32-bit units (host_kvslot.c:833-839)."""
    return (logical + 1) // 2 if dtype_code == DTYPE_FP16 else logical


def pool_head_dim(head_dim: int) -> int:
    """Head dim of the pool a slot lives in: the next power of two >= 8."""
    d = 8
    while d < head_dim:
        d *= 2
    return d


class _Reader:
    def __init__(self, stream: BinaryIO):
        self.stream = stream

    def read(self, n: int, what: str) -> bytearray:
        buf = bytearray(n)
        view, got = memoryview(buf), 0
        while got < n:
            k = self.stream.readinto(view[got:])
            if not k:
                raise KVSlotProtocolError(f"Failed to read {what}")
            got += k
        return buf


class _Pool:
    """fp32 K and V pools ``[num_blocks, block_size, 1, head_dim]`` of one
    head_dim; grow by doubling, so block ids stay valid."""

    def __init__(self, head_dim: int, block_size: int, num_blocks: int, device: torch.device):
        self.head_dim, self.block_size = head_dim, block_size
        shape = (num_blocks, block_size, 1, head_dim)
        self.k = torch.zeros(shape, dtype=torch.float32, device=device)
        self.v = torch.zeros(shape, dtype=torch.float32, device=device)
        self.free: List[int] = list(range(num_blocks))

    @property
    def num_blocks(self) -> int:
        return self.k.shape[0]

    def take(self, n: int) -> List[int]:
        while len(self.free) < n:
            old = self.num_blocks
            self.k = torch.cat([self.k, torch.zeros_like(self.k)])
            self.v = torch.cat([self.v, torch.zeros_like(self.v)])
            self.free[:0] = range(old, 2 * old)
        return [self.free.pop() for _ in range(n)]

    def give(self, blocks: np.ndarray) -> None:
        self.free.extend(int(b) for b in blocks.ravel())


@dataclass
class _Slot:
    capacity: int
    seq_len: int
    group_heads: int
    head_dim: int
    dtype_code: int
    pool: _Pool
    blocks: np.ndarray  # int64 [group_heads, blocks per head]

    def args(self) -> bytes:
        return SLOT_ARGS.pack(self.capacity, self.seq_len, self.group_heads, self.head_dim,
                              self.dtype_code)

    def slots(self, t0: int, t1: int) -> np.ndarray:
        """Pool slot of (token t, head h) for t in [t0, t1), row order (t, h)."""
        bs = self.pool.block_size
        t = np.arange(t0, t1, dtype=np.int64)[:, None]
        h = np.arange(self.group_heads, dtype=np.int64)[None, :]
        return (self.blocks[h, t // bs] * bs + t % bs).reshape(-1)


class KVSlotServer:
    """Serves the slot protocol's messages from device pools.

    ``num_dpus`` is the helper's ``--num-dpus``: slot ids must stay below
    ``num_dpus * 256`` and GET_STATS / GET_TOPOLOGY report that many units.
    """

    def __init__(self, num_dpus: int = 1, device="cuda", block_size: int = 16,
                 initial_blocks: int = 1024):
        if num_dpus <= 0:
            raise ValueError("num_dpus must be positive")
        if block_size <= 0 or block_size & (block_size - 1):
            raise ValueError("block_size must be a power of two")
        self.num_dpus = int(num_dpus)
        self.device = torch.device(device)
        self.block_size = int(block_size)
        self.initial_blocks = int(initial_blocks)
        self.pools: Dict[int, _Pool] = {}
        self.slots: Dict[int, _Slot] = {}
        self.profile = [0] * 32

    # -- message loop -------------------------------------------------------

    def serve(self, fin: BinaryIO, fout: BinaryIO, errors: BinaryIO | None = None) -> int:
        """Answers messages until end of input (0) or an invalid message (1)."""
        reader = _Reader(fin)
        while True:
            head = bytearray(HEADER.size)
            got = 0
            while got < HEADER.size:
                k = fin.readinto(memoryview(head)[got:])
                if not k:
                    break
                got += k
            if got < HEADER.size:
                return 0
            try:
                reply = self.handle(head, reader)
            except KVSlotProtocolError as exc:
                err = errors if errors is not None else sys.stderr
                print(exc, file=err, flush=True)
                return 1
            fout.write(reply)
            fout.flush()

    def request(self, payload: bytes) -> bytes:
        """Answers every message in ``payload``; raises KVSlotProtocolError
        on the first invalid one."""
        fin = io.BytesIO(payload)
        reader = _Reader(fin)
        out = []
        while fin.tell() < len(payload):
            out.append(self.handle(reader.read(HEADER.size, "kvslot header"), reader))
        return b"".join(out)

    def handle(self, head: bytes, reader: _Reader) -> bytes:
        magic, cmd, slot_id, _ = HEADER.unpack(bytes(head))
        if magic != MAGIC:
            raise KVSlotProtocolError("Invalid kvslot magic")
        if cmd == CMD_ALLOCATE:
            return self._allocate(slot_id, reader)
        if cmd == CMD_APPEND:
            return self._append(slot_id, reader)
        if cmd == CMD_READBACK:
            return self._readback(slot_id)
        if cmd == CMD_FREE:
            return self._free(slot_id)
        if cmd == CMD_GET_STATS:
            return self._stats()
        if cmd == CMD_GET_PROFILE:
            return PROFILE.pack(*self.profile)
        if cmd == CMD_GET_TOPOLOGY:
            return BATCH_ARGS.pack(self.num_dpus, 1, 0, 0) + b"".join(
                TOPOLOGY_ITEM.pack(i, 0, 0, 0) for i in range(self.num_dpus))
        if cmd in (CMD_QK_SOFTMAX_AV_BATCH, CMD_QK_SOFTMAX_AV_PARTIAL_BATCH):
            return self._attention(reader, cmd == CMD_QK_SOFTMAX_AV_PARTIAL_BATCH)
        raise KVSlotProtocolError(f"Unknown kvslot command {cmd}")

    # -- slot commands ------------------------------------------------------

    def _check_id(self, slot_id: int, what: str) -> None:
        if slot_id >= self.num_dpus * MAX_SLOTS_PER_DPU:
            raise KVSlotProtocolError(f"Invalid slot id {slot_id} for {what}")

    def _pool(self, head_dim: int) -> _Pool:
        d = pool_head_dim(head_dim)
        pool = self.pools.get(d)
        if pool is None:
            pool = _Pool(d, self.block_size, self.initial_blocks, self.device)
            self.pools[d] = pool
        return pool

    def _release(self, slot_id: int) -> None:
        slot = self.slots.pop(slot_id, None)
        if slot is not None:
            slot.pool.give(slot.blocks)

    def _write(self, slot: _Slot, t0: int, n: int, kb: bytearray, vb: bytearray) -> None:
        from . import kernels

        pool, hd, dev = slot.pool, slot.head_dim, self.device
        rows = n * slot.group_heads
        wire = elem_format(slot.dtype_code)[1]
        k = torch.frombuffer(kb, dtype=wire).view(rows, 1, hd).to(dev).float()
        v = torch.frombuffer(vb, dtype=wire).view(rows, 1, hd).to(dev).float()
        if pool.head_dim != hd:
            pad = (0, pool.head_dim - hd)
            k, v = torch.nn.functional.pad(k, pad), torch.nn.functional.pad(v, pad)
        slots = torch.from_numpy(slot.slots(t0, t0 + n)).to(dev)
        kernels.reshape_and_cache(k, v, pool.k, pool.v, slots)

    def _allocate(self, slot_id: int, reader: _Reader) -> bytes:
        capacity, seq_len, heads, head_dim, code = SLOT_ARGS.unpack(
            bytes(reader.read(SLOT_ARGS.size, "allocate args")))
        self._check_id(slot_id, "allocate")
        if not (0 < capacity <= MAX_CAPACITY and 0 < heads <= MAX_HEADS
                and 0 < head_dim <= MAX_HEAD_DIM):
            raise KVSlotProtocolError(
                f"Invalid slot shape capacity={capacity} heads={heads} head_dim={head_dim}")
        self._release(slot_id)
        if seq_len > capacity:
            raise KVSlotProtocolError("Initial seq_len exceeds capacity")
        nbytes = seq_len * heads * head_dim * elem_format(code)[0]
        kb = reader.read(nbytes, "allocate payload")
        vb = reader.read(nbytes, "allocate payload")
        pool = self._pool(head_dim)
        per_head = -(-capacity // self.block_size)
        blocks = np.asarray(pool.take(heads * per_head), dtype=np.int64).reshape(heads, per_head)
        slot = _Slot(capacity, seq_len, heads, head_dim, code, pool, blocks)
        self.slots[slot_id] = slot
        if seq_len:
            self._write(slot, 0, seq_len, kb, vb)
        return slot.args()

    def _append(self, slot_id: int, reader: _Reader) -> bytes:
        _, seq_len, heads, head_dim, code = SLOT_ARGS.unpack(
            bytes(reader.read(SLOT_ARGS.size, "append args")))
        self._check_id(slot_id, "append")
        slot = self.slots.get(slot_id)
        if slot is None:
            raise KVSlotProtocolError(f"Append on uninitialized slot {slot_id}")
        if (seq_len != 1 or heads != slot.group_heads or head_dim != slot.head_dim
                or code != slot.dtype_code):
            raise KVSlotProtocolError(f"Append args mismatch for slot {slot_id}")
        if slot.seq_len + 1 > slot.capacity:
            raise KVSlotProtocolError(f"Slot {slot_id} capacity exceeded")
        nbytes = heads * head_dim * elem_format(code)[0]
        kb = reader.read(nbytes, "append payload")
        vb = reader.read(nbytes, "append payload")
        self._write(slot, slot.seq_len, 1, kb, vb)
        slot.seq_len += 1
        return slot.args()

    def _readback(self, slot_id: int) -> bytes:
        self._check_id(slot_id, "readback")
        slot = self.slots.get(slot_id)
        if slot is None:
            raise KVSlotProtocolError(f"Readback on uninitialized slot {slot_id}")
        if slot.seq_len == 0:
            return slot.args()
        pool, hd = slot.pool, slot.head_dim
        idx = torch.from_numpy(slot.slots(0, slot.seq_len)).to(self.device)
        k = pool.k.view(-1, pool.head_dim).index_select(0, idx)[:, :hd]
        v = pool.v.view(-1, pool.head_dim).index_select(0, idx)[:, :hd]
        kv = torch.stack([k, v]).to(elem_format(slot.dtype_code)[1]).cpu().contiguous()
        return slot.args() + kv.numpy().tobytes()

    def _free(self, slot_id: int) -> bytes:
        self._check_id(slot_id, "free")
        self._release(slot_id)
        return bytes(SLOT_ARGS.size)

    def _stats(self) -> bytes:
        """Per unit (slot_id % num_dpus): live slots and their elements in
        32-bit units. The pools grow on demand, so the free-range fields
        (next free element, free ranges, free elements, largest range) are 0."""
        live = [0] * self.num_dpus
        elems = [0] * self.num_dpus
        for sid, s in self.slots.items():
            u = sid % self.num_dpus
            live[u] += 1
            elems[u] += packed_elems(s.capacity * s.group_heads * s.head_dim, s.dtype_code)
        return b"".join(STATS.pack(0, 0, 0, 0, live[u], elems[u]) for u in range(self.num_dpus))

    # -- attention batches --------------------------------------------------

    def _attention(self, reader: _Reader, partial: bool) -> bytes:
        raw = bytes(reader.read(BATCH_ARGS.size, "qk-softmax-av batch args"))
        num_slots = BATCH_ARGS.unpack(raw)[0]
        if num_slots == 0 or num_slots > MAX_HEADS:
            raise KVSlotProtocolError(f"Invalid qk-softmax-av batch num_slots={num_slots}")
        items = []
        for idx in range(num_slots):
            slot_id = struct.unpack("<I", bytes(reader.read(4, f"qk-softmax-av slot id {idx}")))[0]
            heads, window, head_dim, scale = ITEM_ARGS.unpack(
                bytes(reader.read(ITEM_ARGS.size, f"qk-softmax-av item args {idx}")))
            self._check_id(slot_id, "qk slot batch")
            slot = self.slots.get(slot_id)
            if slot is None:
                raise KVSlotProtocolError(f"QK slot batch on uninitialized slot {slot_id}")
            if heads == 0 or heads > slot.group_heads or heads > MAX_HEADS:
                raise KVSlotProtocolError(
                    f"Invalid qk slot batch num_heads={heads} for slot {slot_id}")
            if head_dim == 0 or head_dim > slot.head_dim or head_dim > MAX_HEAD_DIM:
                raise KVSlotProtocolError(
                    f"Invalid qk slot batch head_dim={head_dim} for slot {slot_id}")
            window = min(window, slot.seq_len)
            local = np.frombuffer(reader.read(4 * heads, "qk slot batch payload"), dtype="<u4")
            q = np.frombuffer(reader.read(4 * heads * head_dim, "qk slot batch payload"),
                              dtype="<f4").reshape(heads, head_dim)
            bad = np.nonzero(local >= slot.group_heads)[0]
            if bad.size:
                r = int(bad[0])
                raise KVSlotProtocolError(
                    f"Invalid local head idx {int(local[r])} for slot {slot_id} at row {r}")
            if slot.seq_len != window or slot.group_heads != heads:
                raise KVSlotProtocolError(f"QK-softmax-av slot shape mismatch at item {idx}")
            items.append((slot, local.astype(np.int64), q, scale))

        started = time.perf_counter_ns()
        results = self._attend(items)
        ns = time.perf_counter_ns() - started
        p = self.profile
        for base, items_at, batched_items_at, max_at, ns_at in (
                (_P_QK_ROUNDS, _P_QK_ITEMS, _P_QK_BATCHED_ITEMS, _P_QK_MAX, _P_QK_BATCHED_NS),
                (_P_AV_ROUNDS, _P_AV_ITEMS, _P_AV_BATCHED_ITEMS, _P_AV_MAX, _P_AV_BATCHED_NS)):
            p[base] += 1
            p[base + 1] += 1
            p[items_at] += num_slots
            p[batched_items_at] += num_slots
            p[max_at] = max(p[max_at], num_slots)
            p[ns_at] += ns

        out = [raw]
        for (slot, _, _, _), (ctx, m, s) in zip(items, results):
            out.append(slot.args())
            out.append(ctx.tobytes())
            if partial:
                out.append(m.tobytes())
                out.append(s.tobytes())
        return b"".join(out)

    def _attend(self, items) -> List[Tuple[np.ndarray, np.ndarray, np.ndarray]]:
        """Context [heads, slot head_dim], row max and row sum (fp32) of every
        item; one decode launch per pool the batch touches."""
        results: List[Optional[tuple]] = [None] * len(items)
        by_pool: Dict[int, List[int]] = {}
        for i, (slot, _, _, _) in enumerate(items):
            by_pool.setdefault(id(slot.pool), []).append(i)
        for members in by_pool.values():
            pool = items[members[0]][0].pool
            ctx, m, s = self._attend_pool(pool, [items[i] for i in members])
            row = 0
            for i in members:
                slot, local, _, _ = items[i]
                n = len(local)
                results[i] = (np.ascontiguousarray(ctx[row:row + n, :slot.head_dim]),
                              np.ascontiguousarray(m[row:row + n]),
                              np.ascontiguousarray(s[row:row + n]))
                row += n
        return results

    def _attend_pool(self, pool: _Pool, items):
        from . import kernels

        rows = sum(len(local) for _, local, _, _ in items)
        d = pool.head_dim
        width = max(slot.blocks.shape[1] for slot, _, _, _ in items)
        q = np.zeros((rows, d), dtype=np.float32)
        tables = np.full((rows, width), -1, dtype=np.int32)
        lens = np.zeros(rows, dtype=np.int32)
        r = 0
        for slot, local, qi, scale in items:
            n = len(local)
            # score_scale is folded into the query: the kernel runs with scale 1.
            q[r:r + n, :qi.shape[1]] = qi * np.float32(scale)
            tables[r:r + n, :slot.blocks.shape[1]] = slot.blocks[local]
            lens[r:r + n] = slot.seq_len
            r += n
        ctx = np.zeros((rows, d), dtype=np.float32)
        m = np.full(rows, -np.inf, dtype=np.float32)
        s = np.zeros(rows, dtype=np.float32)
        max_len = int(lens.max())
        if max_len == 0:
            return ctx, m, s
        dev = self.device
        qd = torch.from_numpy(q).to(dev).view(rows, 1, d)
        out = torch.empty_like(qd)
        td = torch.from_numpy(tables).to(dev)
        ld = torch.from_numpy(lens).to(dev)
        a = kernels.decode_args(out, qd, pool.k, pool.v, td, ld, pool.block_size, max_len,
                                scale=1.0)
        part = 32 * -(-max_len // 32)
        ws = kernels.splitk_workspace(dev, kernels.workspace_bytes(a, part))
        kernels.paged_decode_partials(a, part, ws, torch.cuda.current_stream(dev).cuda_stream)
        # Workspace layout of one partition per row: fp32 contexts [rows, d],
        # then row maxima and row sums, each section 256-byte aligned.
        off_m = _round256(rows * d * 4)
        off_s = off_m + _round256(rows * 4)
        host = ws[:off_s + rows * 4].cpu().numpy()
        live = lens > 0
        ctx[live] = host[:rows * d * 4].view(np.float32).reshape(rows, d)[live]
        m[live] = host[off_m:off_m + rows * 4].view(np.float32)[live]
        s[live] = host[off_s:off_s + rows * 4].view(np.float32)[live]
        return ctx, m, s


def _round256(n: int) -> int:
    return (n + 255) // 256 * 256


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(
        description="Serve the resident-KV slot protocol on stdin/stdout from device pools.")
    ap.add_argument("--stdio", action="store_true", help="serve on stdin/stdout (required)")
    ap.add_argument("--num-dpus", type=int, default=1,
                    help="units the client addresses (slot ids < 256 * N)")
    ap.add_argument("--device", default="cuda")
    ap.add_argument("--block-size", type=int, default=16)
    args = ap.parse_args(argv)
    if not args.stdio:
        print(f"Usage: {sys.argv[0]} --stdio [--num-dpus N]", file=sys.stderr)
        return 1
    server = KVSlotServer(num_dpus=args.num_dpus, device=args.device,
                          block_size=args.block_size)
    return server.serve(sys.stdin.buffer, sys.stdout.buffer)


if __name__ == "__main__":
    sys.exit(main())

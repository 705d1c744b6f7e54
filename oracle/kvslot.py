"""CPU restatement of the resident-KV slot helper (test infrastructure only).

What one helper session does with the slot protocol's messages, in plain
Python/torch on the CPU: slot state and its validation follow
src/pim/upmem_kvslot/host_kvslot.c:812-839 (shape limits), :1140-1372
(allocate, append, readback, free) and :1780-1876, :3332-3420 (attention
item checks); the attention math follows the reference's host slot store,
src/core/resident_kv_store.py:1057-1094 (fp32 upcast, scores over the last
``window`` tokens of the row's local head, softmax, weighted V), with the
row max / row sum of the partial variant in the natural-log domain that
the merge at src/core/resident_kv_store.py:2486-2509 consumes.

Message encoders restate the client, src/core/resident_kv_store.py:268-347
and :649-783: they are how the tests talk to the server.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from typing import Dict, List, Sequence, Tuple

import numpy as np
import torch

MAGIC = 0x4B56534C
MAX_HEADS, MAX_HEAD_DIM, MAX_CAPACITY, MAX_SLOTS_PER_DPU = 32, 128, 256, 256


class OracleProtocolError(RuntimeError):
    pass


def wire_dtype(code: int) -> torch.dtype:
    """fp16 for code 1, fp32 otherwise (host_kvslot.c:828-831)."""
    return torch.float16 if code == 1 else torch.float32


# -- client-side message encoders (resident_kv_store.py:268-347, 649-783) ----

def _kv_bytes(t: torch.Tensor, code: int) -> bytes:
    return t.detach().cpu().to(wire_dtype(code)).contiguous().numpy().tobytes()


def msg_allocate(slot_id: int, capacity: int, k: torch.Tensor, v: torch.Tensor, code: int) -> bytes:
    seq_len, heads, head_dim = (int(x) for x in k.shape)
    return (struct.pack("<IIII", MAGIC, 1, slot_id, 0)
            + struct.pack("<IIIII", capacity, seq_len, heads, head_dim, code)
            + _kv_bytes(k, code) + _kv_bytes(v, code))


def msg_append(slot_id: int, k: torch.Tensor, v: torch.Tensor, code: int) -> bytes:
    n, heads, head_dim = (int(x) for x in k.shape)
    return (struct.pack("<IIII", MAGIC, 2, slot_id, 0)
            + struct.pack("<IIIII", 0, n, heads, head_dim, code)
            + _kv_bytes(k, code) + _kv_bytes(v, code))


def msg_simple(cmd: int, slot_id: int = 0) -> bytes:
    return struct.pack("<IIII", MAGIC, cmd, slot_id, 0)


def msg_attention(items: Sequence[Tuple[int, Sequence[int], int, torch.Tensor, float]],
                  partial: bool) -> bytes:
    """items: (slot_id, local_head_indices, window, queries [heads, head_dim], score_scale)."""
    parts = [struct.pack("<IIII", MAGIC, 12 if partial else 11, 0, 0),
             struct.pack("<IIII", len(items), 0, 0, 0)]
    for slot_id, local, window, q, scale in items:
        q = q.detach().cpu().to(torch.float32).contiguous()
        heads, head_dim = (int(x) for x in q.shape)
        parts.append(struct.pack("<I", slot_id))
        parts.append(struct.pack("<IIIf", heads, window, head_dim, float(scale)))
        parts.append(struct.pack(f"<{heads}I", *[int(i) for i in local]))
        parts.append(q.numpy().tobytes())
    return b"".join(parts)


def parse_slot_args(buf: bytes, off: int = 0) -> Tuple[Tuple[int, ...], int]:
    return struct.unpack_from("<IIIII", buf, off), off + 20


def parse_attention_reply(buf: bytes, metas: Sequence[Tuple[int, int]], partial: bool):
    """metas: (heads, head_dim) per item -> (echoed batch args, [(slot args,
    context, row max, row sum)]), as the client reads it."""
    head = struct.unpack_from("<IIII", buf, 0)
    off, out = 16, []
    for heads, head_dim in metas:
        args, off = parse_slot_args(buf, off)
        n = args[2] * args[3]
        ctx = np.frombuffer(buf, dtype="<f4", count=n, offset=off).reshape(args[2], args[3])
        off += 4 * n
        m = s = None
        if partial:
            m = np.frombuffer(buf, dtype="<f4", count=args[2], offset=off)
            s = np.frombuffer(buf, dtype="<f4", count=args[2], offset=off + 4 * args[2])
            off += 8 * args[2]
        out.append((args, ctx, m, s))
    if off != len(buf):
        raise OracleProtocolError(f"reply has {len(buf) - off} trailing bytes")
    return head, out


# -- the helper's slot state --------------------------------------------------

@dataclass
class OracleSlot:
    capacity: int
    seq_len: int
    heads: int
    head_dim: int
    code: int
    k: torch.Tensor  # [capacity, heads, head_dim], wire dtype
    v: torch.Tensor

    def args(self) -> Tuple[int, ...]:
        return (self.capacity, self.seq_len, self.heads, self.head_dim, self.code)


class SlotHelperOracle:
    """One helper session: slot state, validation and the attention math."""

    def __init__(self, num_dpus: int = 1):
        self.num_dpus = num_dpus
        self.slots: Dict[int, OracleSlot] = {}

    def _check_id(self, slot_id: int) -> None:
        if slot_id >= self.num_dpus * MAX_SLOTS_PER_DPU:
            raise OracleProtocolError(f"invalid slot id {slot_id}")

    def allocate(self, slot_id: int, capacity: int, k: torch.Tensor, v: torch.Tensor,
                 code: int) -> Tuple[int, ...]:
        """host_kvslot.c:1140-1210 (ensure_slot :812-826)."""
        self._check_id(slot_id)
        seq_len, heads, head_dim = (int(x) for x in k.shape)
        if not (0 < capacity <= MAX_CAPACITY and 0 < heads <= MAX_HEADS
                and 0 < head_dim <= MAX_HEAD_DIM):
            raise OracleProtocolError("invalid slot shape")
        self.slots.pop(slot_id, None)
        if seq_len > capacity:
            raise OracleProtocolError("initial seq_len exceeds capacity")
        dt = wire_dtype(code)
        kk = torch.zeros(capacity, heads, head_dim, dtype=dt)
        vv = torch.zeros(capacity, heads, head_dim, dtype=dt)
        kk[:seq_len] = k.to(dt)
        vv[:seq_len] = v.to(dt)
        slot = OracleSlot(capacity, seq_len, heads, head_dim, code, kk, vv)
        self.slots[slot_id] = slot
        return slot.args()

    def append(self, slot_id: int, k: torch.Tensor, v: torch.Tensor, code: int) -> Tuple[int, ...]:
        """host_kvslot.c:1226-1294: one token, same shape and dtype code."""
        self._check_id(slot_id)
        slot = self.slots.get(slot_id)
        if slot is None:
            raise OracleProtocolError("append on uninitialized slot")
        n, heads, head_dim = (int(x) for x in k.shape)
        if n != 1 or heads != slot.heads or head_dim != slot.head_dim or code != slot.code:
            raise OracleProtocolError("append args mismatch")
        if slot.seq_len + 1 > slot.capacity:
            raise OracleProtocolError("slot capacity exceeded")
        slot.k[slot.seq_len] = k[0].to(slot.k.dtype)
        slot.v[slot.seq_len] = v[0].to(slot.v.dtype)
        slot.seq_len += 1
        return slot.args()

    def readback(self, slot_id: int) -> Tuple[Tuple[int, ...], bytes]:
        """host_kvslot.c:1296-1348: args, then K and V [seq_len, heads, head_dim]."""
        self._check_id(slot_id)
        slot = self.slots.get(slot_id)
        if slot is None:
            raise OracleProtocolError("readback on uninitialized slot")
        data = (slot.k[:slot.seq_len].contiguous().numpy().tobytes()
                + slot.v[:slot.seq_len].contiguous().numpy().tobytes())
        return slot.args(), data

    def free(self, slot_id: int) -> None:
        self._check_id(slot_id)
        self.slots.pop(slot_id, None)

    def attention(self, items, partial: bool):
        """host_kvslot.c:1780-1876 and :3344-3420 checks; math of
        resident_kv_store.py:1057-1094. Returns [(context, row max, row sum)]."""
        if not 0 < len(items) <= MAX_HEADS:
            raise OracleProtocolError("invalid batch size")
        out = []
        for slot_id, local, window, q, scale in items:
            self._check_id(slot_id)
            slot = self.slots.get(slot_id)
            if slot is None:
                raise OracleProtocolError("qk on uninitialized slot")
            heads, head_dim = (int(x) for x in q.shape)
            if heads == 0 or heads > slot.heads or head_dim == 0 or head_dim > slot.head_dim:
                raise OracleProtocolError("invalid item shape")
            window = min(int(window), slot.seq_len)
            if any(int(h) >= slot.heads for h in local):
                raise OracleProtocolError("invalid local head idx")
            if slot.seq_len != window or slot.heads != heads:
                raise OracleProtocolError("slot shape mismatch")
            out.append(row_attention(slot.k[:slot.seq_len], slot.v[:slot.seq_len], local,
                                     q, scale))
        return out


def row_attention(keys: torch.Tensor, values: torch.Tensor, local: Sequence[int],
                  q: torch.Tensor, scale: float):
    """Per query row r: softmax(scale * K[:, h_r, :hd] q_r) V[:, h_r, :] in
    fp32, with its row max and row sum (resident_kv_store.py:1077-1092)."""
    heads, head_dim = q.shape
    length = keys.shape[0]
    ctx = torch.zeros(heads, keys.shape[2], dtype=torch.float32)
    m = torch.full((heads,), float("-inf"))
    s = torch.zeros(heads)
    if length == 0:
        return ctx.numpy(), m.numpy(), s.numpy()
    qf = q.float()
    for r, h in enumerate(local):
        k = keys[:, int(h), :head_dim].float()
        scores = torch.einsum("ld,d->l", k, qf[r]) * float(scale)
        w = torch.softmax(scores, dim=-1)
        ctx[r] = torch.einsum("l,ld->d", w, values[:, int(h), :].float())
        m[r] = scores.max()
        s[r] = torch.exp(scores - m[r]).sum()
    return ctx.numpy(), m.numpy(), s.numpy()


def merge_partials(parts: List[Tuple[np.ndarray, np.ndarray, np.ndarray]]) -> np.ndarray:
    """The reference's running merge of per-segment (context, row max, row
    sum) triples, resident_kv_store.py:2486-2509."""
    ctx, m, s = (torch.from_numpy(np.array(x, dtype=np.float32)) for x in parts[0])
    for c2, m2, s2 in parts[1:]:
        c2, m2, s2 = (torch.from_numpy(np.array(x, dtype=np.float32)) for x in (c2, m2, s2))
        mm = torch.maximum(m, m2)
        a, b = torch.exp(m - mm), torch.exp(m2 - mm)
        tot = s * a + s2 * b
        safe = torch.clamp(tot, min=1e-12)
        ctx = ctx * (s * a / safe).unsqueeze(1) + c2 * (s2 * b / safe).unsqueeze(1)
        m, s = mm, tot
    return ctx.numpy()

"""Paged KV-cache manager with the reference's block-allocation API.

Drop-in for ``KVCacheManager`` (src/core/memory_manager.py:18-239): same
constructor arguments, methods, public attributes (``k_cache``, ``v_cache``,
``free_blocks``, ``block_tables``, ``context_lens``, ``block_size``,
``num_heads``, ``head_dim``), allocation order, error classes and -1
padding. Additive only:

* ``num_kv_heads`` (default ``num_heads``): pools are
  ``[num_blocks, block_size, num_kv_heads, head_dim]`` and ``num_heads``
  query heads share them with the repeat_kv grouping;
* ``scale`` (default 1/sqrt(head_dim), the reference kernel's constant);
* bfloat16 pools;
* ``write_new_kv_batch`` and ``slot_mapping`` (one device launch for a batch);
* on a HIP device, ``attention`` reads a device-resident mirror of the block
  tables that allocate / append_slot / free keep up to date (one row write
  per request, one entry per new block) instead of the per-call host build
  that ``get_kernel_inputs`` keeps for callers that want the tensors.

Data movement and attention always run the HIP kernels through the C ABI;
on a CPU device the bookkeeping works but the data path raises. The
reference's private slow path ``_paged_attention_ref``, against which its
tests check the kernel, is plain torch on the device (an independent
computation) and is never called by ``attention``.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence

import numpy as np
import torch

from . import kernels
from .block_table import DeviceBlockTable


class KVCacheManager:
    def __init__(self, num_blocks: int, block_size: int, num_heads: int, head_dim: int,
                 dtype=torch.float32, device="cuda", num_kv_heads: Optional[int] = None,
                 scale: Optional[float] = None):
        if num_blocks <= 0 or block_size <= 0 or num_heads <= 0 or head_dim <= 0:
            raise ValueError("num_blocks, block_size, num_heads and head_dim must be positive")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_heads = num_heads
        self.num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if self.num_heads % self.num_kv_heads:
            raise ValueError("num_heads must be a multiple of num_kv_heads")
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        self.scale = 1.0 / math.sqrt(head_dim) if scale is None else float(scale)

        shape = (num_blocks, block_size, self.num_kv_heads, head_dim)
        self.k_cache = torch.zeros(shape, dtype=dtype, device=device)
        self.v_cache = torch.zeros(shape, dtype=dtype, device=device)

        # LIFO free stack, popped from the end (memory_manager.py:49).
        self.free_blocks: List[int] = list(range(num_blocks))
        self.block_tables: Dict[str, List[int]] = {}
        self.context_lens: Dict[str, int] = {}
        # Device mirror of block_tables for attention() (HIP pools only).
        self._dev_tables: Optional[DeviceBlockTable] = (
            DeviceBlockTable(torch.device(device)) if torch.device(device).type == "cuda" else None)
        self._dev_rows: Dict[str, int] = {}

    # ------------------------------------------------------------ bookkeeping
    def allocate(self, request_id: str, seq_len: int = 0) -> None:
        """Reserve ceil((seq_len + 1) / block_size) blocks (memory_manager.py:55-72)."""
        if request_id in self.block_tables:
            raise ValueError(f"Request {request_id} already exists")
        required = max(1, math.ceil((seq_len + 1) / self.block_size))
        if len(self.free_blocks) < required:
            raise RuntimeError("OOM: Not enough blocks")
        self.block_tables[request_id] = [self.free_blocks.pop() for _ in range(required)]
        self.context_lens[request_id] = seq_len
        if self._dev_tables is not None:
            self._dev_rows[request_id] = self._dev_tables.add(self.block_tables[request_id])

    def append_slot(self, request_id: str):
        """Advance the context by one token, taking a new block when the
        table is full; returns (physical block, offset) of the new token
        (memory_manager.py:95-121)."""
        current = self.context_lens[request_id]
        blocks = self.block_tables[request_id]
        if current >= len(blocks) * self.block_size:
            if not self.free_blocks:
                raise RuntimeError("OOM during append")
            blocks.append(self.free_blocks.pop())
            if self._dev_tables is not None:
                self._dev_tables.set(self._dev_rows[request_id], len(blocks) - 1, blocks[-1])
        self.context_lens[request_id] = current + 1
        return blocks[current // self.block_size], current % self.block_size

    def free(self, request_id: str) -> None:
        """Return the request's blocks in table order (memory_manager.py:134-143)."""
        blocks = self.block_tables.pop(request_id, None)
        if blocks is None:
            return
        self.free_blocks.extend(blocks)
        del self.context_lens[request_id]
        if self._dev_tables is not None:
            self._dev_tables.remove(self._dev_rows.pop(request_id))

    def slot_mapping(self, request_id: str, positions: Sequence[int]) -> List[int]:
        """Cache slots (block * block_size + offset) of token positions."""
        blocks = self.block_tables[request_id]
        bs = self.block_size
        return [blocks[p // bs] * bs + p % bs for p in positions]

    def get_kernel_inputs(self, request_ids: List[str]):
        """(block_tables int32 [S, max_blocks] padded with -1, context_lens
        int32 [S], max_context_len), as memory_manager.py:145-173; built on
        the host and copied with one transfer per tensor."""
        lens = [self.context_lens[r] for r in request_ids]
        tables = [self.block_tables[r] for r in request_ids]
        width = max((len(t) for t in tables), default=0)
        host = np.full((len(request_ids), width), -1, dtype=np.int32)
        for i, t in enumerate(tables):
            host[i, :len(t)] = t
        bt = torch.from_numpy(host).to(self.device, non_blocking=False)
        ctx = torch.tensor(lens, dtype=torch.int32).to(self.device)
        return bt, ctx, max(lens, default=0)

    # ------------------------------------------------------------ data path
    def _require_gpu(self, what: str) -> None:
        if torch.device(self.device).type != "cuda":
            raise RuntimeError(
                f"KVCacheManager.{what} runs on the HIP kernels; this manager's pools are on "
                f"{self.device} (there is no CPU fallback)"
            )

    def _write(self, slots: Sequence[int], k: torch.Tensor, v: torch.Tensor) -> None:
        if not len(slots):
            return
        k = k.to(device=self.device, dtype=self.dtype)
        v = v.to(device=self.device, dtype=self.dtype)
        sm = torch.tensor(list(slots), dtype=torch.int64).to(self.device)
        kernels.reshape_and_cache(k, v, self.k_cache, self.v_cache, sm)

    def load_initial_kv(self, request_id: str, k_data: torch.Tensor, v_data: torch.Tensor) -> None:
        """Allocate (if needed) and fill the blocks with prefill KV
        ``[seq_len, num_kv_heads, head_dim]`` (memory_manager.py:74-93), in
        one reshape_and_cache launch."""
        self._require_gpu("load_initial_kv")
        seq_len = k_data.shape[0]
        if request_id not in self.block_tables:
            self.allocate(request_id, seq_len)
        blocks = self.block_tables[request_id]
        capacity = len(blocks) * self.block_size
        n = min(seq_len, capacity)
        self._write(self.slot_mapping(request_id, range(n)), k_data[:n], v_data[:n])
        self.context_lens[request_id] = seq_len

    def write_new_kv(self, request_id: str, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append one token's KV ``[num_kv_heads, head_dim]`` or
        ``[1, num_kv_heads, head_dim]`` (memory_manager.py:123-132)."""
        self._require_gpu("write_new_kv")
        if k.dim() == 3:
            k = k.squeeze(0)
        if v.dim() == 3:
            v = v.squeeze(0)
        blk, off = self.append_slot(request_id)
        self._write([blk * self.block_size + off], k.unsqueeze(0), v.unsqueeze(0))

    def write_new_kv_batch(self, request_ids: Sequence[str], k: torch.Tensor,
                           v: torch.Tensor) -> None:
        """Append one token per request (``k``/``v`` ``[B, num_kv_heads, head_dim]``)
        with one launch; equal to ``write_new_kv`` per request in order.
        All or nothing: a batch that would run out of blocks raises the
        reference's OOM error before any request advances."""
        self._require_gpu("write_new_kv_batch")
        if k.shape[0] != len(request_ids) or v.shape[0] != len(request_ids):
            raise ValueError("k and v need one row per request id")
        if self._blocks_needed(request_ids) > len(self.free_blocks):
            raise RuntimeError("OOM during append")
        slots = []
        for rid in request_ids:
            blk, off = self.append_slot(rid)
            slots.append(blk * self.block_size + off)
        self._write(slots, k, v)

    def _blocks_needed(self, request_ids: Sequence[str]) -> int:
        """New blocks that appending one token per listed request (in order)
        takes from the free list; a request listed twice may need a block for
        its second token only. KeyError for an unknown request, as
        append_slot."""
        lens: Dict[str, int] = {}
        held: Dict[str, int] = {}
        need = 0
        for rid in request_ids:
            if rid not in lens:
                lens[rid] = self.context_lens[rid]
                held[rid] = len(self.block_tables[rid])
            if lens[rid] >= held[rid] * self.block_size:
                held[rid] += 1
                need += 1
            lens[rid] += 1
        return need

    def _decode(self, q: torch.Tensor, request_ids: List[str],
                partition_size: Optional[int]) -> torch.Tensor:
        """Paged decode of ``q`` over the requests' contexts; the result has
        q's dtype and device (the kernels compute in the pool dtype)."""
        self._require_gpu("attention")
        lens = [self.context_lens[r] for r in request_ids]
        block_tables = self._dev_tables.rows([self._dev_rows[r] for r in request_ids])
        ctx_lens = torch.tensor(lens, dtype=torch.int32).to(self.device)
        max_len = max(lens, default=0)
        qk = q.to(device=self.device, dtype=self.dtype)
        if not qk.is_contiguous():
            qk = qk.contiguous()
        out = torch.empty_like(qk)
        kernels.paged_attention(out, qk, self.k_cache, self.v_cache, block_tables, ctx_lens,
                                self.block_size, max_len, scale=self.scale,
                                partition_size=partition_size)
        if out.dtype != q.dtype or out.device != q.device:
            out = out.to(device=q.device, dtype=q.dtype)
        return out

    def attention(self, q: torch.Tensor, request_ids: List[str],
                  partition_size: Optional[int] = None) -> torch.Tensor:
        """Paged decode for ``q [num_seqs, num_heads, head_dim]`` (memory_manager.py:175-190).

        Returns a tensor like ``q`` (its dtype and device), as the reference's
        ``out = torch.empty_like(q)``. A query whose dtype differs from the
        pool dtype is converted to it first, and the result back to q's dtype.
        ``partition_size``: None picks the schedule (see
        ``kernels.paged_attention``)."""
        return self._decode(q, request_ids, partition_size)

    def _paged_attention_ref(self, q: torch.Tensor, request_ids: List[str]) -> torch.Tensor:
        """The reference's second, slow path for the same attention
        (memory_manager.py:192-239; tests/verify_attention.py:88-136 checks
        the kernel against it), an independent computation in plain torch on
        the pools' device: per request, gather its blocks, view them as
        ``[n_blocks * block_size, num_kv_heads, head_dim][:context_len]``,
        then ``softmax(q K^T * scale) V`` with query head h on kv head
        ``h // (num_heads // num_kv_heads)``. The reference computes in q's
        dtype; this computes in fp32 (never less accurate, and it keeps
        torch's batched 16-bit products out) and returns q's dtype and device.
        ``attention`` never takes this path, and like the data path it runs
        on a HIP device only."""
        self._require_gpu("_paged_attention_ref")
        num_seqs, num_heads, head_dim = q.shape
        hkv = self.num_kv_heads
        g = num_heads // hkv
        dev = self.k_cache.device
        out = torch.empty_like(q)
        for i, rid in enumerate(request_ids):
            blocks = torch.tensor(self.block_tables[rid], dtype=torch.long, device=dev)
            ctx = self.context_lens[rid]
            k = self.k_cache[blocks].reshape(-1, hkv, head_dim)[:ctx].float()
            v = self.v_cache[blocks].reshape(-1, hkv, head_dim)[:ctx].float()
            qi = q[i].to(device=dev, dtype=torch.float32).reshape(hkv, g, head_dim)
            scores = torch.matmul(qi, k.permute(1, 2, 0).contiguous()) * self.scale  # [Hkv, G, L]
            weights = torch.softmax(scores, dim=-1)
            ctx_out = torch.matmul(weights, v.permute(1, 0, 2).contiguous())  # [Hkv, G, D]
            out[i] = ctx_out.reshape(num_heads, head_dim).to(device=q.device, dtype=q.dtype)
        return out

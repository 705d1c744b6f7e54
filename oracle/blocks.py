"""CPU restatement of KVCacheManager's block bookkeeping
(src/core/memory_manager.py:55-173). Test infrastructure only.

Pure Python lists and dicts, no tensors: the allocation order, the error
classes and messages, and the -1 padding are what the product's manager
must reproduce bit for bit.
"""
from __future__ import annotations

import math
from typing import Dict, List, Sequence, Tuple


class BlockBookkeeping:
    def __init__(self, num_blocks: int, block_size: int):
        self.num_blocks = num_blocks
        self.block_size = block_size
        # LIFO free stack: allocation pops from the end (memory_manager.py:49, :69).
        self.free_blocks: List[int] = list(range(num_blocks))
        self.block_tables: Dict[str, List[int]] = {}
        self.context_lens: Dict[str, int] = {}

    def allocate(self, request_id: str, seq_len: int = 0) -> None:
        """memory_manager.py:55-72: ceil((seq_len + 1) / bs) blocks, at least one."""
        if request_id in self.block_tables:
            raise ValueError(f"Request {request_id} already exists")
        required = math.ceil((seq_len + 1) / self.block_size)
        if required == 0:
            required = 1
        if len(self.free_blocks) < required:
            raise RuntimeError("OOM: Not enough blocks")
        self.block_tables[request_id] = [self.free_blocks.pop() for _ in range(required)]
        self.context_lens[request_id] = seq_len

    def load_initial_kv(self, request_id: str, seq_len: int) -> List[int]:
        """Bookkeeping of memory_manager.py:74-93; returns the slot of each of
        the seq_len tokens (block * bs + offset), in token order."""
        if request_id not in self.block_tables:
            self.allocate(request_id, seq_len)
        blocks = self.block_tables[request_id]
        slots: List[int] = []
        cursor = 0
        for blk in blocks:
            if cursor >= seq_len:
                break
            chunk = min(self.block_size, seq_len - cursor)
            slots.extend(blk * self.block_size + off for off in range(chunk))
            cursor += chunk
        self.context_lens[request_id] = seq_len
        return slots

    def append_slot(self, request_id: str) -> Tuple[int, int]:
        """memory_manager.py:95-121."""
        cur = self.context_lens[request_id]
        blocks = self.block_tables[request_id]
        if cur >= len(blocks) * self.block_size:
            if not self.free_blocks:
                raise RuntimeError("OOM during append")
            blocks.append(self.free_blocks.pop())
        self.context_lens[request_id] += 1
        return blocks[cur // self.block_size], cur % self.block_size

    def free(self, request_id: str) -> None:
        """memory_manager.py:134-143: blocks return in table order."""
        if request_id not in self.block_tables:
            return
        self.free_blocks.extend(self.block_tables[request_id])
        del self.block_tables[request_id]
        del self.context_lens[request_id]

    def kernel_inputs(self, request_ids: Sequence[str]):
        """memory_manager.py:145-173 as plain lists: (table padded with -1 to
        the longest table, context lengths, max context length)."""
        lens = [self.context_lens[r] for r in request_ids]
        tables = [self.block_tables[r] for r in request_ids]
        width = max((len(t) for t in tables), default=0)
        padded = [list(t) + [-1] * (width - len(t)) for t in tables]
        return padded, lens, max(lens, default=0)

"""Device-resident, incrementally updated block tables.

The reference builds the kernel's block table on the host for every call
(``KVCacheManager.get_kernel_inputs``, src/core/memory_manager.py:145-173:
one padded row per request, then a host-to-device copy). Here every request
owns one row of a persistent int32 device table ``[rows, width]`` (-1
padded): a row is written once when the request is created, and a block
taken during decode costs one queued entry, applied to the device with the
next flush. A launch then uses a slice of the table when its requests hold
consecutive rows, or one device gather otherwise.

All device work is stream-ordered on the current stream, so table updates
and the kernels that read the table never race.
"""
from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np
import torch


class DeviceBlockTable:
    def __init__(self, device: torch.device, rows: int = 64, width: int = 64):
        self.device = torch.device(device)
        self.table = torch.full((max(1, rows), max(1, width)), -1, dtype=torch.int32,
                                device=self.device)
        self._free_rows: List[int] = list(range(self.table.shape[0] - 1, -1, -1))
        self._pending: List[Tuple[int, int, int]] = []  # (row, column, block)

    @property
    def width(self) -> int:
        return self.table.shape[1]

    def _grow(self, rows: int, width: int) -> None:
        r0, w0 = self.table.shape
        if rows <= r0 and width <= w0:
            return
        r1 = max(r0, rows if rows <= r0 else max(rows, 2 * r0))
        w1 = max(w0, width if width <= w0 else max(width, 2 * w0))
        t = torch.full((r1, w1), -1, dtype=torch.int32, device=self.device)
        t[:r0, :w0] = self.table
        self.table = t
        self._free_rows = list(range(r1 - 1, r0 - 1, -1)) + self._free_rows

    def add(self, blocks: Sequence[int]) -> int:
        """Give a new request a row holding ``blocks``; returns the row."""
        if not self._free_rows:
            self._grow(2 * self.table.shape[0], self.width)
        self._grow(self.table.shape[0], len(blocks))
        row = self._free_rows.pop()
        host = torch.full((self.width,), -1, dtype=torch.int32)
        if len(blocks):
            host[:len(blocks)] = torch.tensor(list(blocks), dtype=torch.int32)
        self.table[row].copy_(host)
        return row

    def set(self, row: int, column: int, block: int) -> None:
        """Queue ``table[row, column] = block`` (applied by the next flush)."""
        self._pending.append((row, column, block))

    def flush(self) -> None:
        """Apply the queued entries (one small host-to-device copy)."""
        upd = self.take_pending()
        if upd:
            self.apply(torch.tensor(upd, dtype=torch.int64).t().contiguous().to(self.device),
                       max(c for _, c, _ in upd))

    def pending_count(self) -> int:
        return len(self._pending)

    def requeue(self, upd: List[Tuple[int, int, int]]) -> None:
        """Put entries handed out by ``take_pending`` back in front of the
        queue (their upload did not happen)."""
        self._pending = list(upd) + self._pending

    def take_pending(self) -> List[Tuple[int, int, int]]:
        """Hand the queued entries to a caller that uploads them itself (with
        other data), then applies them with ``apply``."""
        upd, self._pending = self._pending, []
        return upd

    def flat_updates(self, upd: List[Tuple[int, int, int]]):
        """Host side of :meth:`apply_flat`: widens the table if a column is
        past its width and returns the entries as (int64 flat indices into
        the table, int32 blocks), numpy arrays to upload."""
        a = np.asarray(upd, dtype=np.int64)
        self._grow(self.table.shape[0], int(a[:, 1].max()) + 1)
        return a[:, 0] * self.width + a[:, 1], a[:, 2].astype(np.int32)

    def apply_flat(self, flat: torch.Tensor, blocks: torch.Tensor) -> None:
        """One scatter of uploaded :meth:`flat_updates` into the table."""
        self.table.view(-1).scatter_(0, flat, blocks)

    def apply(self, upd: torch.Tensor, max_column: int) -> None:
        """``upd``: int64 device tensor [3, P] of (row, column, block). One
        scatter into the flattened table (no host synchronisation)."""
        self._grow(self.table.shape[0], max_column + 1)
        flat = upd[0] * self.width + upd[1]
        self.table.view(-1).scatter_(0, flat, upd[2].to(torch.int32))

    def remove(self, row: int) -> None:
        """Release a row (it is rewritten whole when reused)."""
        self._pending = [p for p in self._pending if p[0] != row]
        self._free_rows.append(row)

    def rows_range(self, first: int, n: int) -> torch.Tensor:
        """The table of the consecutive rows ``first .. first + n - 1`` (a
        view). Flushes queued entries."""
        self.flush()
        return self.table[first:first + n]

    def rows(self, rows: Sequence[int], rows_dev: torch.Tensor | None = None) -> torch.Tensor:
        """The contiguous ``[len(rows), width]`` block table of these requests
        (a view when the rows are consecutive, else a device gather; pass the
        rows as a device tensor to save an upload). Flushes queued entries."""
        self.flush()
        n = len(rows)
        if n and list(rows) == list(range(rows[0], rows[0] + n)):
            return self.table[rows[0]:rows[0] + n]
        if rows_dev is None:
            rows_dev = torch.tensor(list(rows), dtype=torch.int64).to(self.device)
        return self.table.index_select(0, rows_dev)

"""DeviceBlockTable bookkeeping on the CPU (the same torch ops run on the
HIP device): rows are -1 padded copies of each request's block list, kept up
to date by queued single entries, across growth of rows and columns."""
import random

import torch

from cloverinfer_amd.block_table import DeviceBlockTable


def _expect(tables, rows, width):
    out = torch.full((len(rows), width), -1, dtype=torch.int32)
    for i, r in enumerate(rows):
        out[i, :len(tables[r])] = torch.tensor(tables[r], dtype=torch.int32)
    return out


def test_add_set_rows_and_growth():
    t = DeviceBlockTable(torch.device("cpu"), rows=2, width=2)
    rng = random.Random(0)
    tables = {}  # row -> block list
    for step in range(300):
        op = rng.random()
        if op < 0.2 or not tables:
            blocks = [rng.randrange(10_000) for _ in range(rng.randrange(0, 5))]
            tables[t.add(blocks)] = blocks
        elif op < 0.3:
            row = rng.choice(list(tables))
            t.remove(row)
            del tables[row]
        else:
            row = rng.choice(list(tables))
            blk = rng.randrange(10_000)
            t.set(row, len(tables[row]), blk)
            tables[row].append(blk)
        if step % 7 == 0 and tables:
            rows = rng.sample(list(tables), k=min(len(tables), 5))
            got = t.rows(rows)
            assert got.shape == (len(rows), t.width)
            assert torch.equal(got, _expect(tables, rows, t.width))
    rows = sorted(tables)
    assert torch.equal(t.rows(rows), _expect(tables, rows, t.width))


def test_consecutive_rows_are_a_view_and_reuse_is_lifo():
    t = DeviceBlockTable(torch.device("cpu"), rows=4, width=4)
    assert [t.add([i]) for i in range(3)] == [0, 1, 2]
    view = t.rows([0, 1, 2])
    assert view.data_ptr() == t.table.data_ptr()
    t.remove(1)
    assert t.add([7, 8]) == 1
    assert t.rows([1]).tolist() == [[7, 8, -1, -1]]


def test_uploaded_updates_match_queued_ones():
    t = DeviceBlockTable(torch.device("cpu"), rows=2, width=2)
    a, b = t.add([1, 2]), t.add([3])
    t.set(a, 2, 9)
    t.set(b, 1, 4)
    t.set(b, 2, 5)
    upd = t.take_pending()
    assert t.take_pending() == []
    t.apply(torch.tensor(upd, dtype=torch.int64).t().contiguous(), max(c for _, c, _ in upd))
    assert t.rows([a, b]).tolist() == [[1, 2, 9, -1], [3, 4, 5, -1]]


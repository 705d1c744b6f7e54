"""The node backend's native payload gather (cloverinfer_amd/host/node_gather.cpp),
on the CPU: rows copied exactly as torch.stack places them, and every
payload it cannot copy as is refused before anything is written."""
import os

import pytest
import torch

from cloverinfer_amd import _native, build


@pytest.fixture(scope="module")
def gather():
    if not os.path.exists(build.HOST_EXT_PATH):
        build.build_host_ext()
    mod = _native.load_host()
    assert mod is not None
    return mod


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(1, 28, 128), (4, 128), (12, 64)])
def test_rows_equal_torch_stack(gather, dtype, shape):
    g = torch.Generator().manual_seed(1)
    ts = [torch.randn(shape, generator=g).to(dtype) for _ in range(130)]
    ts[3] = torch.randn((2,) + shape, generator=g).to(dtype)[1]  # a view at an offset
    dst = torch.full((130, ts[0].numel()), float("nan"), dtype=dtype)
    assert gather.gather_rows(ts, dst)
    assert torch.equal(dst.view((130,) + shape), torch.stack(ts))


def test_refusals_write_nothing(gather):
    row = 4 * 128
    good = [torch.randn(4, 128) for _ in range(5)]
    bad_cases = {
        "dtype": torch.randn(4, 128, dtype=torch.float64),
        "elements": torch.randn(4, 129),
        "strided": torch.randn(128, 4).t(),
        "conjugate view": torch.randn(4, 128, dtype=torch.complex64).conj(),
        "not a tensor": [1.0] * row,
        "meta": torch.empty(4, 128, device="meta"),
    }
    for what, bad in bad_cases.items():
        dst = torch.zeros(6, row)
        ts = good[:2] + [bad] + good[2:]
        assert not gather.gather_rows(ts, dst), what
        assert torch.equal(dst, torch.zeros(6, row)), f"{what}: rows written"
    # destination checks: wrong row count, non-contiguous destination
    assert not gather.gather_rows(good, torch.zeros(4, row))
    assert not gather.gather_rows(good, torch.zeros(row, 5).t())
    assert gather.gather_rows([], torch.zeros(0, row))


def test_copy_rows(gather):
    src = torch.randn(128, 28, 128).to(torch.bfloat16)
    dst = torch.zeros(128 * 28 * 128, dtype=torch.bfloat16).view(128, 28, 128)
    assert gather.copy_rows(src, dst) and torch.equal(src, dst)
    for bad in (src.float(), src[:, :, :64], src.transpose(0, 1)):
        out = torch.zeros_like(dst)
        assert not gather.copy_rows(bad, out) and torch.equal(out, torch.zeros_like(dst))


class _Req:
    __slots__ = ("blocks", "row")

    def __init__(self, row):
        self.blocks, self.row = [], row


def test_parse_batch_uniform_and_refusals(gather):
    """The native one-pass batch check: a batch of one layer and scale over
    distinct known requests comes back as the backend's Python checks would
    build it; anything else is refused with None (the backend's general path
    then takes it), and errors of the lookups themselves propagate."""
    import numpy as np
    reqs = {f"r{i}": _Req(7 + 3 * i) for i in range(6)}

    def items(**over):
        out = [{"request_id": f"r{i}", "layer_idx": 1, "query": torch.randn(2, 4),
                "key": torch.randn(1, 4), "value": torch.randn(1, 4), "score_scale": 0.25}
               for i in range(6)]
        for i, (k, v) in over.items():
            if v is None:
                del out[i][k]
            else:
                out[i][k] = v
        return out

    it = items()
    layer, scale, rq, rows, first, qs, ks, vs = gather.parse_batch(it, reqs)
    assert (layer, scale) == (1, 0.25)
    assert rq == [reqs[x["request_id"]] for x in it]
    assert rows.dtype == np.int64 and rows.tolist() == [r.row for r in rq]
    assert first == -1                                    # rows 7, 10, 13, ...: not consecutive
    seq = {f"s{i}": _Req(40 + i) for i in range(5)}
    run = [{"request_id": f"s{i}", "layer_idx": 0, "query": torch.randn(2, 4),
            "key": torch.randn(1, 4), "value": torch.randn(1, 4)} for i in range(5)]
    assert gather.parse_batch(run, seq)[4] == 40          # rows 40..44 in order
    assert gather.parse_batch(run[::-1], seq)[4] == -1    # the same rows, descending
    swap = [run[1], run[0]] + run[2:]
    assert gather.parse_batch(swap, seq)[4] == -1
    assert gather.parse_batch(run[:1], seq)[4] == 40      # one request
    dup = [run[0], run[0]]
    assert gather.parse_batch(dup, seq) is None           # repeated request, rows 40, 40
    assert all(a is x["query"] and b is x["key"] and c is x["value"]
               for a, b, c, x in zip(qs, ks, vs, it))
    nos = [{k: v for k, v in x.items() if k != "score_scale"} for x in it]
    assert gather.parse_batch(nos, reqs)[1] == 1.0       # the default scale
    mixed = [dict(x) for x in it]
    mixed[2]["layer_idx"] = 1.0                            # equal as a set would count it
    assert gather.parse_batch(mixed, reqs) is not None
    for what, bad in {
        "mixed layers": lambda b: b[3].__setitem__("layer_idx", 2),
        "mixed scales": lambda b: b[0].__setitem__("score_scale", 0.5),
        "repeated request": lambda b: b[4].__setitem__("request_id", "r1"),
        "unknown request": lambda b: b[5].__setitem__("request_id", "nope"),
        "missing value": lambda b: b[1].pop("value"),
        "missing layer": lambda b: b[1].pop("layer_idx"),
        "not a dict": lambda b: b.__setitem__(2, ("r2", 1)),
    }.items():
        b = [dict(x) for x in it]
        bad(b)
        assert gather.parse_batch(b, reqs) is None, what
    assert gather.parse_batch([], reqs) is None
    b = [dict(x) for x in it]
    b[0]["request_id"] = ["unhashable"]
    with pytest.raises(TypeError):
        gather.parse_batch(b, reqs)

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

"""clv_paged_decode_balanced_noalloc (fixed device scratch, no allocation)
through the C ABI: bit for bit what clv_paged_decode_balanced returns with a
caller workspace and the same wave count, over two calls in a row (the
second with a smaller batch, so stale scratch contents from the first would
show), and a clear refusal, launching nothing, for a call too large for the
scratch."""
import math

import pytest
import torch

from cloverinfer_amd import _native, kernels
from oracle import attention as oa
from tests.helpers import assert_attention_close, make_paged_kv, padded_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(seed, ctx, hq, hkv, d, dtype):
    k, v, tables = make_paged_kv(seed, ctx, hkv, d, 16, dtype, spare_blocks=2)
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(len(ctx), hq, d, generator=g).to(dtype)
    return q, k, v, tables


@pytest.mark.parametrize("dtype,hq,hkv,d", [(torch.bfloat16, 28, 4, 128),
                                            (torch.float32, 12, 12, 64)])
def test_noalloc_equals_workspace_call(dtype, hq, hkv, d):
    lib = _native.load()
    stream = torch.cuda.current_stream().cuda_stream
    big = [300, 1, 0, 4097, 77, 16, 2500, 33]
    small = [5, 900, 17]
    for step, ctx in enumerate((big, small)):
        print(f"noalloc step {step} {dtype} {hq}/{hkv} d{d} ctx {ctx}", flush=True)
        q, k, v, tables = _case(100 + step, ctx, hq, hkv, d, dtype)
        qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
        bt = padded_tables(tables).to(DEV)
        cl = torch.tensor(ctx, dtype=torch.int32, device=DEV)
        scale = 1 / math.sqrt(d)
        out_ws = torch.full_like(qg, float("nan"))
        out_na = torch.full_like(qg, float("nan"))
        a_ws = kernels.decode_args(out_ws, qg, kg, vg, bt, cl, 16, max(ctx), scale=scale)
        a_na = kernels.decode_args(out_na, qg, kg, vg, bt, cl, 16, max(ctx), scale=scale)
        waves = 0 if step == 0 else 37
        w = waves or lib.clv_default_num_waves()
        ws = torch.empty(lib.clv_balanced_workspace_bytes(len(ctx), hq, hkv, d, w),
                         dtype=torch.uint8, device=DEV)
        _native.check(lib.clv_paged_decode_balanced(a_ws, w, ws.data_ptr(), ws.numel(), stream),
                      "clv_paged_decode_balanced")
        _native.check(lib.clv_paged_decode_balanced_noalloc(a_na, waves, stream),
                      "clv_paged_decode_balanced_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out_na, out_ws), f"step {step}: outputs differ"
        ref = oa.paged_decode(q, k, v, tables, ctx, scale)
        assert_attention_close(out_na.cpu(), ref, what=f"step {step}")


def test_noalloc_refuses_oversized_call():
    lib = _native.load()
    q, k, v, tables = _case(7, [40, 50], 8, 2, 128, torch.float16)
    qg = q.to(DEV)
    out = torch.full_like(qg, float("nan"))
    a = kernels.decode_args(out, qg, k.to(DEV), v.to(DEV), padded_tables(tables).to(DEV),
                            torch.tensor([40, 50], dtype=torch.int32, device=DEV), 16, 50)
    waves = 1 << 20  # workspace of ~8.7 GB: far beyond the scratch
    assert lib.clv_balanced_workspace_bytes(2, 8, 2, 128, waves) > 32 << 20
    rc = lib.clv_paged_decode_balanced_noalloc(a, waves, torch.cuda.current_stream().cuda_stream)
    assert rc == _native.CLV_ESCRATCH
    assert b"scratch" in lib.clv_status_string(rc)
    torch.cuda.synchronize()
    assert torch.isnan(out).all()  # nothing was launched

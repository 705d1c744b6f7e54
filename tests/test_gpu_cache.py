"""reshape_and_cache on the GPU: bit-exact against CPU index-put
(src/core/memory_manager.py:131-132), through the C ABI."""
import pytest
import torch

from cloverinfer_amd import kernels
from cloverinfer_amd.memory_manager import KVCacheManager
from oracle.blocks import BlockBookkeeping

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cpu_scatter(k_cache, v_cache, key, value, slots):
    bs = k_cache.shape[1]
    for i, s in enumerate(slots):
        if s < 0 or s >= k_cache.shape[0] * bs:
            continue
        k_cache[s // bs, s % bs] = key[i]
        v_cache[s // bs, s % bs] = value[i]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hkv,d,bs", [(1, 8, 4), (4, 128, 16), (8, 64, 32), (2, 4, 16), (3, 256, 8)])
def test_reshape_and_cache_bit_exact(dtype, hkv, d, bs):
    print(f"reshape_and_cache dtype={dtype} hkv={hkv} d={d} bs={bs}", flush=True)
    g = torch.Generator().manual_seed(hkv * 1000 + d + bs)
    nb, n = 23, 57
    k_cache = torch.zeros(nb, bs, hkv, d, dtype=dtype)
    v_cache = torch.zeros(nb, bs, hkv, d, dtype=dtype)
    # A strided source: key/value are views into a wider [n, 3*hkv, d] buffer.
    src = torch.randn(n, 3 * hkv, d, generator=g).to(dtype)
    key, value = src[:, :hkv], src[:, hkv:2 * hkv]
    slots = torch.randperm(nb * bs, generator=g)[:n].tolist()
    slots[3] = -1                # skipped
    slots[5] = nb * bs + 7       # out of range: skipped
    _cpu_scatter(k_cache, v_cache, key, value, slots)
    kg = torch.zeros(nb, bs, hkv, d, dtype=dtype, device=DEV)
    vg = torch.zeros_like(kg)
    kernels.reshape_and_cache(key.to(DEV), value.to(DEV), kg, vg,
                              torch.tensor(slots, dtype=torch.int64, device=DEV))
    torch.cuda.synchronize()
    assert torch.equal(kg.cpu(), k_cache) and torch.equal(vg.cpu(), v_cache)


def test_manager_writes_match_index_put():
    """load_initial_kv + write_new_kv(_batch) through the manager equal the
    reference's per-block copies and index-puts on the same pools."""
    g = torch.Generator().manual_seed(5)
    nb, bs, h, d = 64, 16, 12, 64
    m = KVCacheManager(nb, bs, h, d, dtype=torch.float32, device=DEV)
    o = BlockBookkeeping(nb, bs)
    kc = torch.zeros(nb, bs, h, d)
    vc = torch.zeros(nb, bs, h, d)
    rids = [f"seq{i}" for i in range(8)]
    for rid in rids:  # OPT-125m shape: 127 prefill tokens -> 8 blocks each
        kd, vd = torch.randn(127, h, d, generator=g), torch.randn(127, h, d, generator=g)
        m.load_initial_kv(rid, kd.to(DEV), vd.to(DEV))
        slots = o.load_initial_kv(rid, 127)
        _cpu_scatter(kc, vc, kd, vd, slots)
    kn, vn = torch.randn(8, h, d, generator=g), torch.randn(8, h, d, generator=g)
    m.write_new_kv_batch(rids, kn.to(DEV), vn.to(DEV))
    new_slots = []
    for rid in rids:
        b, off = o.append_slot(rid)
        assert off == 15  # the appended token lands at the last offset of block 8
        new_slots.append(b * bs + off)
    _cpu_scatter(kc, vc, kn, vn, new_slots)
    torch.cuda.synchronize()
    assert m.block_tables == o.block_tables and m.context_lens == o.context_lens
    assert all(m.context_lens[r] == 128 for r in rids)
    assert len(m.free_blocks) == 0
    assert torch.equal(m.k_cache.cpu(), kc) and torch.equal(m.v_cache.cpu(), vc)
    # single-token path
    m2 = KVCacheManager(4, 4, 2, 8, device=DEV)
    m2.allocate("a", 0)
    for t in range(5):
        m2.write_new_kv("a", torch.full((1, 2, 8), float(t), device=DEV),
                        torch.full((2, 8), float(-t), device=DEV))
    assert m2.block_tables["a"] == [3, 2]
    assert torch.equal(m2.k_cache[3, :, 0, 0].cpu(), torch.tensor([0.0, 1, 2, 3]))
    assert torch.equal(m2.v_cache[2, 0].cpu(), torch.full((2, 8), -4.0))


def test_prebuilt_cache_args_reused_across_steps():
    """An argument block built once with kernels.cache_args and launched
    directly through the C ABI step after step writes what reshape_and_cache
    writes (new values in the same source buffers each step)."""
    g = torch.Generator().manual_seed(5)
    nb, bs, hkv, d, n = 9, 16, 12, 64, 8
    src_k = torch.empty(n, hkv, d, device=DEV)
    src_v = torch.empty(n, hkv, d, device=DEV)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(DEV)
    k_a = torch.zeros(nb, bs, hkv, d, device=DEV)
    v_a = torch.zeros_like(k_a)
    k_b, v_b = k_a.clone(), v_a.clone()
    a = kernels.cache_args(src_k, src_v, k_a, v_a, slots)
    lib = kernels._native.load()
    for step in range(3):
        src_k.copy_(torch.randn(n, hkv, d, generator=g))
        src_v.copy_(torch.randn(n, hkv, d, generator=g))
        kernels._native.check(lib.clv_reshape_and_cache(a, torch.cuda.current_stream().cuda_stream),
                              "clv_reshape_and_cache")
        kernels.reshape_and_cache(src_k, src_v, k_b, v_b, slots)
        torch.cuda.synchronize()
        assert torch.equal(k_a, k_b) and torch.equal(v_a, v_b), f"step {step}"
    with pytest.raises(ValueError):
        kernels.cache_args(src_k, src_v, k_a.to(torch.float16), v_a.to(torch.float16), slots)

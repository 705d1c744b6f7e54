"""Shared test helpers: seeded paged-KV construction and the parity bar."""
from __future__ import annotations

import math

import torch

# Parity bar for attention outputs against the fp32 oracle, elementwise
#     |got - ref| <= ATOL + RTOL * |ref|      (ATOL = 2e-3, RTOL = 1e-2)
# i.e. max-abs 2e-3 near zero and max-rel 1e-2 elsewhere. A pure max-abs
# bound cannot hold for 16-bit outputs: rounding a bf16 value in [2, 4) to the
# output dtype alone moves it by up to 2^-7 = 7.8e-3 (the reference
# CpuAttentionBackend rounds its fp32 result to the query dtype the same way).
ATOL = 2e-3
RTOL = 1e-2


def assert_attention_close(got: torch.Tensor, ref: torch.Tensor, atol: float = ATOL,
                           rtol: float = RTOL, what: str = "") -> None:
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    if not got.numel():
        return
    err = (got - ref).abs()
    bound = atol + rtol * ref.abs()
    bad = err > bound
    if bad.any():
        i = int(torch.argmax((err - bound).flatten()))
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.numel()} elements outside {atol:g} + {rtol:g}*|ref|; "
            f"worst got {got.flatten()[i].item():.6f} ref {ref.flatten()[i].item():.6f}; "
            f"max-abs {err.max().item():.3e}")


def make_paged_kv(seed: int, context_lens, num_kv_heads: int, head_dim: int, block_size: int,
                  dtype: torch.dtype, value_scale: float = 1.0, spare_blocks: int = 0,
                  pool_slack: float = 0.0):
    """Random paged pools and block tables (CPU tensors).

    Every sequence gets ceil(ctx / bs) blocks (at least one) drawn without
    replacement from a shuffled pool; unused slots hold NaN so that a kernel
    reading outside a context shows up in its output. Returns
    (k_cache, v_cache, tables: list[list[int]]).
    """
    g = torch.Generator().manual_seed(seed)
    need = [max(1, math.ceil(c / block_size)) for c in context_lens]
    nb = int(math.ceil(sum(need) * (1.0 + pool_slack))) + spare_blocks
    perm = torch.randperm(nb, generator=g).tolist()
    tables, pos = [], 0
    for n in need:
        tables.append(perm[pos:pos + n])
        pos += n
    shape = (nb, block_size, num_kv_heads, head_dim)
    k = torch.full(shape, float("nan"), dtype=dtype)
    v = torch.full(shape, float("nan"), dtype=dtype)
    kf = k.view(nb * block_size, num_kv_heads, head_dim)
    vf = v.view(nb * block_size, num_kv_heads, head_dim)
    for tbl, ctx in zip(tables, context_lens):
        if ctx == 0:
            continue
        t = torch.arange(ctx)
        slots = torch.tensor(tbl, dtype=torch.long)[t // block_size] * block_size + t % block_size
        kf[slots] = (torch.randn(ctx, num_kv_heads, head_dim, generator=g) * value_scale).to(dtype)
        vf[slots] = (torch.randn(ctx, num_kv_heads, head_dim, generator=g) * value_scale).to(dtype)
    return k, v, tables


def padded_tables(tables, width: int | None = None) -> torch.Tensor:
    width = width or max(len(t) for t in tables)
    out = torch.full((len(tables), width), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        out[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    return out


# The literal bar of the hot path's parity requirement, for the five
# benchmark workloads: max-abs 2e-3 against the fp32 oracle everywhere, and
# max-rel 1e-2 where |ref| >= 0.2 (a relative bound on near-zero outputs is
# ill-posed: a 16-bit output of 1e-4 is rounded by more than 1 % of itself).
PARITY_ATOL = 2e-3
PARITY_RTOL = 1e-2
PARITY_REL_FLOOR = 0.2


def assert_parity_bar(got: torch.Tensor, ref: torch.Tensor, what: str) -> dict:
    """Assert max-abs <= 2e-3 and max-rel <= 1e-2 (where |ref| >= 0.2);
    print the observed margins and, when CLV_PARITY_LOG names a file, append
    them to it as a JSON line. Returns the figures."""
    import json
    import os

    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    err = (got - ref).abs()
    big = ref.abs() >= PARITY_REL_FLOOR
    rec = {
        "what": what,
        "elements": err.numel(),
        "max_abs": err.max().item(),
        "mean_abs": err.mean().item(),
        "max_rel": (err[big] / ref.abs()[big]).max().item() if big.any() else 0.0,
        "rel_elements": int(big.sum()),
        "max_abs_ref": ref.abs().max().item(),
    }
    print(f"[parity] {what}: max-abs {rec['max_abs']:.3e} (bar {PARITY_ATOL:g}), max-rel "
          f"{rec['max_rel']:.3e} over {rec['rel_elements']} elements with |ref| >= "
          f"{PARITY_REL_FLOOR:g} (bar {PARITY_RTOL:g}); max |ref| {rec['max_abs_ref']:.3f}", flush=True)
    path = os.environ.get("CLV_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")
    assert rec["max_abs"] <= PARITY_ATOL, f"{what}: max-abs {rec['max_abs']:.3e} > {PARITY_ATOL:g}"
    assert rec["max_rel"] <= PARITY_RTOL, f"{what}: max-rel {rec['max_rel']:.3e} > {PARITY_RTOL:g}"
    return rec

"""CPU restatement of the reference attention math (test infrastructure only).

All math is fp32 (float64 in ``brute_attention_fp64``), on torch CPU tensors,
as in the reference's CpuAttentionBackend.
"""
from __future__ import annotations

import math
from typing import Dict, List, Sequence

import numpy as np
import torch


def attend(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
           score_scale: float) -> torch.Tensor:
    """fp32 attention of one decode step, GQA-aware.

    q ``[Hq, D]``, keys/values ``[L, Hkv, D]`` -> fp32 ``[Hq, D]``.
    For Hq == Hkv this is src/core/attention_backend.py:116-118:
    ``einsum("hd,lhd->hl") * scale``, softmax over l, ``einsum("hl,lhd->hd")``.
    For Hq = G*Hkv, query head h uses kv head h // G (the repeat_kv grouping
    of src/core/model_adapter.py:506-507), computed grouped without expanding
    K/V.
    """
    hq, d = q.shape
    length, hkv, _ = keys.shape
    g = hq // hkv
    qf = q.float().reshape(hkv, g, d)
    scores = torch.einsum("kgd,lkd->kgl", qf, keys.float()) * float(score_scale)
    weights = torch.softmax(scores, dim=-1)
    ctx = torch.einsum("kgl,lkd->kgd", weights, values.float())
    return ctx.reshape(hq, d)


def attend_repeat_kv(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                     score_scale: float) -> torch.Tensor:
    """Same result as :func:`attend` via explicit repeat_kv expansion
    (src/core/model_adapter.py:506-507) and the reference's MHA einsums
    (src/core/attention_backend.py:116-118)."""
    hq = q.shape[0]
    g = hq // keys.shape[1]
    k = keys.float().repeat_interleave(g, dim=1)
    v = values.float().repeat_interleave(g, dim=1)
    scores = torch.einsum("hd,lhd->hl", q.float(), k) * float(score_scale)
    weights = torch.softmax(scores, dim=-1)
    return torch.einsum("hl,lhd->hd", weights, v)


def partial_attend(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                   score_scale: float):
    """One segment's (context, row_max, row_sum), the triple the reference's
    blocked store returns per segment (src/core/resident_kv_store.py:715-783):
    normalised fp32 context, max scaled score and sum of exp(score - max)."""
    hq, d = q.shape
    hkv = keys.shape[1]
    g = hq // hkv
    scores = torch.einsum("kgd,lkd->kgl", q.float().reshape(hkv, g, d), keys.float())
    scores = scores * float(score_scale)
    row_max = scores.amax(dim=-1)
    e = torch.exp(scores - row_max.unsqueeze(-1))
    row_sum = e.sum(dim=-1)
    ctx = torch.einsum("kgl,lkd->kgd", e / row_sum.unsqueeze(-1), values.float())
    return ctx.reshape(hq, d), row_max.reshape(hq), row_sum.reshape(hq)


def lse_merge(partials: Sequence[tuple]) -> torch.Tensor:
    """Sequential partial-softmax merge, src/core/resident_kv_store.py:2497-2509."""
    ctx, row_max, row_sum = (t.float() for t in partials[0])
    for seg_ctx, seg_max, seg_sum in partials[1:]:
        seg_ctx, seg_max, seg_sum = seg_ctx.float(), seg_max.float(), seg_sum.float()
        comb_max = torch.maximum(row_max, seg_max)
        prev_scale = torch.exp(row_max - comb_max)
        seg_scale = torch.exp(seg_max - comb_max)
        comb_sum = row_sum * prev_scale + seg_sum * seg_scale
        safe = torch.clamp(comb_sum, min=1e-12)
        prev_w = (row_sum * prev_scale / safe).unsqueeze(1)
        seg_w = (seg_sum * seg_scale / safe).unsqueeze(1)
        ctx = ctx * prev_w + seg_ctx * seg_w
        row_max, row_sum = comb_max, comb_sum
    return ctx


def split_attend(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                 score_scale: float, partition_size: int) -> torch.Tensor:
    """Split-K decode: partials over partitions of ``partition_size`` tokens,
    then :func:`lse_merge`."""
    length = keys.shape[0]
    parts = [partial_attend(q, keys[i:i + partition_size], values[i:i + partition_size],
                            score_scale)
             for i in range(0, length, partition_size)]
    return lse_merge(parts)


# fp8 pools (OCP e4m3, torch.float8_e4m3fn): a stored byte b stands for
# e4m3(b) * scale of its kv head. The reference has no fp8 pool (its resident
# KV dtypes are fp32 and fp16, src/core/attention_backend.py:201); this is the
# definition the fp8 kernels are checked against.
E4M3_MAX = 448.0


def quantize_fp8(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``x`` [..., H, D] (any float dtype) -> float8_e4m3fn codes of
    clamp(x / scale[h], -448, 448) rounded to nearest even; NaN becomes the
    positive NaN code 0x7f. The division is fp32 and correctly rounded."""
    y = x.float() / scale.float().view(-1, 1)
    y = torch.where(y > E4M3_MAX, torch.full_like(y, E4M3_MAX),
                    torch.where(y < -E4M3_MAX, torch.full_like(y, -E4M3_MAX), y))
    codes = y.to(torch.float8_e4m3fn).view(torch.uint8)
    codes = torch.where(torch.isnan(y), torch.full_like(codes, 0x7F), codes)
    return codes.view(torch.float8_e4m3fn)


def dequantize_fp8(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32 values of fp8 codes [..., H, D] with per-head ``scale``."""
    return codes.float() * scale.float().view(-1, 1)


def e4m3_value(code: int) -> float:
    """Value of one OCP e4m3 byte from its fields (sign, 4-bit exponent of
    bias 7, 3-bit mantissa; exponent 0 is subnormal; 0x7f/0xff are NaN)."""
    sign = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 0xF, code & 0x7
    if e == 0xF and m == 0x7:
        return math.nan
    if e == 0:
        return sign * m * 2.0 ** -9
    return sign * (1 + m / 8) * 2.0 ** (e - 7)


def e4m3_round(x: float) -> int:
    """e4m3 code of a finite |x| <= 448: the sign bit of x, then the nearest
    non-negative code, ties to the even one (brute force over the table)."""
    sign = 0x80 if math.copysign(1.0, x) < 0 else 0
    a = abs(x)
    best = None
    for c in range(0x7F):  # the non-negative finite codes, in increasing value
        d = abs(e4m3_value(c) - a)
        if best is None or d < best[0] or (d == best[0] and (c & 1) == 0):
            best = (d, c)
    return sign | best[1]


def gather_context(k_cache: torch.Tensor, v_cache: torch.Tensor, blocks: Sequence[int],
                   context_len: int):
    """Contiguous ``[L, Hkv, D]`` K/V of one sequence from paged pools
    ``[NB, bs, Hkv, D]`` (token t at block blocks[t // bs], offset t % bs),
    as KVCacheManager._paged_attention_ref gathers it
    (src/core/memory_manager.py:212-221)."""
    bs = k_cache.shape[1]
    if context_len == 0:
        shape = (0,) + tuple(k_cache.shape[2:])
        return k_cache.new_zeros(shape), v_cache.new_zeros(shape)
    nb = (context_len + bs - 1) // bs
    idx = torch.as_tensor(list(blocks[:nb]), dtype=torch.long)
    k = k_cache[idx].reshape(-1, *k_cache.shape[2:])[:context_len]
    v = v_cache[idx].reshape(-1, *v_cache.shape[2:])[:context_len]
    return k, v


def paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 block_tables: Sequence[Sequence[int]], context_lens: Sequence[int],
                 scale: float) -> torch.Tensor:
    """fp32 ``[S, Hq, D]``: the paged decode op on CPU tensors.

    An empty context gives zeros, which is what the reference's einsum over
    an empty token axis returns."""
    out = torch.zeros(q.shape, dtype=torch.float32)
    for s in range(q.shape[0]):
        k, v = gather_context(k_cache, v_cache, block_tables[s], int(context_lens[s]))
        if k.shape[0]:
            out[s] = attend(q[s], k, v, scale)
    return out


def chunked_prefill(q_new: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                    score_scale: float) -> torch.Tensor:
    """fp32 ``[n, Hq, D]``: query row i attends to ``keys[: L - n + i + 1]``
    (keys/values hold the whole context, the n new tokens last). Row i is the
    output of the i-th successive append-then-attend decode step."""
    n = q_new.shape[0]
    length = keys.shape[0]
    out = torch.empty(q_new.shape, dtype=torch.float32)
    for i in range(n):
        lim = length - n + i + 1
        out[i] = attend(q_new[i], keys[:lim], values[:lim], score_scale)
    return out


def chunked_prefill_masked(q_new: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                           score_scale: float) -> torch.Tensor:
    """Same result as :func:`chunked_prefill` as one causal-masked fp32
    contraction per kv head (scores ``[G*n, L]``, key ``j`` visible to query
    row ``i`` iff ``j <= L - n + i``, softmax, times V): the dense
    formulation of the n successive append-then-attend steps of
    src/core/attention_backend.py:105-118, with the GQA grouping of
    src/core/model_adapter.py:506-507 (query head h reads kv head h // G)."""
    n, hq, d = q_new.shape
    length, hkv, _ = keys.shape
    g = hq // hkv
    lim = length - n + torch.arange(n)                     # last visible key per row
    visible = torch.arange(length)[None, :] <= lim[:, None]  # [n, L]
    qf = q_new.float().reshape(n, hkv, g, d).permute(1, 0, 2, 3).reshape(hkv, n * g, d)
    kf = keys.float().permute(1, 2, 0)                      # [Hkv, D, L]
    vf = values.float().permute(1, 0, 2)                    # [Hkv, L, D]
    scores = torch.bmm(qf, kf) * float(score_scale)         # [Hkv, n*G, L]
    mask = visible.repeat_interleave(g, dim=0)              # row r is token r // G
    scores = scores.masked_fill(~mask[None], float("-inf"))
    ctx = torch.bmm(torch.softmax(scores, dim=-1), vf)      # [Hkv, n*G, D]
    return ctx.reshape(hkv, n, g, d).permute(1, 0, 2, 3).reshape(n, hq, d)


def brute_attention_fp64(q: np.ndarray, keys: np.ndarray, values: np.ndarray,
                         score_scale: float) -> np.ndarray:
    """Explicit-loop float64 attention for tiny shapes (an independent
    formulation: two-pass softmax with max subtraction, kv head h // G)."""
    hq, d = q.shape
    length, hkv, _ = keys.shape
    g = hq // hkv
    out = np.zeros((hq, d), dtype=np.float64)
    for h in range(hq):
        kh = h // g
        s = [score_scale * sum(float(q[h, e]) * float(keys[t, kh, e]) for e in range(d))
             for t in range(length)]
        if not s:
            continue
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = math.fsum(w)
        for e in range(d):
            out[h, e] = math.fsum(w[t] * float(values[t, kh, e]) for t in range(length)) / z
    return out


class CpuAttentionOracle:
    """Restatement of CpuAttentionBackend (src/core/attention_backend.py:56-144).

    Per (request, layer) contiguous ``[T, Hkv, D]`` KV grown by concatenation;
    ``decode_layer`` appends the new K/V first, then attends in fp32 and casts
    to the query dtype; the context length advances after the last layer.
    Differences from the reference class, both additive: ``init_request``
    accepts ``decode_reserve_tokens`` (the AttentionNode passes it,
    src/core/nodes.py:125-131), and Hq may be a multiple of Hkv (GQA).
    """

    def __init__(self):
        self.k_cache: Dict[str, List[torch.Tensor]] = {}
        self.v_cache: Dict[str, List[torch.Tensor]] = {}
        self.context_lens: Dict[str, int] = {}

    def init_request(self, request_id: str, initial_kv: List[Dict[str, torch.Tensor]],
                     decode_reserve_tokens: int = 0) -> int:
        if request_id in self.k_cache:
            raise ValueError(f"Request {request_id} already exists")
        if not initial_kv:
            raise ValueError("initial_kv must contain at least one layer")
        self.k_cache[request_id] = [l["key"].detach().cpu().contiguous() for l in initial_kv]
        self.v_cache[request_id] = [l["value"].detach().cpu().contiguous() for l in initial_kv]
        seq_len = int(self.k_cache[request_id][0].shape[0])
        self.context_lens[request_id] = seq_len
        return seq_len

    def decode_layer(self, request_id: str, layer_idx: int, query: torch.Tensor,
                     key: torch.Tensor, value: torch.Tensor,
                     score_scale: float = 1.0) -> torch.Tensor:
        if request_id not in self.k_cache:
            raise KeyError(f"Unknown request {request_id}")
        q = query.detach().cpu().contiguous()
        k_new = key.detach().cpu().contiguous()
        v_new = value.detach().cpu().contiguous()
        if q.dim() == 3:
            q = q.squeeze(0)
        if k_new.dim() == 3:
            k_new = k_new.squeeze(0)
        if v_new.dim() == 3:
            v_new = v_new.squeeze(0)
        layers_k = self.k_cache[request_id]
        layers_v = self.v_cache[request_id]
        layers_k[layer_idx] = torch.cat([layers_k[layer_idx], k_new.unsqueeze(0)], dim=0)
        layers_v[layer_idx] = torch.cat([layers_v[layer_idx], v_new.unsqueeze(0)], dim=0)
        ctx = attend(q, layers_k[layer_idx], layers_v[layer_idx], score_scale)
        if layer_idx == len(layers_k) - 1:
            self.context_lens[request_id] += 1
        return ctx.to(query.dtype).unsqueeze(0)

    def decode_layer_batch(self, items: List[Dict[str, object]]) -> List[torch.Tensor]:
        return [
            self.decode_layer(str(it["request_id"]), int(it["layer_idx"]), it["query"],
                              it["key"], it["value"], float(it.get("score_scale", 1.0)))
            for it in items
        ]

    def get_context_len(self, request_id: str) -> int:
        return self.context_lens[request_id]

    def free_request(self, request_id: str) -> None:
        self.k_cache.pop(request_id, None)
        self.v_cache.pop(request_id, None)
        self.context_lens.pop(request_id, None)

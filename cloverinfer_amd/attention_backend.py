"""The ``"gpu"`` attention backend for CloverInfer's AttentionNode.

Implements the node-level backend protocol of CpuAttentionBackend
(src/core/attention_backend.py:56-144): ``init_request``, ``decode_layer``,
``decode_layer_batch``, ``get_context_len``, ``free_request`` and
``get_debug_info``, with the same semantics (append-then-attend, fp32 math,
output in the query dtype, context length advancing after the last layer,
ValueError on a duplicate request, KeyError on an unknown one).

Storage is paged instead of one contiguous tensor per (request, layer):
per-layer pools ``[num_blocks, block_size, num_kv_heads, head_dim]`` share
one block table per request, so token p of a request lives in the same slot
of every layer. A batch of decode items for one layer becomes one
reshape_and_cache launch plus one paged-decode launch.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional

import numpy as np
import torch

from . import kernels


class _Request:
    __slots__ = ("blocks", "layer_lens", "context_len")

    def __init__(self, blocks: List[int], num_layers: int, seq_len: int):
        self.blocks = blocks
        self.layer_lens = [seq_len] * num_layers
        self.context_len = seq_len


class GpuAttentionBackend:
    def __init__(self, num_blocks: int = 4096, block_size: int = 16, device: str = "cuda",
                 kv_dtype: Optional[torch.dtype] = None, partition_size: Optional[int] = None):
        if num_blocks <= 0 or block_size <= 0 or block_size & (block_size - 1):
            raise ValueError("num_blocks must be positive and block_size a power of two")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("GpuAttentionBackend needs a HIP device (there is no CPU fallback)")
        self.kv_dtype = kv_dtype
        self.partition_size = partition_size
        self.k_pools: Optional[torch.Tensor] = None  # [L, NB, bs, Hkv, D]
        self.v_pools: Optional[torch.Tensor] = None
        self.num_layers = 0
        self.free_blocks: List[int] = list(range(num_blocks))
        self.requests: Dict[str, _Request] = {}
        self.stats = {"decode_items": 0, "decode_launches": 0, "init_requests": 0}

    # ------------------------------------------------------------ pools
    def _ensure_pools(self, num_layers: int, num_kv_heads: int, head_dim: int,
                      dtype: torch.dtype) -> None:
        if self.k_pools is not None:
            _, _, _, hkv, d = self.k_pools.shape
            if (num_layers, num_kv_heads, head_dim) != (self.num_layers, hkv, d):
                raise ValueError(
                    f"request shape (layers={num_layers}, kv_heads={num_kv_heads}, "
                    f"head_dim={head_dim}) differs from the pools "
                    f"(layers={self.num_layers}, kv_heads={hkv}, head_dim={d})"
                )
            return
        dtype = self.kv_dtype or dtype
        shape = (num_layers, self.num_blocks, self.block_size, num_kv_heads, head_dim)
        self.k_pools = torch.zeros(shape, dtype=dtype, device=self.device)
        self.v_pools = torch.zeros(shape, dtype=dtype, device=self.device)
        self.num_layers = num_layers

    def _take_blocks(self, n: int, what: str) -> List[int]:
        if len(self.free_blocks) < n:
            raise RuntimeError(what)
        return [self.free_blocks.pop() for _ in range(n)]

    def _slot(self, req: _Request, pos: int) -> int:
        bs = self.block_size
        return req.blocks[pos // bs] * bs + pos % bs

    # ------------------------------------------------------------ protocol
    def init_request(self, request_id: str, initial_kv: List[Dict[str, torch.Tensor]],
                     decode_reserve_tokens: int = 0) -> int:
        if request_id in self.requests:
            raise ValueError(f"Request {request_id} already exists")
        if not initial_kv:
            raise ValueError("initial_kv must contain at least one layer")
        k0 = initial_kv[0]["key"]
        seq_len, hkv, d = int(k0.shape[0]), int(k0.shape[1]), int(k0.shape[2])
        self._ensure_pools(len(initial_kv), hkv, d, k0.dtype)
        reserve = max(1, int(decode_reserve_tokens))
        nblocks = max(1, math.ceil((seq_len + reserve) / self.block_size))
        req = _Request(self._take_blocks(nblocks, "OOM: Not enough blocks"), self.num_layers,
                       seq_len)
        if seq_len:
            slots = torch.tensor([self._slot(req, p) for p in range(seq_len)],
                                 dtype=torch.int64).to(self.device)
            for layer, kv in enumerate(initial_kv):
                k = kv["key"].to(device=self.device, dtype=self.k_pools.dtype)
                v = kv["value"].to(device=self.device, dtype=self.v_pools.dtype)
                if k.shape != (seq_len, hkv, d) or v.shape != k.shape:
                    self.free_blocks.extend(req.blocks)
                    raise ValueError(f"layer {layer}: key/value shape differs from layer 0")
                kernels.reshape_and_cache(k, v, self.k_pools[layer], self.v_pools[layer], slots)
        self.requests[request_id] = req
        self.stats["init_requests"] += 1
        return seq_len

    def decode_layer(self, request_id: str, layer_idx: int, query: torch.Tensor,
                     key: torch.Tensor, value: torch.Tensor,
                     score_scale: float = 1.0) -> torch.Tensor:
        return self.decode_layer_batch([{
            "request_id": request_id, "layer_idx": layer_idx, "query": query,
            "key": key, "value": value, "score_scale": score_scale,
        }])[0]

    def decode_layer_batch(self, items: List[Dict[str, object]]) -> List[torch.Tensor]:
        """Items in order; consecutive items of one (layer, scale) with distinct
        requests form one launch pair (append + decode)."""
        out: List[torch.Tensor] = []
        wave: List[Dict[str, object]] = []
        key = None
        for it in items:
            rid = str(it["request_id"])
            if rid not in self.requests:
                raise KeyError(f"Unknown request {rid}")
            k = (int(it["layer_idx"]), float(it.get("score_scale", 1.0)))
            if wave and (k != key or any(str(w["request_id"]) == rid for w in wave)):
                out.extend(self._run_wave(wave, *key))
                wave = []
            key = k
            wave.append(it)
        if wave:
            out.extend(self._run_wave(wave, *key))
        return out

    def _run_wave(self, items: List[Dict[str, object]], layer: int,
                  score_scale: float) -> List[torch.Tensor]:
        if not 0 <= layer < self.num_layers:
            raise IndexError(f"layer_idx {layer} outside [0, {self.num_layers})")
        dt = self.k_pools.dtype

        def rows(name: str) -> torch.Tensor:
            ts = []
            for it in items:
                t = it[name]
                ts.append(t.squeeze(0) if t.dim() == 3 else t)
            return torch.stack(ts).to(device=self.device, dtype=dt)

        q, k, v = rows("query"), rows("key"), rows("value")
        reqs = [self.requests[str(it["request_id"])] for it in items]
        slots = []
        for req in reqs:
            pos = req.layer_lens[layer]
            if pos >= len(req.blocks) * self.block_size:
                req.blocks.extend(self._take_blocks(1, "OOM during append"))
            slots.append(self._slot(req, pos))
        kernels.reshape_and_cache(k, v, self.k_pools[layer], self.v_pools[layer],
                                  torch.tensor(slots, dtype=torch.int64).to(self.device))
        for req in reqs:
            req.layer_lens[layer] += 1
        lens = [req.layer_lens[layer] for req in reqs]
        width = max(len(req.blocks) for req in reqs)
        table = np.full((len(reqs), width), -1, dtype=np.int32)
        for i, req in enumerate(reqs):
            table[i, :len(req.blocks)] = req.blocks
        bt = torch.from_numpy(table).to(self.device)
        ctx = torch.tensor(lens, dtype=torch.int32).to(self.device)
        ctx_out = torch.empty_like(q)
        kernels.paged_attention(ctx_out, q, self.k_pools[layer], self.v_pools[layer], bt, ctx,
                                self.block_size, max(lens), scale=score_scale,
                                partition_size=self.partition_size)
        if layer == self.num_layers - 1:
            for req in reqs:
                req.context_len += 1
        self.stats["decode_items"] += len(items)
        self.stats["decode_launches"] += 1
        results = []
        for i, it in enumerate(items):
            qin = it["query"]
            results.append(ctx_out[i].unsqueeze(0).to(device=qin.device, dtype=qin.dtype))
        return results

    def get_context_len(self, request_id: str) -> int:
        return self.requests[request_id].context_len

    def free_request(self, request_id: str) -> None:
        req = self.requests.pop(request_id, None)
        if req is not None:
            self.free_blocks.extend(req.blocks)

    def get_debug_info(self) -> Dict[str, object]:
        return {
            "backend": "gpu",
            "device": str(self.device),
            "num_blocks": self.num_blocks,
            "block_size": self.block_size,
            "free_blocks": len(self.free_blocks),
            "requests": len(self.requests),
            "num_layers": self.num_layers,
            "kv_dtype": str(self.k_pools.dtype) if self.k_pools is not None else None,
            **self.stats,
        }


def create_attention_backend(backend: str, backend_kwargs: Optional[Dict[str, object]] = None):
    """The ``"gpu"`` branch of AttentionNode's backend switch (src/core/nodes.py:88-98).

    Other names belong to the reference's own backends and are not part of
    this package.
    """
    if backend == "gpu":
        return GpuAttentionBackend(**(backend_kwargs or {}))
    raise ValueError(f"Unsupported attention backend for this package: {backend}")

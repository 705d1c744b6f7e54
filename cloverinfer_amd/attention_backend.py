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
append-then-attend step on the GPU: a fused append + decode launch for short
contexts, and for contexts past 512 tokens the decode over the cached tokens,
started as soon as the queries are uploaded, followed by a merge that takes
each request's new token and writes its rows. It is fed by:

* a device-resident block table (``DeviceBlockTable``): a request's row is
  written once at ``init_request``; a block taken during decode is one
  queued entry (the reference rebuilds the table on the host every call,
  src/core/memory_manager.py:145-173);
* the batch's q/k/v rows and metadata (slots, context lengths, table rows)
  staged in pinned memory and uploaded in one copy, or in two around the
  decode's start (the second on a copy stream of its own);
* one device-to-host copy of the batch's outputs, or none where the merge
  writes them straight into the pinned tensor the call returns.
"""
from __future__ import annotations

import math
import operator
from typing import Dict, List, Optional

import numpy as np
import torch

from . import _native, kernels
from .block_table import DeviceBlockTable


class _Request:
    __slots__ = ("blocks", "row")

    def __init__(self, blocks: List[int], row: int):
        self.blocks = blocks  # blocks held, in table order
        self.row = row        # row of the device block table and of the host state


_get_layer = operator.itemgetter("layer_idx")
_get_rid = operator.itemgetter("request_id")
_get_row = operator.attrgetter("row")
_get_scale = operator.methodcaller("get", "score_scale", 1.0)
_get_query = operator.itemgetter("query")
_get_key = operator.itemgetter("key")
_get_value = operator.itemgetter("value")


def _align(n: int) -> int:
    return (n + 255) // 256 * 256


# Names accepted for the pool dtype: the resident KV dtype strings of the
# reference's PIM backends (src/core/attention_backend.py:201, "fp32" and
# "fp16"; src/core/config.py:38) plus bf16, and torch's own names.
_KV_DTYPES = {
    "fp32": torch.float32, "float32": torch.float32,
    "fp16": torch.float16, "float16": torch.float16, "half": torch.float16,
    "bf16": torch.bfloat16, "bfloat16": torch.bfloat16,
    "fp8": torch.float8_e4m3fn, "fp8_e4m3": torch.float8_e4m3fn,
    "float8_e4m3fn": torch.float8_e4m3fn,
}


def _kv_dtype(value) -> Optional[torch.dtype]:
    if value is None or isinstance(value, torch.dtype):
        if value is not None and value not in _KV_DTYPES.values():
            raise ValueError(f"Unsupported kv dtype: {value}")
        return value
    name = str(value).lower().replace("torch.", "")
    if name not in _KV_DTYPES:
        raise ValueError(f"Unsupported resident_kv_dtype: {value}")
    return _KV_DTYPES[name]


class GpuAttentionBackend:
    def __init__(self, num_blocks: int = 4096, block_size: int = 16, device: str = "cuda",
                 kv_dtype=None, partition_size: Optional[int] = None,
                 resident_kv_dtype=None, kv_scale=1.0):
        """``kv_dtype`` (or ``resident_kv_dtype``, the reference's knob name
        as the scheduler passes it to KV-resident backends) selects the pool
        dtype: a torch dtype or "fp32" / "fp16" / "bf16" / "fp8". Default: the
        dtype of the first request's KV. Queries, keys and values are converted
        to it; outputs come back in each query's dtype. "fp8" keeps OCP e4m3
        pools with ``kv_scale`` (a number or one value per kv head, the same
        for keys and values): values are stored as e4m3(x / scale), queries
        and the attention math stay 16-bit / fp32."""
        if num_blocks <= 0 or block_size <= 0 or block_size & (block_size - 1):
            raise ValueError("num_blocks must be positive and block_size a power of two")
        if kv_dtype is not None and resident_kv_dtype is not None and \
                _kv_dtype(kv_dtype) != _kv_dtype(resident_kv_dtype):
            raise ValueError("kv_dtype and resident_kv_dtype disagree")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("GpuAttentionBackend needs a HIP device (there is no CPU fallback)")
        self.kv_dtype = _kv_dtype(kv_dtype if kv_dtype is not None else resident_kv_dtype)
        self.partition_size = partition_size
        self.kv_scale = kv_scale
        self.k_scales: Optional[torch.Tensor] = None  # fp8 pools: [num_kv_heads] on the device
        self.v_scales: Optional[torch.Tensor] = None
        self.k_pools: Optional[torch.Tensor] = None  # [L, NB, bs, Hkv, D]
        self._layer_pools: List[tuple] = []  # (k, v) views of each layer's pools
        self.v_pools: Optional[torch.Tensor] = None
        self.num_layers = 0
        self.free_blocks: List[int] = list(range(num_blocks))
        self.requests: Dict[str, _Request] = {}
        self.tables = DeviceBlockTable(self.device)
        # Host state per table row (so a batch is bookkept with array
        # operations): tokens held per layer, context length (advanced after
        # the last layer), blocks held and the row's block-table entries.
        self._lens = np.zeros((0, 0), dtype=np.int64)
        self._ctx = np.zeros(0, dtype=np.int64)
        self._nblk = np.zeros(0, dtype=np.int64)
        self._htab = np.zeros((0, 0), dtype=np.int64)
        self._bshift = block_size.bit_length() - 1
        self._stage: Dict[str, torch.Tensor] = {}  # pinned host staging buffers, grow-only
        self._stage_np: Dict[str, np.ndarray] = {}  # their bytes as numpy arrays
        self._split_ok: Dict[tuple, bool] = {}  # batch shapes the split decode covers
        self._offsets: Dict[tuple, tuple] = {}  # staging-buffer offsets per batch shape
        self._stage_done: Optional[torch.cuda.Event] = None  # copies out of them issued
        # Device twin of the staging buffer, reused by every wave: a wave
        # whose results stay on the device returns while its kernels may still
        # read it, so the next wave's upload into it is ordered after them
        # (stream order on the same stream, an event wait across streams).
        # The device output buffer serves only waves whose results go back to
        # the host (such a call waits for them before it returns). And the
        # fused launches built for the staged views.
        self._dstage: Optional[torch.Tensor] = None
        self._dstage_free: Optional[torch.cuda.Event] = None  # after the last reader of _dstage
        self._dstage_stream: Optional[int] = None  # stream of that reader
        self._dout: Optional[torch.Tensor] = None
        # The split decode's second upload (k, v, slots, table updates) goes
        # on a copy stream of its own (default priority), so that it runs
        # while the decode over the cached tokens does; events order it after
        # the first upload and before the merge.
        self._up_stream: Optional[torch.cuda.Stream] = None
        self._up_done: Optional[torch.cuda.Event] = None
        self._h1_done: Optional[torch.cuda.Event] = None
        self._launches: Dict[tuple, "kernels.AppendDecodeLaunch"] = {}
        self._views: Dict[tuple, tuple] = {}  # device views into _dstage per batch shape
        self._filled_host = False
        self._gathered = False
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
        if dtype == kernels.FP8:
            self.k_scales = kernels.kv_scales(self.kv_scale, num_kv_heads, self.device)
            self.v_scales = self.k_scales
        self.k_pools = torch.zeros(shape, dtype=dtype, device=self.device)
        self.v_pools = torch.zeros(shape, dtype=dtype, device=self.device)
        self.num_layers = num_layers
        self._layer_pools = [(self.k_pools[i], self.v_pools[i]) for i in range(num_layers)]

    @property
    def _fp8(self) -> bool:
        return self.k_pools is not None and self.k_pools.dtype == kernels.FP8

    def _append_dtype(self, src: torch.dtype) -> torch.dtype:
        """dtype new K/V rows are handed to the append in: the pool dtype, or
        for fp8 pools a float dtype the quantising append reads."""
        if not self._fp8:
            return self.k_pools.dtype
        return src if src in (torch.float32, torch.float16, torch.bfloat16) else torch.float32

    def _compute_dtype(self, qdt: torch.dtype) -> torch.dtype:
        """dtype of q and out in the kernels: the pool dtype, or for fp8
        pools fp16 for fp16 queries and bf16 otherwise."""
        if not self._fp8:
            return self.k_pools.dtype
        return torch.float16 if qdt == torch.float16 else torch.bfloat16

    def _append(self, k, v, layer: int, slots: torch.Tensor) -> None:
        kernels.reshape_and_cache(k, v, self.k_pools[layer], self.v_pools[layer], slots,
                                  k_scale=self.k_scales, v_scale=self.v_scales)

    def _take_blocks(self, n: int, what: str) -> List[int]:
        if len(self.free_blocks) < n:
            raise RuntimeError(what)
        return [self.free_blocks.pop() for _ in range(n)]

    def _slot(self, req: _Request, pos: int) -> int:
        bs = self.block_size
        return req.blocks[pos // bs] * bs + pos % bs

    def _host_row(self, req: _Request, seq_len: int) -> None:
        """(Re)initialise the host state of the request's row."""
        row, nb = req.row, len(req.blocks)
        rows = max(self._lens.shape[0], 1)
        while rows <= row:
            rows *= 2
        width = max(self._htab.shape[1], 1)
        while width < nb:
            width *= 2
        if rows > self._lens.shape[0] or self.num_layers > self._lens.shape[1]:
            lens = np.zeros((rows, self.num_layers), dtype=np.int64)
            lens[:self._lens.shape[0], :self._lens.shape[1]] = self._lens
            self._lens = lens
            self._ctx = np.concatenate([self._ctx, np.zeros(rows - self._ctx.size, np.int64)])
            self._nblk = np.concatenate([self._nblk, np.zeros(rows - self._nblk.size, np.int64)])
        if rows > self._htab.shape[0] or width > self._htab.shape[1]:
            tab = np.full((rows, width), -1, dtype=np.int64)
            tab[:self._htab.shape[0], :self._htab.shape[1]] = self._htab
            self._htab = tab
        self._lens[row] = seq_len
        self._ctx[row] = seq_len
        self._nblk[row] = nb
        self._htab[row] = -1
        self._htab[row, :nb] = req.blocks

    def _grow_request(self, req: _Request) -> None:
        """One more block for a request whose blocks are full."""
        blk = self._take_blocks(1, "OOM during append")[0]
        col = len(req.blocks)
        self.tables.set(req.row, col, blk)
        req.blocks.append(blk)
        if col >= self._htab.shape[1]:
            tab = np.full((self._htab.shape[0], 2 * self._htab.shape[1]), -1, dtype=np.int64)
            tab[:, :self._htab.shape[1]] = self._htab
            self._htab = tab
        self._htab[req.row, col] = blk
        self._nblk[req.row] = col + 1

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
        blocks = self._take_blocks(nblocks, "OOM: Not enough blocks")
        req = _Request(blocks, self.tables.add(blocks))
        if seq_len:
            slots = torch.tensor([self._slot(req, p) for p in range(seq_len)],
                                 dtype=torch.int64).to(self.device)
            for layer, kv in enumerate(initial_kv):
                k = kv["key"].to(device=self.device, dtype=self._append_dtype(kv["key"].dtype))
                v = kv["value"].to(device=self.device, dtype=k.dtype)
                if k.shape != (seq_len, hkv, d) or v.shape != k.shape:
                    self.free_blocks.extend(req.blocks)
                    self.tables.remove(req.row)
                    raise ValueError(f"layer {layer}: key/value shape differs from layer 0")
                self._append(k, v, layer, slots)
        self._host_row(req, seq_len)
        self.requests[request_id] = req
        self.stats["init_requests"] += 1
        return seq_len

    def init_request_from_hf(self, request_id: str, past_key_values, layout: str = "bhtd",
                             batch_index: int = 0, seq_len: Optional[int] = None,
                             decode_reserve_tokens: int = 0) -> int:
        """``init_request`` straight from a Hugging Face cache: no permute,
        no contiguous copy, no host round trip (the reference normalises every
        layer to a contiguous ``[T, heads, D]`` CPU tensor first,
        src/core/model_adapter.py:174-182, 205-240).

        ``past_key_values``: one entry per layer, a ``(key, value)`` pair or an
        object with ``key_cache``/``value_cache`` or ``keys``/``values``;
        tensors ``[B, H, T, D]`` (``layout="bhtd"``, the common one) or
        ``[B, T, H, D]`` (``"bthd"``). Sequence ``batch_index`` is ingested,
        its first ``seq_len`` tokens (default: all T). Each layer is one strided
        reshape_and_cache launch into the shared block table's slots.
        """
        if request_id in self.requests:
            raise ValueError(f"Request {request_id} already exists")
        if layout not in ("bhtd", "bthd"):
            raise ValueError(f"layout must be 'bhtd' or 'bthd', got {layout!r}")

        def pair(entry):
            for a, b in (("key_cache", "value_cache"), ("keys", "values")):
                if hasattr(entry, a) and hasattr(entry, b):
                    return getattr(entry, a), getattr(entry, b)
            return entry[0], entry[1]

        layers = [pair(e) for e in past_key_values]
        if not layers:
            raise ValueError("past_key_values must contain at least one layer")
        views = []
        for li, (k, v) in enumerate(layers):
            if k.dim() != 4 or v.shape != k.shape:
                raise ValueError(f"layer {li}: expected 4-D key/value of one shape")
            k, v = k[batch_index], v[batch_index]
            if layout == "bhtd":  # [H, T, D] -> [T, H, D] view
                k, v = k.transpose(0, 1), v.transpose(0, 1)
            views.append((k, v))
        total, hkv, d = views[0][0].shape
        T = total if seq_len is None else int(seq_len)
        if not 0 <= T <= total:
            raise ValueError(f"seq_len {T} outside [0, {total}]")
        dt = self.kv_dtype or views[0][0].dtype
        self._ensure_pools(len(views), hkv, d, dt)
        reserve = max(1, int(decode_reserve_tokens))
        nblocks = max(1, math.ceil((T + reserve) / self.block_size))
        blocks = self._take_blocks(nblocks, "OOM: Not enough blocks")
        req = _Request(blocks, self.tables.add(blocks))
        if T:
            bs = self.block_size
            pos = torch.arange(T)
            slots = (torch.tensor(blocks, dtype=torch.int64)[pos // bs] * bs + pos % bs).to(
                self.device)
            for layer, (k, v) in enumerate(views):
                if k.shape[1:] != (hkv, d):
                    self.free_blocks.extend(blocks)
                    self.tables.remove(req.row)
                    raise ValueError(f"layer {layer}: key/value shape differs from layer 0")
                k = k[:T].to(device=self.device, dtype=self._append_dtype(k.dtype))
                v = v[:T].to(device=self.device, dtype=k.dtype)
                if k.stride(2) != 1:
                    k = k.contiguous()
                if v.stride(2) != 1:
                    v = v.contiguous()
                self._append(k, v, layer, slots)
        self._host_row(req, T)
        self.requests[request_id] = req
        self.stats["init_requests"] += 1
        return T

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
        requests = self.requests
        if items:
            # The node's batch: one layer and scale, distinct known requests,
            # checked in one native pass (or a few C-level passes without the
            # native module) instead of a loop per item.
            host = _native.load_host()
            if host is not None and type(items) is list and type(requests) is dict:
                parsed = host.parse_batch(items, requests)
                if parsed is not None:
                    layer, scale, reqs, rows, first, qs, ks, vs = parsed
                    return self._run_wave(qs, ks, vs, reqs, int(layer), float(scale), rows=rows,
                                          rows_first=first)
            layers = set(map(_get_layer, items))
            scales = set(map(_get_scale, items))
            if len(layers) == 1 and len(scales) == 1:
                reqs = list(map(requests.get, map(_get_rid, items)))
                if None not in reqs and len(set(map(_get_row, reqs))) == len(reqs):
                    return self._run_wave(*self._payloads(items), reqs, int(layers.pop()),
                                          float(scales.pop()))
        out: List[torch.Tensor] = []
        wave: List[Dict[str, object]] = []
        reqs = []
        in_wave = set()
        key = None
        for it in items:
            rid = it["request_id"]
            req = requests.get(rid)
            if req is None:
                req = requests.get(str(rid))
                if req is None:
                    raise KeyError(f"Unknown request {rid}")
            k = (int(it["layer_idx"]), float(it.get("score_scale", 1.0)))
            if wave and (k != key or req.row in in_wave):
                out.extend(self._run_wave(*self._payloads(wave), reqs, *key))
                wave, reqs, in_wave = [], [], set()
            key = k
            wave.append(it)
            reqs.append(req)
            in_wave.add(req.row)
        if wave:
            out.extend(self._run_wave(*self._payloads(wave), reqs, *key))
        return out

    @staticmethod
    def _payloads(items: List[Dict[str, object]]):
        return (list(map(_get_query, items)), list(map(_get_key, items)),
                list(map(_get_value, items)))

    def decode_layer_packed(self, request_ids: List[str], layer_idx: int, query: torch.Tensor,
                            key: torch.Tensor, value: torch.Tensor,
                            score_scale: float = 1.0) -> torch.Tensor:
        """decode_layer_batch for one layer of distinct requests with the
        payloads stacked: query [B, Hq, D], key / value [B, Hkv, D] (host or
        device) -> contexts [B, 1, Hq, D] in the query's dtype and on its
        device. Row i is exactly what decode_layer_batch returns for item i;
        the stacked form spares the per-tensor cost of B separate payloads
        and outputs."""
        n = len(request_ids)
        if query.dim() != 3 or query.shape[0] != n or key.shape[0] != n or value.shape[0] != n:
            raise ValueError("query, key and value need one row per request id")
        reqs = []
        for rid in request_ids:
            req = self.requests.get(rid)
            if req is None:
                req = self.requests.get(str(rid))
                if req is None:
                    raise KeyError(f"Unknown request {rid}")
            reqs.append(req)
        if len({r.row for r in reqs}) != n:
            raise ValueError("decode_layer_packed takes each request at most once")
        if n == 0:
            return query.new_empty((0, 1) + tuple(query.shape[1:]))
        return self._run_wave(query, key, value, reqs, int(layer_idx), float(score_scale),
                              packed=True)

    def _staging(self, name: str, shape, dtype: torch.dtype) -> torch.Tensor:
        """A pinned host buffer of at least ``shape``, reused across calls (the
        caller waits for the previous call's copies out of it first)."""
        n = 1
        for x in shape:
            n *= x
        buf = self._stage.get(name)
        if buf is None or buf.dtype != dtype or buf.numel() < n:
            buf = torch.empty(max(n, 1), dtype=dtype, pin_memory=True)
            self._stage[name] = buf
            self._stage_np[name] = buf.numpy()
            self._views.clear()  # they hold slices of the old buffer
        return buf[:n].view(*shape)

    def _fill(self, ts: List[torch.Tensor], heads: int, d: int, dt: torch.dtype,
              raw: torch.Tensor):
        """The tensors ``ts`` ([heads, d] or [1, heads, d] each) as rows of
        [B, heads, d]: written into the pinned bytes ``raw`` (returns None; the
        caller uploads them with the rest), or, when they are already on the
        device, stacked there (returns that tensor)."""
        n = len(ts)
        t0 = ts[0]
        host = raw.view(dt).view(n, heads, d)
        if isinstance(ts, torch.Tensor):  # stacked payloads
            if ts.numel() != n * heads * d:
                raise ValueError(f"payload of shape {tuple(ts.shape)}, expected {n} x {heads} x {d}")
            if ts.is_cuda:
                # reshape() of a strided view can keep a strided head_dim,
                # which the kernels refuse: make it contiguous.
                return ts.reshape(n, heads, d).to(device=self.device, dtype=dt).contiguous()
            gather = _native.load_host()
            if gather is None or not gather.copy_rows(ts, host):
                host.copy_(ts.reshape(n, heads, d))
            return None
        if t0.device.type == "cpu" and t0.numel() == heads * d:
            # The node's case (host tensors of one shape): the native gather
            # checks every payload and copies the rows into the pinned buffer
            # (about 10 us for 128 payloads, against 40 us for torch.stack);
            # payloads it refuses (another dtype, strided, on the device) go
            # through one stack straight into the pinned buffer, where torch
            # checks shapes and devices and converts dtypes; anything else
            # takes the general path.
            gather = _native.load_host()
            if gather is not None and isinstance(ts, list) and \
                    gather.gather_rows(ts, host.view(n, heads * d)):
                self._filled_host = True  # every payload was a host tensor
                self._gathered = True     # ... of dtype dt
                return None
            try:
                torch.stack(ts, out=host.view(n, *t0.shape))
                self._filled_host = True  # every payload was a host tensor
                return None
            except (RuntimeError, TypeError):
                pass
        idx = self.device.index
        if t0.numel() == heads * d and all(
                t.shape == t0.shape and t.is_cuda and (idx is None or t.get_device() == idx)
                for t in ts):
            return torch.stack(ts).view(n, heads, d).to(dt)
        for t in ts:
            if t.numel() != heads * d:
                raise ValueError(f"payload of shape {tuple(t.shape)}, expected {heads} x {d}")
        host.copy_(torch.stack([t.reshape(heads, d).to("cpu") for t in ts]))
        return None

    def _run_wave(self, qs, ks, vs, reqs: List[_Request], layer: int, score_scale: float,
                  packed: bool = False, rows: Optional[np.ndarray] = None,
                  rows_first: Optional[int] = None):
        """One append + decode over distinct requests. qs / ks / vs: lists of
        per-request payloads, or stacked tensors (packed; returns one tensor).
        rows / rows_first: the requests' table rows and, when known, whether
        they run consecutively from rows_first (-1: they do not).

        Payloads are validated and staged before any request state changes:
        a malformed call raises and leaves every request as it was (the
        reference backend raises from torch.cat before it appends anything,
        src/core/attention_backend.py:105-110). Should a later step fail,
        the token counts are rolled back and the block-table entries queued
        again."""
        if not 0 <= layer < self.num_layers:
            raise IndexError(f"layer_idx {layer} outside [0, {self.num_layers})")
        _, _, bs, hkv, d = self.k_pools.shape
        n = len(reqs)
        q0 = qs[0]
        hq = q0.numel() // d
        if hq * d != q0.numel() or hq == 0 or hq % hkv:
            raise ValueError(f"query of shape {tuple(q0.shape)}: expected [{hkv}*G, {d}] rows "
                             f"for {hkv} kv heads of head_dim {d}")
        if self._stage_done is not None:
            self._stage_done.synchronize()  # the staging buffer is free again
        dt = self._compute_dtype(q0.dtype)
        kdt = self._append_dtype(ks[0].dtype)  # fp8 pools: quantised once, from the payload

        # One pinned buffer for the call's uploads: q | int32 context lengths
        # and rows | k | v | int64 slots | table updates (int64 flat table
        # indices, then int32 blocks). The updates come last: their count is
        # known only after the bookkeeping, and a wave takes at most one new
        # block per request. Everything before them sits at offsets fixed by
        # the batch shape, so their device views are built once per shape.
        # q and the lengths lead, so that the split decode below can upload
        # them and start before k, v and the bookkeeping are done.
        okey = (n, hq, hkv, d, dt, kdt)
        offs = self._offsets.get(okey)
        if offs is None:
            qb = n * hq * d * dt.itemsize
            kb = n * hkv * d * kdt.itemsize
            o_i = _align(qb)
            o_k = o_i + _align(8 * n)
            o_v = o_k + _align(kb)
            o_w = o_v + _align(kb)
            offs = self._offsets[okey] = (qb, kb, o_i, o_k, o_v, o_w, o_w + 8 * n)
        qb, kb, o_i, o_k, o_v, o_w, o_u = offs
        nu_max = self.tables.pending_count() + n
        buf = self._staging("wave", (o_u + 12 * nu_max,), torch.uint8)
        bnp = self._stage_np["wave"]
        # Position of each request's new token in this layer: its cached
        # length (a request whose blocks are full takes one more first).
        if rows is None:  # the requests' table rows
            rows = np.fromiter(map(_get_row, reqs), dtype=np.int64, count=n)
        pos = self._lens[rows, layer]
        narrow = bnp[o_i:o_i + 8 * n].view(np.int32)
        narrow[n:] = rows
        max_old = int(pos.max())
        kp, vp = self._layer_pools[layer]
        # The split decode (partials over the cached tokens now, the new token
        # merged in by the reduce later) lets the GPU attend while the host
        # stages k and v and does the bookkeeping. Short contexts keep the
        # single-pass fused launch, fp8 pools and a forced split-K their own.
        skey = (n, hq)
        split_ok = self._split_ok.get(skey)
        if split_ok is None:
            split_ok = self._split_ok[skey] = (not self._fp8 and
                                               kernels.append_fusable_shape(hq, kp, n))
        split = split_ok and self.partition_size is None and max_old + 1 > 512
        stream = torch.cuda.current_stream(self.device)
        upd: list = []
        applied = False
        issued = False  # a kernel that reads the device staging is queued
        h1 = False  # the split decode's first upload is issued, its second not
        direct = None  # the pinned result tensor the merge writes, if any
        try:
            if self._dstage_free is not None and self._dstage_stream != stream.cuda_stream:
                stream.wait_event(self._dstage_free)  # the previous wave's kernels read it
            total_max = o_u + 12 * nu_max
            if self._dstage is None or self._dstage.numel() < total_max:
                self._dstage = torch.empty(max(2 * total_max, 1 << 20), dtype=torch.uint8,
                                           device=self.device)
                self._views.clear()
            if self._stage_done is None:
                self._stage_done = torch.cuda.Event()
            vkey = (n, hq, hkv, d, dt, kdt)
            views = self._views.get(vkey)
            if views is None:
                narrow_dev = self._dstage[o_i:o_i + 8 * n].view(torch.int32)
                hb = self._stage["wave"]
                e = o_u + 12 * n  # end of the uploads with up to n table updates
                views = (self._dstage[:qb].view(dt).view(n, hq, d),
                         self._dstage[o_k:o_k + kb].view(kdt).view(n, hkv, d),
                         self._dstage[o_v:o_v + kb].view(kdt).view(n, hkv, d),
                         narrow_dev[:n], narrow_dev[n:],
                         self._dstage[o_w:o_u].view(torch.int64),
                         # (device, host) byte ranges of the uploads: q and
                         # the integers, the integers alone, the rest, all
                         (self._dstage[:o_k], hb[:o_k]), (self._dstage[o_i:o_k], hb[o_i:o_k]),
                         (self._dstage[o_k:e], hb[o_k:e]), (self._dstage[:e], hb[:e]))
                self._views[vkey] = views
            self._filled_host = self._gathered = False
            q = self._fill(qs, hq, d, dt, buf[:qb])
            q_host = self._filled_host
            q_same = self._gathered and dt == q0.dtype  # every query: a host tensor of q0's dtype
            q_staged = q is None  # the queries are in the pinned buffer
            if split:
                # Upload q, the cached lengths and the rows right away.
                narrow[:n] = pos
                dst, src = views[6] if q_staged else views[7]
                dst.copy_(src, non_blocking=True)
                h1 = True
                if self._h1_done is None:
                    self._h1_done = torch.cuda.Event()
                    self._up_done = torch.cuda.Event()
                    self._up_stream = torch.cuda.Stream(device=self.device)
                self._h1_done.record(stream)
            q = views[0] if q_staged else q
            ctx_dev, rows_dev, slots_dev = views[3], views[4], views[5]
            to_host = (not qs.is_cuda) if packed else (q_host or all(not t.is_cuda for t in qs))
            if to_host:
                # The call waits for its results: the output buffer is free
                # again when it returns.
                if self._dout is None or self._dout.numel() < q.numel() or \
                        self._dout.dtype != dt:
                    self._dout = torch.empty(q.numel(), dtype=dt, device=self.device)
                ctx_out = self._dout[:q.numel()].view(q.shape)
            else:
                ctx_out = torch.empty_like(q)

            def table():
                if rows_first is not None:
                    if rows_first >= 0:
                        return self.tables.rows_range(rows_first, n)
                elif rows[-1] - rows[0] == n - 1 and (n < 3 or bool((np.diff(rows) == 1).all())):
                    return self.tables.rows_range(int(rows[0]), n)
                return self.tables.rows(rows.tolist(), rows_dev)

            launch = None
            if split:
                # Attend over the cached tokens.
                bt = table()
                lkey = ("split", n, hq, layer, float(score_scale), dt, q.stride())
                launch = self._launches.get(lkey)
                if launch is None:
                    if len(self._launches) >= 256:
                        self._launches.clear()
                    launch = kernels.SplitAppendDecode(ctx_out, q, kp, vp, bt, ctx_dev, bs,
                                                       max_old, scale=score_scale)
                    self._launches[lkey] = launch
                else:
                    launch.update(ctx_out, q, bt, ctx_dev, max_old)
                launch.partials(stream.cuda_stream)
                issued = True

            k = self._fill(ks, hkv, d, kdt, buf[o_k:o_k + kb])
            v = self._fill(vs, hkv, d, kdt, buf[o_v:o_v + kb])
            full = np.nonzero(pos >= (self._nblk[rows] << self._bshift))[0].tolist()
            if len(full) > len(self.free_blocks):
                raise RuntimeError("OOM during append")
            for i in full:
                self._grow_request(reqs[i])
            slots = self._htab[rows, pos >> self._bshift] * bs + (pos & (bs - 1))
            lens = pos + 1
            self._lens[rows, layer] = lens
            upd = self.tables.take_pending()
            nu = len(upd)
            total = o_u + 12 * nu
            bnp[o_w:o_u].view(np.int64)[:] = slots
            if nu:
                flat, blocks = self.tables.flat_updates(upd)
                bnp[o_u:o_u + 8 * nu].view(np.int64)[:] = flat
                bnp[o_u + 8 * nu:total].view(np.int32)[:] = blocks
            k = views[1] if k is None else k
            v = views[2] if v is None else v
            if split:
                # The rest (k, v, slots and table updates) on the copy stream,
                # after the first upload and after the kernels of the previous
                # wave that read the device staging; then merge the new tokens
                # in (the reduce also writes their rows at the slots).
                up = self._up_stream
                up.wait_event(self._h1_done)
                if self._dstage_free is not None:
                    up.wait_event(self._dstage_free)
                dst, src = views[8] if nu <= n else (self._dstage[o_k:total], buf[o_k:total])
                with torch.cuda.stream(up):
                    dst.copy_(src, non_blocking=True)
                self._up_done.record(up)
                self._stage_done.record(up)  # both uploads (up waited for the first)
                h1 = False
                stream.wait_event(self._up_done)
                if nu:
                    self.tables.apply_flat(self._dstage[o_u:o_u + 8 * nu].view(torch.int64),
                                           self._dstage[o_u + 8 * nu:total].view(torch.int32))
                applied = True
                # Results that go to the host in the queries' dtype are
                # written by the merge straight into the pinned tensor the
                # call returns, where the device can address it: no copy back.
                if to_host and dt == q0.dtype and q0.device.type == "cpu" and (packed or q_same):
                    direct = torch.empty((n, 1, hq, d), dtype=dt, pin_memory=True)
                    addr = _native.mapped_device_address(direct.data_ptr())
                    if addr is None:
                        direct = None
                launch.reduce(k, v, slots_dev, stream.cuda_stream,
                              out_address=addr if direct is not None else None)
            else:
                narrow[:n] = lens
                dst, src = views[9] if nu <= n else (self._dstage[:total], buf[:total])
                dst.copy_(src, non_blocking=True)
                self._stage_done.record(stream)
                if nu:
                    self.tables.apply_flat(self._dstage[o_u:o_u + 8 * nu].view(torch.int64),
                                           self._dstage[o_u + 8 * nu:total].view(torch.int32))
                applied = True
                bt = table()
                max_len = int(lens.max())
                # Append and decode in one call (the new rows land at
                # position lens - 1, the slots computed above) where the
                # fused kernel covers the shape; the launch is built once per
                # batch shape, layer and scale (the pools are never
                # reallocated).
                lkey = (n, hq, layer, float(score_scale), dt, kdt, q.stride(), k.stride())
                launch = self._launches.get(lkey) if self.partition_size is None else None
                if launch is not None:
                    launch.update(ctx_out, q, bt, ctx_dev, max_len, k, v)
                    issued = True
                    launch.launch(stream.cuda_stream)
                elif self.partition_size is None and kernels.append_fusable(q, kp, n):
                    if len(self._launches) >= 256:
                        self._launches.clear()
                    launch = kernels.AppendDecodeLaunch(ctx_out, q, kp, vp, bt, ctx_dev, bs,
                                                        max_len, k, v, scale=score_scale)
                    self._launches[lkey] = launch
                    issued = True
                    launch.launch(stream.cuda_stream)
                else:
                    issued = True
                    self._append(k, v, layer, slots_dev)
                    kernels.paged_attention(ctx_out, q, kp, vp, bt, ctx_dev, bs, max_len,
                                            scale=score_scale,
                                            partition_size=self.partition_size,
                                            k_scale=self.k_scales, v_scale=self.v_scales)
        except BaseException:
            self._lens[rows, layer] = pos
            if not applied:
                self.tables.requeue(upd)
            if h1:  # the pinned buffer is read until the first upload is done
                self._stage_done.record(stream)
            if direct is not None:  # a merge may be writing the pinned result: let it end
                stream.synchronize()
            raise
        finally:
            if issued:
                if self._dstage_free is None:
                    self._dstage_free = torch.cuda.Event()
                self._dstage_free.record(stream)
                self._dstage_stream = stream.cuda_stream
        if layer == self.num_layers - 1:
            self._ctx[rows] += 1
        self.stats["decode_items"] += n
        self.stats["decode_launches"] += 1
        # Outputs in each query's dtype and on its device: one copy for the
        # batch when the queries agree (the node's case), per item otherwise.
        qdt, qdev = q0.dtype, q0.device
        if direct is not None:
            out = direct if packed else list(direct.unbind(0))
            stream.synchronize()
            return out
        if packed or q_same or (all(t.dtype == qdt for t in qs) and (
                (qdev.type == "cpu" and to_host) or all(t.device == qdev for t in qs))):
            if qdev.type == "cpu":
                # One copy into pinned host memory (a pageable destination goes
                # through the driver's bounce buffer at a fraction of the rate),
                # then wait for it.
                res = torch.empty((n, 1, hq, d), dtype=qdt, pin_memory=True)
                res.view(n, hq, d).copy_(ctx_out if dt == qdt else ctx_out.to(qdt),
                                         non_blocking=True)
                # The per-item views are built while the GPU works.
                out = res if packed else list(res.unbind(0))
                stream.synchronize()
                return out
            res = ctx_out.to(device=qdev, dtype=qdt).view(n, 1, hq, d)
            return res if packed else list(res.unbind(0))
        return [ctx_out[i:i + 1].to(device=t.device, dtype=t.dtype) for i, t in enumerate(qs)]

    def get_context_len(self, request_id: str) -> int:
        return int(self._ctx[self.requests[request_id].row])

    def free_request(self, request_id: str) -> None:
        req = self.requests.pop(request_id, None)
        if req is not None:
            self.free_blocks.extend(req.blocks)
            self.tables.remove(req.row)

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

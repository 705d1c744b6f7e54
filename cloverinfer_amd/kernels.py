"""Tensor-level entry points over the C ABI (the ``clover_kernels`` mirror).

``paged_attention`` keeps the reference binding's signature and meaning
(src/kernels/csrc/manager.cpp:19-38): the caller allocates ``out``, sizes come
from the tensors, the call is asynchronous on the current stream and returns
nothing. The other functions are the new operations of the hot path. Every
call goes through ``libclover_attn.so``; tensors must live on a HIP device.
"""
from __future__ import annotations

import functools
import math
import threading

import torch

from . import _native

_DTYPES = {
    torch.float32: _native.CLV_F32,
    torch.float16: _native.CLV_F16,
    torch.bfloat16: _native.CLV_BF16,
}

# Tokens per split-K partition when the caller does not choose one.
DEFAULT_PARTITION = 512

_ws_lock = threading.Lock()
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
# Hand-outs of each stream's workspace so far: a launch that keeps partials in
# it between two calls (SplitAppendDecode) can tell whether another launch
# took the same buffer in between.
_ws_epochs: dict[tuple[int, int], int] = {}
_num_cus: dict[int, int] = {}


# fp8 pool dtype: OCP e4m3 (the format gfx950's conversions use), one scale
# per kv head.
FP8 = torch.float8_e4m3fn


def kv_scales(scale, num_kv_heads: int, device: torch.device) -> torch.Tensor:
    """Per-kv-head fp32 scales of an fp8 pool as a device tensor: a number (the
    same for every head), a sequence or a tensor of num_kv_heads values."""
    if scale is None:
        raise ValueError("fp8 pools need k_scale and v_scale")
    if isinstance(scale, torch.Tensor) and scale.device == device and \
            scale.dtype == torch.float32 and scale.shape == (num_kv_heads,) and scale.is_contiguous():
        return scale  # already a device tensor (not re-validated: that would synchronise)
    t = torch.as_tensor(scale, dtype=torch.float32, device="cpu")
    if t.dim() == 0:
        t = t.expand(num_kv_heads)
    if t.shape != (num_kv_heads,):
        raise ValueError(f"scales must be a number or [{num_kv_heads}] values")
    if not bool(torch.isfinite(t).all()) or not bool((t > 0).all()):
        raise ValueError("scales must be positive and finite")
    return t.to(device=device).contiguous()


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}; expected float32, float16 or bfloat16")


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            "paged-attention kernels run on a HIP device only; got tensors on "
            f"{dev} (there is no CPU fallback)"
        )
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}, found one on {t.device}")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError(
            "k_cache and v_cache must both be [num_blocks, block_size, num_kv_heads, head_dim]"
        )
    if k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share strides")
    if k_cache.stride(3) != 1:
        raise ValueError("the cache head_dim must be contiguous")
    if v_cache.dtype != k_cache.dtype:
        raise ValueError("k_cache and v_cache dtypes differ")


def num_compute_units(dev: torch.device) -> int:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _num_cus:
        _num_cus[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _num_cus[idx]


def choose_partition(num_seqs: int, num_kv_heads: int, group: int, max_context_len: int,
                     num_cus: int) -> int:
    """Split-K partition size (0 = single pass) for a decode batch.

    A single pass launches one workgroup per (sequence, kv head, group
    chunk); it is used when that already gives every compute unit several
    workgroups and contexts are short enough to stay balanced.
    """
    if max_context_len <= DEFAULT_PARTITION:
        return 0
    single = num_seqs * num_kv_heads * ((group + 15) // 16)
    if single >= 4 * num_cus:
        return 0
    return DEFAULT_PARTITION


def splitk_workspace(dev: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor:
    """A cached, grow-only uint8 workspace of at least ``nbytes`` for the
    current stream of ``dev`` (one per stream, so that launches on different
    streams never share partials); ``stream``: that stream's handle, when the
    caller has looked it up already."""
    return _workspace_lease(dev, nbytes, stream)[0]


def _workspace_lease(dev: torch.device, nbytes: int, stream: int | None = None):
    """:func:`splitk_workspace` plus the (stream key, hand-out count) that
    :func:`_workspace_reused` checks."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, stream if stream is not None else _stream(torch.device("cuda", idx)))
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
            _workspaces[key] = ws
        epoch = _ws_epochs[key] = _ws_epochs.get(key, 0) + 1
    return ws, key, epoch


def _workspace_reused(ws: torch.Tensor, key, epoch: int) -> bool:
    """Whether the stream's workspace ``ws``, leased at ``epoch``, has been
    handed out again since (a grown, different buffer leaves ``ws`` alone)."""
    with _ws_lock:
        return _workspaces.get(key) is ws and _ws_epochs.get(key) != epoch


def _decode_args(out, q, k_cache, v_cache, block_tables, context_lens, block_size,
                 max_context_len, scale) -> _native.DecodeArgs:
    if q.dim() != 3 or out.shape != q.shape:
        raise ValueError("q and out must both be [num_seqs, num_heads, head_dim]")
    _check_cache(k_cache, v_cache)
    num_seqs, num_heads, head_dim = q.shape
    num_blocks, bs, num_kv_heads, kd = k_cache.shape
    if kd != head_dim:
        raise ValueError(f"head_dim mismatch: q has {head_dim}, cache has {kd}")
    if bs != block_size:
        raise ValueError(f"block_size {block_size} does not match the cache ({bs})")
    if num_heads % num_kv_heads:
        raise ValueError(f"num_heads {num_heads} is not a multiple of num_kv_heads {num_kv_heads}")
    fp8 = k_cache.dtype == FP8
    if out.dtype != q.dtype or (q.dtype != k_cache.dtype and not fp8):
        raise ValueError("q, out and the caches must share one dtype")
    if fp8 and q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("fp8 pools need float16 or bfloat16 queries")
    if q.stride(2) != 1 or out.stride(2) != 1:
        raise ValueError("q and out need a contiguous head_dim")
    if block_tables.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise ValueError("block_tables and context_lens must be int32")
    if block_tables.dim() != 2 or block_tables.shape[0] != num_seqs or not block_tables.is_contiguous():
        raise ValueError("block_tables must be a contiguous [num_seqs, max_blocks_per_seq] tensor")
    if context_lens.shape != (num_seqs,) or not context_lens.is_contiguous():
        raise ValueError("context_lens must be a contiguous [num_seqs] tensor")
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    a = _native.DecodeArgs()
    a.out = out.data_ptr()
    a.q = q.data_ptr()
    a.k_cache = k_cache.data_ptr()
    a.v_cache = v_cache.data_ptr()
    a.block_tables = block_tables.data_ptr()
    a.context_lens = context_lens.data_ptr()
    a.q_stride_seq, a.q_stride_head = q.stride(0), q.stride(1)
    a.out_stride_seq, a.out_stride_head = out.stride(0), out.stride(1)
    a.kv_stride_block, a.kv_stride_token, a.kv_stride_head = k_cache.stride()[:3]
    a.num_seqs, a.num_heads, a.num_kv_heads, a.head_dim = num_seqs, num_heads, num_kv_heads, head_dim
    a.block_size = block_size
    a.max_blocks_per_seq = block_tables.shape[1]
    a.max_context_len = int(max_context_len)
    a.num_blocks = num_blocks
    a.dtype = _dtype_code(q)
    a.scale = float(scale)
    return a


def decode_args(out: torch.Tensor, q: torch.Tensor, k_cache: torch.Tensor,
                v_cache: torch.Tensor, block_tables: torch.Tensor, context_lens: torch.Tensor,
                block_size: int, max_context_len: int,
                scale: float | None = None) -> _native.DecodeArgs:
    """Validated C-ABI argument block of a paged decode (tensors stay owned
    by the caller and must outlive every launch made with it)."""
    _require_device(out, q, k_cache, v_cache, block_tables, context_lens)
    return _decode_args(out, q, k_cache, v_cache, block_tables, context_lens, block_size,
                        max_context_len, scale)


# Largest num_seqs * num_kv_heads * ceil(group / 16) of the balanced decode.
BALANCED_MAX_SEGMENTS = 4096


def balanced_supported(a: _native.DecodeArgs) -> bool:
    group = a.num_heads // a.num_kv_heads
    nseg = a.num_seqs * a.num_kv_heads * ((group + 15) // 16)
    return (a.dtype in (_native.CLV_F16, _native.CLV_BF16, _native.CLV_F32)
            and a.head_dim in (64, 128) and a.block_size >= 4 and nseg <= BALANCED_MAX_SEGMENTS)


def choose_schedule(a: _native.DecodeArgs, num_cus: int) -> tuple[str, int]:
    """Decode schedule for a batch: ("single", 0), ("balanced", 0) or
    ("split", partition_size).

    Contexts of at most DEFAULT_PARTITION tokens take the single pass (one
    workgroup per (sequence, kv head, 16 query heads), no merge): its longest
    workgroup is short, so the load imbalance the balanced schedule removes
    costs less than the balanced schedule's merge launch. Longer contexts
    take the balanced stream decode where it applies, else split-K or the
    single pass by :func:`choose_partition`."""
    if a.max_context_len <= DEFAULT_PARTITION:
        return "single", 0
    if balanced_supported(a):
        return "balanced", 0
    part = choose_partition(a.num_seqs, a.num_kv_heads, a.num_heads // a.num_kv_heads,
                            a.max_context_len, num_cus)
    return ("split", part) if part > 0 and a.max_context_len > part else ("single", 0)


def paged_attention(out: torch.Tensor, q: torch.Tensor, k_cache: torch.Tensor,
                    v_cache: torch.Tensor, block_tables: torch.Tensor,
                    context_lens: torch.Tensor, block_size: int, max_context_len: int,
                    scale: float | None = None, partition_size: int | None = None,
                    num_waves: int = 0, k_scale=None, v_scale=None) -> None:
    """``out[s,h] = softmax(scale * q[s,h] . K^T) V`` over each sequence's paged context.

    Same arguments as the reference op (src/kernels/csrc/manager.cpp:19-27);
    ``scale`` defaults to 1/sqrt(head_dim) as in src/kernels/csrc/attention.cu:60.
    GQA follows from ``k_cache.shape[2] < q.shape[1]``. ``partition_size``:
    None picks the schedule (:func:`choose_schedule`: the single pass for
    contexts up to 512 tokens, else the balanced stream decode where it
    applies; a positive ``num_waves`` asks for the balanced decode with that
    many waves, 0 = the device default), 0 forces a single pass per
    (sequence, kv head), a positive multiple of 32 forces split-K with that
    many tokens per partition.

    fp8 pools (``k_cache.dtype == FP8``): K = e4m3 * ``k_scale``, V = e4m3 *
    ``v_scale`` (numbers or per-kv-head values), balanced schedule only
    (head_dim 128, block_size >= 16), ``partition_size`` must be None.
    """
    dev = _require_device(out, q, k_cache, v_cache, block_tables, context_lens)
    a = _decode_args(out, q, k_cache, v_cache, block_tables, context_lens, block_size,
                     max_context_len, scale)
    lib = _native.load()
    stream = _stream(dev)
    if k_cache.dtype == FP8:
        if partition_size is not None:
            raise ValueError("fp8 pools use the balanced schedule (partition_size=None)")
        ks = kv_scales(k_scale, a.num_kv_heads, dev)
        vs = kv_scales(v_scale, a.num_kv_heads, dev)
        num_waves = num_waves or lib.clv_default_num_waves_fp8()
        nbytes = lib.clv_balanced_workspace_bytes(a.num_seqs, a.num_heads, a.num_kv_heads,
                                                  a.head_dim, num_waves)
        ws = splitk_workspace(dev, nbytes, stream)
        _native.check(lib.clv_paged_decode_fp8(a, ks.data_ptr(), vs.data_ptr(), num_waves,
                                               ws.data_ptr(), ws.numel(), stream),
                      "clv_paged_decode_fp8")
        return
    if partition_size is None:
        if num_waves > 0 and balanced_supported(a):
            mode = "balanced"  # an explicit wave count asks for the balanced schedule
        else:
            mode, partition_size = choose_schedule(a, num_compute_units(dev))
        if mode == "balanced":
            nbytes = lib.clv_balanced_workspace_bytes(a.num_seqs, a.num_heads, a.num_kv_heads,
                                                      a.head_dim, num_waves)
            ws = splitk_workspace(dev, nbytes, stream)
            _native.check(lib.clv_paged_decode_balanced(a, num_waves, ws.data_ptr(), ws.numel(),
                                                        stream), "clv_paged_decode_balanced")
            return
    if partition_size == 0 or a.max_context_len <= partition_size:
        _native.check(lib.clv_paged_decode(a, stream), "clv_paged_decode")
        return
    ws = splitk_workspace(dev, workspace_bytes(a, partition_size), stream)
    _native.check(
        lib.clv_paged_decode_splitk(a, partition_size, ws.data_ptr(), ws.numel(), stream),
        "clv_paged_decode_splitk",
    )


class AppendDecodeLaunch:
    """A validated fused append + decode (clv_paged_decode_append) that can
    be issued again: a caller whose batch keeps its shapes, pools and scale
    from call to call (the AttentionNode's layer after layer) builds it once
    and, per call, points it at that call's buffers with :meth:`update` (no
    checks: the new tensors must have the shapes and strides of the ones it
    was built with) before :meth:`launch`."""

    def __init__(self, out: torch.Tensor, q: torch.Tensor, k_cache: torch.Tensor,
                 v_cache: torch.Tensor, block_tables: torch.Tensor, context_lens: torch.Tensor,
                 block_size: int, max_context_len: int, key_new: torch.Tensor,
                 value_new: torch.Tensor, scale: float | None = None, num_waves: int = 0):
        self.device = _require_device(out, q, k_cache, v_cache, block_tables, context_lens,
                                      key_new, value_new)
        a = _decode_args(out, q, k_cache, v_cache, block_tables, context_lens, block_size,
                         max_context_len, scale)
        if not balanced_supported(a):
            raise NotImplementedError("paged_attention_append covers the balanced decode's shapes only")
        shape = (a.num_seqs, a.num_kv_heads, a.head_dim)
        if key_new.shape != shape or value_new.shape != shape:
            raise ValueError(f"key_new/value_new must be {shape}, got {tuple(key_new.shape)} and "
                             f"{tuple(value_new.shape)}")
        if key_new.dtype != k_cache.dtype or value_new.dtype != k_cache.dtype:
            raise ValueError("key_new/value_new dtype must match the cache dtype")
        key_new, value_new = self._rows(key_new, value_new)
        self.args = a
        self.num_waves = num_waves
        # The launch holds the tensors whose addresses it passes (a contiguous
        # copy made above would otherwise be freed, and its memory reused,
        # before the kernel reads it); update() replaces them.
        self._key_new, self._value_new = key_new, value_new
        self.key_ptr, self.value_ptr = key_new.data_ptr(), value_new.data_ptr()
        self.kv_new_strides = (key_new.stride(0), key_new.stride(1))
        lib = _native.load()
        self.workspace_bytes = lib.clv_balanced_workspace_bytes(a.num_seqs, a.num_heads,
                                                                a.num_kv_heads, a.head_dim,
                                                                num_waves)
        self._fn = lib.clv_paged_decode_append

    @staticmethod
    def _rows(key_new: torch.Tensor, value_new: torch.Tensor):
        """The new rows as the kernel reads them: key and value with one
        pair of (token, head) strides and a contiguous head_dim, copied to
        contiguous tensors otherwise."""
        if key_new.stride() != value_new.stride() or key_new.stride(2) != 1:
            key_new, value_new = key_new.contiguous(), value_new.contiguous()
        return key_new, value_new

    def update(self, out: torch.Tensor, q: torch.Tensor, block_tables: torch.Tensor,
               context_lens: torch.Tensor, max_context_len: int, key_new: torch.Tensor,
               value_new: torch.Tensor) -> None:
        """Point the launch at this call's buffers. ``out``/``q``/tables must
        have the shapes and strides of the build; new rows whose strides
        differ from the build's are copied to contiguous tensors, and a launch
        whose strides the copy still does not match raises ValueError."""
        key_new, value_new = self._rows(key_new, value_new)
        if (key_new.stride(0), key_new.stride(1)) != self.kv_new_strides:
            raise ValueError(f"key_new/value_new strides {key_new.stride()} differ from the "
                             f"launch's {self.kv_new_strides}")
        a = self.args
        a.out, a.q = out.data_ptr(), q.data_ptr()
        a.block_tables, a.max_blocks_per_seq = block_tables.data_ptr(), block_tables.shape[1]
        a.context_lens = context_lens.data_ptr()
        a.max_context_len = int(max_context_len)
        self._key_new, self._value_new = key_new, value_new
        self.key_ptr, self.value_ptr = key_new.data_ptr(), value_new.data_ptr()

    def launch(self, stream: int | None = None) -> None:
        """Issue on the current stream (with that stream's workspace);
        ``stream``: the current stream's handle, when the caller has it."""
        if stream is None:
            stream = _stream(self.device)
        ws = splitk_workspace(self.device, self.workspace_bytes, stream)
        _native.check(self._fn(self.args, self.key_ptr, self.value_ptr, *self.kv_new_strides,
                               self.num_waves, ws.data_ptr(), ws.numel(), stream),
                      "clv_paged_decode_append")

    def bind(self):
        """A callable that reissues this launch, as it stands now, on the
        stream that is current when bind() is called (and that stream's
        workspace), with no further Python work beyond the C call (for a
        caller that replays one step over fixed buffers); it returns the C
        status code. The callable holds a copy of the argument block and
        the tensors it points into that the launch owns (the new rows if
        they were copied, the workspace), so a later :meth:`update` or a
        grown workspace does not change or free what it reads."""
        ws = splitk_workspace(self.device, self.workspace_bytes)
        a = type(self.args).from_buffer_copy(self.args)
        call = functools.partial(self._fn, a, self.key_ptr, self.value_ptr,
                                 *self.kv_new_strides, self.num_waves, ws.data_ptr(), ws.numel(),
                                 _stream(self.device))
        call.keepalive = (self._key_new, self._value_new, ws)
        return call


class SplitAppendDecode:
    """One decode step of the append-then-attend protocol in two launches,
    for a caller that can start the decode before the new key/value rows are
    at hand: :meth:`partials` (clv_balanced_partials) attends over the
    ``context_lens[s]`` cached tokens, :meth:`reduce`
    (clv_balanced_reduce_append) merges in each sequence's new token and
    writes its rows at the caller's slots (reshape_and_cache semantics:
    negative slots are skipped; the block tables need not name the new
    token's block yet). The output equals :func:`paged_attention_append`'s
    over ``context_lens + 1`` tokens, up to the fp32 rounding of the new
    token's score. Built once per batch shape and pointed at each call's
    buffers with :meth:`update`, like :class:`AppendDecodeLaunch`; the
    balanced decode's shapes with fp32/fp16/bf16 pools. The partials live in
    the stream's workspace, which every decode of this module on that stream
    uses: between :meth:`partials` and :meth:`reduce` run no other decode
    call on the same stream (:meth:`reduce` raises if one ran)."""

    def __init__(self, out: torch.Tensor, q: torch.Tensor, k_cache: torch.Tensor,
                 v_cache: torch.Tensor, block_tables: torch.Tensor, context_lens: torch.Tensor,
                 block_size: int, max_context_len: int, scale: float | None = None,
                 num_waves: int = 0):
        self.device = _require_device(out, q, k_cache, v_cache, block_tables, context_lens)
        a = _decode_args(out, q, k_cache, v_cache, block_tables, context_lens, block_size,
                         max_context_len, scale)
        if not balanced_supported(a):
            raise NotImplementedError("the split decode covers the balanced decode's shapes only")
        self.args = a
        self.num_waves = num_waves
        self.new_shape = (a.num_seqs, a.num_kv_heads, a.head_dim)
        self.cache_dtype = k_cache.dtype
        lib = _native.load()
        self.workspace_bytes = lib.clv_balanced_workspace_bytes(a.num_seqs, a.num_heads,
                                                                a.num_kv_heads, a.head_dim,
                                                                num_waves)
        self._partials_fn = lib.clv_balanced_partials
        self._reduce_fn = lib.clv_balanced_reduce_append
        self._ws = None

    def update(self, out: torch.Tensor, q: torch.Tensor, block_tables: torch.Tensor,
               context_lens: torch.Tensor, max_context_len: int) -> None:
        """Point the launch at this call's buffers (the shapes and strides of
        the build; not checked)."""
        a = self.args
        a.out, a.q = out.data_ptr(), q.data_ptr()
        a.block_tables, a.max_blocks_per_seq = block_tables.data_ptr(), block_tables.shape[1]
        a.context_lens = context_lens.data_ptr()
        a.max_context_len = int(max_context_len)

    def partials(self, stream: int | None = None) -> None:
        """The decode over the cached tokens, on the current stream (or the
        stream handle given)."""
        if stream is None:
            stream = _stream(self.device)
        # The merge reads what this launch writes: it keeps the workspace
        # (the stream's, which any other decode of this module on the same
        # stream also takes: reduce() checks that none did in between).
        ws, key, epoch = _workspace_lease(self.device, self.workspace_bytes, stream)
        self._ws = None
        _native.check(self._partials_fn(self.args, self.num_waves, ws.data_ptr(), ws.numel(),
                                        stream), "clv_balanced_partials")
        self._ws, self._ws_lease = ws, (key, epoch)

    def reduce(self, key_new: torch.Tensor, value_new: torch.Tensor, slots: torch.Tensor,
               stream: int | None = None, out_address: int | None = None) -> None:
        """Merge in sequence s's new token (key_new/value_new[s], [num_kv_heads,
        head_dim] in the cache dtype) and write its rows at ``slots[s]``
        (int64); after :meth:`partials` on the same stream. ``out_address``:
        write the result there instead of the build's output, with that
        output's strides (for instance the device address of pinned host
        memory, :func:`_native.mapped_device_address`, so that the result
        needs no copy back)."""
        if self._ws is None:
            raise RuntimeError("reduce() needs the partials of this launch first")
        if _workspace_reused(self._ws, *self._ws_lease):
            raise RuntimeError("another decode on this stream took the workspace that holds "
                               "this launch's partials: call partials() again before reduce()")
        if key_new.shape != self.new_shape or value_new.shape != self.new_shape:
            raise ValueError(f"key_new/value_new must be {self.new_shape}, got "
                             f"{tuple(key_new.shape)} and {tuple(value_new.shape)}")
        if key_new.dtype != self.cache_dtype or value_new.dtype != self.cache_dtype:
            raise ValueError("key_new/value_new dtype must match the cache dtype")
        if slots.dtype != torch.int64 or slots.dim() != 1 or slots.shape[0] < self.new_shape[0] \
                or slots.stride(0) != 1:
            raise ValueError("slots must be a contiguous int64 vector, one slot per sequence")
        if _require_device(key_new, value_new, slots) != self.device:
            raise ValueError(f"key_new/value_new/slots must be on {self.device}")
        key_new, value_new = AppendDecodeLaunch._rows(key_new, value_new)
        if stream is None:
            stream = _stream(self.device)
        ws = self._ws
        a = self.args
        if out_address is not None:
            a = type(a).from_buffer_copy(a)
            a.out = out_address
        _native.check(self._reduce_fn(a, key_new.data_ptr(), value_new.data_ptr(),
                                      key_new.stride(0), key_new.stride(1), slots.data_ptr(),
                                      self.num_waves, ws.data_ptr(), ws.numel(), stream),
                      "clv_balanced_reduce_append")


def paged_attention_append(out: torch.Tensor, q: torch.Tensor, k_cache: torch.Tensor,
                           v_cache: torch.Tensor, block_tables: torch.Tensor,
                           context_lens: torch.Tensor, block_size: int, max_context_len: int,
                           key_new: torch.Tensor, value_new: torch.Tensor,
                           scale: float | None = None, num_waves: int = 0) -> None:
    """One decode step of the append-then-attend protocol in one call
    (clv_paged_decode_append): sequence s's ``key_new[s]``/``value_new[s]``
    ([num_kv_heads, head_dim]) are written at its position
    ``context_lens[s] - 1`` (slot from its block-table row), then ``out`` =
    :func:`paged_attention` over all ``context_lens[s]`` tokens. Equal to
    :func:`reshape_and_cache` with those slots followed by
    :func:`paged_attention` with the schedule :func:`choose_schedule` picks:
    batches whose contexts fit the single pass (at most 512 tokens, at most 16
    query heads per kv head, ``num_waves`` 0) are one single-pass launch,
    longer ones the balanced decode. Covers the shapes of the balanced decode
    (:func:`append_fusable`), raises otherwise."""
    AppendDecodeLaunch(out, q, k_cache, v_cache, block_tables, context_lens, block_size,
                       max_context_len, key_new, value_new, scale, num_waves).launch()


def append_fusable(q: torch.Tensor, k_cache: torch.Tensor, num_seqs: int) -> bool:
    """Whether :func:`paged_attention_append` covers this decode shape."""
    return append_fusable_shape(q.shape[1], k_cache, num_seqs)


def append_fusable_shape(num_heads: int, k_cache: torch.Tensor, num_seqs: int) -> bool:
    """:func:`append_fusable` for ``num_heads`` query heads (also the shapes
    of :class:`SplitAppendDecode`)."""
    hq, hkv, d = num_heads, k_cache.shape[2], k_cache.shape[3]
    nseg = num_seqs * hkv * ((hq // hkv + 15) // 16)
    return (k_cache.dtype in (torch.float16, torch.bfloat16, torch.float32) and d in (64, 128)
            and k_cache.shape[1] >= 4 and nseg <= BALANCED_MAX_SEGMENTS)


def workspace_bytes(a: _native.DecodeArgs, partition_size: int) -> int:
    return _native.load().clv_splitk_workspace_bytes(a.num_seqs, a.num_heads, a.head_dim,
                                                     a.max_context_len, partition_size)


def paged_decode_partials(a: _native.DecodeArgs, partition_size: int, workspace: torch.Tensor,
                          stream: int) -> None:
    """First half of split-K (partials into ``workspace``), see clv_paged_decode_partials."""
    _native.check(_native.load().clv_paged_decode_partials(
        a, partition_size, workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        stream), "clv_paged_decode_partials")


def balanced_workspace_bytes(a: _native.DecodeArgs, num_waves: int = 0) -> int:
    return _native.load().clv_balanced_workspace_bytes(a.num_seqs, a.num_heads, a.num_kv_heads,
                                                       a.head_dim, num_waves)


def balanced_partials(a: _native.DecodeArgs, num_waves: int, workspace: torch.Tensor,
                      stream: int) -> None:
    """First half of the balanced decode (stream kernel), see clv_balanced_partials."""
    _native.check(_native.load().clv_balanced_partials(
        a, num_waves, workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        stream), "clv_balanced_partials")


def balanced_reduce(a: _native.DecodeArgs, num_waves: int, workspace: torch.Tensor,
                    stream: int) -> None:
    """Second half of the balanced decode (merge into ``out``), see clv_balanced_reduce."""
    _native.check(_native.load().clv_balanced_reduce(
        a, num_waves, workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        stream), "clv_balanced_reduce")


def splitk_reduce(a: _native.DecodeArgs, partition_size: int, workspace: torch.Tensor,
                  stream: int) -> None:
    """Second half of split-K (merge into ``out``), see clv_splitk_reduce."""
    _native.check(_native.load().clv_splitk_reduce(
        a, partition_size, workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        stream), "clv_splitk_reduce")


def _cache_args(key, value, k_cache, v_cache, slot_mapping) -> _native.CacheArgs:
    _check_cache(k_cache, v_cache)
    num_blocks, bs, num_kv_heads, head_dim = k_cache.shape
    if key.dim() != 3 or value.shape != key.shape or key.shape[1:] != (num_kv_heads, head_dim):
        raise ValueError(
            f"key/value must be [num_tokens, {num_kv_heads}, {head_dim}], got "
            f"{tuple(key.shape)} and {tuple(value.shape)}"
        )
    fp8 = k_cache.dtype == FP8
    if value.dtype != key.dtype or (key.dtype != k_cache.dtype and not fp8):
        raise ValueError("key/value dtype must match the cache dtype")
    if key.stride(2) != 1 or value.stride(2) != 1:
        raise ValueError("key/value need a contiguous head_dim")
    if slot_mapping.dtype != torch.int64 or slot_mapping.shape != (key.shape[0],) \
            or not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be a contiguous int64 [num_tokens] tensor")
    a = _native.CacheArgs()
    a.key, a.value = key.data_ptr(), value.data_ptr()
    a.k_cache, a.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
    a.slot_mapping = slot_mapping.data_ptr()
    a.key_stride_token, a.key_stride_head = key.stride(0), key.stride(1)
    a.value_stride_token, a.value_stride_head = value.stride(0), value.stride(1)
    a.kv_stride_block, a.kv_stride_token, a.kv_stride_head = k_cache.stride()[:3]
    a.num_tokens = key.shape[0]
    a.num_kv_heads, a.head_dim, a.block_size, a.num_blocks = num_kv_heads, head_dim, bs, num_blocks
    a.dtype = _dtype_code(key)
    return a


def cache_args(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
               v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> _native.CacheArgs:
    """Validated C-ABI argument block of a KV append into fp32/fp16/bf16
    pools (the tensors stay owned by the caller and must outlive every launch
    made with it): a caller that appends into the same buffers every step
    builds it once and calls ``clv_reshape_and_cache`` with it directly."""
    _require_device(key, value, k_cache, v_cache, slot_mapping)
    if k_cache.dtype == FP8:
        raise ValueError("cache_args covers fp32/fp16/bf16 pools; fp8 pools take reshape_and_cache")
    return _cache_args(key, value, k_cache, v_cache, slot_mapping)


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                      k_scale=None, v_scale=None) -> None:
    """Write token i's ``key[i]``/``value[i]`` ([num_kv_heads, head_dim]) to cache slot
    ``slot_mapping[i]`` (= block*block_size + offset; negative slots are skipped).
    fp8 pools store e4m3(clamp(x / scale, -448, 448)) with per-kv-head
    ``k_scale``/``v_scale``."""
    dev = _require_device(key, value, k_cache, v_cache, slot_mapping)
    a = _cache_args(key, value, k_cache, v_cache, slot_mapping)
    if k_cache.dtype == FP8:
        num_kv_heads = k_cache.shape[2]
        ks = kv_scales(k_scale, num_kv_heads, dev)
        vs = kv_scales(v_scale, num_kv_heads, dev)
        _native.check(_native.load().clv_reshape_and_cache_fp8(a, ks.data_ptr(), vs.data_ptr(),
                                                               _stream(dev)),
                      "clv_reshape_and_cache_fp8")
        return
    _native.check(_native.load().clv_reshape_and_cache(a, _stream(dev)), "clv_reshape_and_cache")


def chunked_prefill(out: torch.Tensor, q: torch.Tensor, k_cache: torch.Tensor,
                    v_cache: torch.Tensor, block_tables: torch.Tensor,
                    context_lens: torch.Tensor, query_start_loc: torch.Tensor,
                    max_query_len: int | None, scale: float | None = None) -> None:
    """Causal attention of each sequence's new query rows over its paged context.

    Sequence s owns rows ``query_start_loc[s]:query_start_loc[s+1]`` of q/out;
    its new tokens are the last ones of its ``context_lens[s]`` cached tokens,
    and row i sees positions ``<= context_lens[s] - n_s + i``.
    ``max_query_len`` must be at least every chunk length n_s (it sizes the
    launch; a row i >= max_query_len of its chunk comes out as NaN, in every
    kernel form); None computes it from ``query_start_loc`` with one small
    device-to-host copy.
    """
    dev = _require_device(out, q, k_cache, v_cache, block_tables, context_lens, query_start_loc)
    _check_cache(k_cache, v_cache)
    if q.dim() != 3 or out.shape != q.shape:
        raise ValueError("q and out must both be [num_tokens, num_heads, head_dim]")
    num_tokens, num_heads, head_dim = q.shape
    num_blocks, bs, num_kv_heads, kd = k_cache.shape
    if kd != head_dim or num_heads % num_kv_heads:
        raise ValueError("q and the caches disagree on head_dim or the GQA grouping")
    fp8 = k_cache.dtype == FP8
    if out.dtype != q.dtype or (q.dtype != k_cache.dtype and not fp8):
        raise ValueError("q, out and the caches must share one dtype")
    if fp8 and q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("fp8 pools need float16 or bfloat16 queries")
    if q.stride(2) != 1 or out.stride(2) != 1:
        raise ValueError("q and out need a contiguous head_dim")
    num_seqs = context_lens.shape[0]
    for name, t, shape in (("context_lens", context_lens, (num_seqs,)),
                           ("query_start_loc", query_start_loc, (num_seqs + 1,))):
        if t.dtype != torch.int32 or t.shape != shape or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int32 tensor of shape {shape}")
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 \
            or block_tables.shape[0] != num_seqs or not block_tables.is_contiguous():
        raise ValueError("block_tables must be a contiguous int32 [num_seqs, max_blocks] tensor")
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    if max_query_len is None:
        max_query_len = int(query_start_loc.diff().max()) if num_seqs else 0
    a = _native.PrefillArgs()
    a.out, a.q = out.data_ptr(), q.data_ptr()
    a.k_cache, a.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
    a.block_tables = block_tables.data_ptr()
    a.context_lens = context_lens.data_ptr()
    a.query_start_loc = query_start_loc.data_ptr()
    a.q_stride_token, a.q_stride_head = q.stride(0), q.stride(1)
    a.out_stride_token, a.out_stride_head = out.stride(0), out.stride(1)
    a.kv_stride_block, a.kv_stride_token, a.kv_stride_head = k_cache.stride()[:3]
    a.num_seqs, a.num_tokens, a.num_heads, a.num_kv_heads = num_seqs, num_tokens, num_heads, num_kv_heads
    a.head_dim, a.block_size = head_dim, bs
    a.max_blocks_per_seq = block_tables.shape[1]
    a.max_query_len = int(max_query_len)
    a.num_blocks = num_blocks
    a.dtype = _dtype_code(q)
    a.scale = float(scale)
    _native.check(_native.load().clv_chunked_prefill(a, _stream(dev)), "clv_chunked_prefill")

"""ctypes binding of the C ABI in include/clover_attn.h.

This module is the only place that knows the struct layouts of the C ABI.
It loads ``cloverinfer_amd/_lib/libclover_attn.so`` (built by
``cloverinfer_amd.build``) and fails loudly when the library is missing or
was built for another ABI version: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import threading

from . import build as _build

ABI_VERSION = 1

CLV_F32, CLV_F16, CLV_BF16 = 0, 1, 2

CLV_OK = 0
CLV_EINVAL = 1
CLV_EUNSUPPORTED = 2
CLV_ELAUNCH = 3
CLV_EWORKSPACE = 4
CLV_ESCRATCH = 5

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p


class DecodeArgs(ctypes.Structure):
    """Mirror of ``clv_decode_args``."""

    _fields_ = [
        ("out", _c_ptr),
        ("q", _c_ptr),
        ("k_cache", _c_ptr),
        ("v_cache", _c_ptr),
        ("block_tables", _c_ptr),
        ("context_lens", _c_ptr),
        ("q_stride_seq", _c_i64),
        ("q_stride_head", _c_i64),
        ("out_stride_seq", _c_i64),
        ("out_stride_head", _c_i64),
        ("kv_stride_block", _c_i64),
        ("kv_stride_token", _c_i64),
        ("kv_stride_head", _c_i64),
        ("num_seqs", _c_i32),
        ("num_heads", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("block_size", _c_i32),
        ("max_blocks_per_seq", _c_i32),
        ("max_context_len", _c_i32),
        ("num_blocks", _c_i32),
        ("dtype", _c_i32),
        ("scale", ctypes.c_float),
    ]


class CacheArgs(ctypes.Structure):
    """Mirror of ``clv_cache_args``."""

    _fields_ = [
        ("key", _c_ptr),
        ("value", _c_ptr),
        ("k_cache", _c_ptr),
        ("v_cache", _c_ptr),
        ("slot_mapping", _c_ptr),
        ("key_stride_token", _c_i64),
        ("key_stride_head", _c_i64),
        ("value_stride_token", _c_i64),
        ("value_stride_head", _c_i64),
        ("kv_stride_block", _c_i64),
        ("kv_stride_token", _c_i64),
        ("kv_stride_head", _c_i64),
        ("num_tokens", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("block_size", _c_i32),
        ("num_blocks", _c_i32),
        ("dtype", _c_i32),
    ]


class PrefillArgs(ctypes.Structure):
    """Mirror of ``clv_prefill_args``."""

    _fields_ = [
        ("out", _c_ptr),
        ("q", _c_ptr),
        ("k_cache", _c_ptr),
        ("v_cache", _c_ptr),
        ("block_tables", _c_ptr),
        ("context_lens", _c_ptr),
        ("query_start_loc", _c_ptr),
        ("q_stride_token", _c_i64),
        ("q_stride_head", _c_i64),
        ("out_stride_token", _c_i64),
        ("out_stride_head", _c_i64),
        ("kv_stride_block", _c_i64),
        ("kv_stride_token", _c_i64),
        ("kv_stride_head", _c_i64),
        ("num_seqs", _c_i32),
        ("num_tokens", _c_i32),
        ("num_heads", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("block_size", _c_i32),
        ("max_blocks_per_seq", _c_i32),
        ("max_query_len", _c_i32),
        ("num_blocks", _c_i32),
        ("dtype", _c_i32),
        ("scale", ctypes.c_float),
    ]


# Exported symbols and their (restype, argtypes).
SIGNATURES = {
    "clv_abi_version": (ctypes.c_int, []),
    "clv_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "clv_reshape_and_cache": (ctypes.c_int, [ctypes.POINTER(CacheArgs), _c_ptr]),
    "clv_paged_decode": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), _c_ptr]),
    "clv_splitk_workspace_bytes": (ctypes.c_size_t, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "clv_paged_decode_splitk": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeArgs), _c_i32, _c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "clv_paged_decode_partials": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeArgs), _c_i32, _c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "clv_splitk_reduce": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeArgs), _c_i32, _c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "clv_paged_decode_balanced": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeArgs), _c_i32, _c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "clv_balanced_partials": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeArgs), _c_i32, _c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "clv_balanced_reduce": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeArgs), _c_i32, _c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "clv_paged_decode_balanced_noalloc": (
        ctypes.c_int, [ctypes.POINTER(DecodeArgs), _c_i32, _c_ptr],
    ),
    "clv_paged_decode_append": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeArgs), _c_ptr, _c_ptr, ctypes.c_int64, ctypes.c_int64, _c_i32,
         _c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "clv_balanced_reduce_append": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeArgs), _c_ptr, _c_ptr, ctypes.c_int64, ctypes.c_int64, _c_ptr,
         _c_i32, _c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "clv_reshape_and_cache_fp8": (
        ctypes.c_int, [ctypes.POINTER(CacheArgs), _c_ptr, _c_ptr, _c_ptr],
    ),
    "clv_paged_decode_fp8": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeArgs), _c_ptr, _c_ptr, _c_i32, _c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "clv_paged_decode_fp8_partials": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeArgs), _c_ptr, _c_ptr, _c_i32, _c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "clv_balanced_workspace_bytes": (ctypes.c_size_t, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "clv_default_num_waves": (_c_i32, []),
    "clv_default_num_waves_fp8": (_c_i32, []),
    "clv_chunked_prefill": (ctypes.c_int, [ctypes.POINTER(PrefillArgs), _c_ptr]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> str:
    """The in-tree library, or the file ``CLV_LIB_PATH`` names (the
    host-sanitized build, see cloverinfer_amd/build.py)."""
    return os.environ.get("CLV_LIB_PATH") or _build.LIB_PATH


def load() -> ctypes.CDLL:
    """Load the library once; raise RuntimeError if it is absent or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: build it with `python -m cloverinfer_amd.build` "
                "(there is no CPU fallback for the paged-attention kernels)"
            )
        # Import torch first so that its HIP runtime is the one the library binds.
        import torch  # noqa: F401

        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.clv_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path}: ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


_host = None
_host_tried = False


def load_host():
    """The node backend's native payload gather (cloverinfer_amd/_lib/_clv_host.so,
    built by cloverinfer_amd/build.py), or None when it is absent or does not
    load: it is host plumbing, and the backend then stages payloads with
    torch.stack."""
    global _host, _host_tried
    if _host_tried:
        return _host
    with _lock:
        if not _host_tried:
            import importlib.util

            import torch  # noqa: F401  (its libraries resolve the module's)

            path = _build.HOST_EXT_PATH
            if os.path.exists(path):
                try:
                    spec = importlib.util.spec_from_file_location(_build.HOST_EXT_NAME, path)
                    mod = importlib.util.module_from_spec(spec)
                    spec.loader.exec_module(mod)
                    _host = mod
                except ImportError:
                    _host = None
            _host_tried = True
    return _host


_host_ptr_fns = None


def mapped_device_address(host_ptr: int) -> int | None:
    """The device address of pinned host memory that kernels can access
    directly (hipHostGetDevicePointer), or None when the memory is not
    mapped for the device. Resolved through the library's own HIP runtime
    (dlsym on its handle searches its dependencies), the one torch uses. A
    refused query's error is cleared, so that the next launch's error check
    does not report it."""
    global _host_ptr_fns
    if _host_ptr_fns is None:
        lib = load()
        fn, last = lib.hipHostGetDevicePointer, lib.hipGetLastError
        fn.restype = last.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_uint]
        last.argtypes = []
        _host_ptr_fns = (fn, last)
    fn, last = _host_ptr_fns
    dev = ctypes.c_void_p()
    if fn(ctypes.byref(dev), ctypes.c_void_p(host_ptr), 0) != 0:
        last()
        return None
    return dev.value or None


def status_string(code: int) -> str:
    return load().clv_status_string(code).decode()


def check(code: int, what: str) -> None:
    """Map a C-ABI status to the Python exception classes."""
    if code == CLV_OK:
        return
    msg = f"{what}: {status_string(code)} (status {code})"
    if code in (CLV_EINVAL, CLV_EWORKSPACE, CLV_ESCRATCH):
        raise ValueError(msg)
    if code == CLV_EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)

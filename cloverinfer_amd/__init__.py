"""MI355X-native (gfx950) paged-attention hot path for CloverInfer.

* ``kernels``: tensor-level ops over the C ABI of ``libclover_attn.so``
  (paged decode with split-K, reshape_and_cache, chunked prefill);
* ``memory_manager.KVCacheManager``: the reference's paged KV manager API;
* ``attention_backend.GpuAttentionBackend``: the ``"gpu"`` AttentionNode backend.

Names are resolved lazily so that ``python -m cloverinfer_amd.build`` does not
import torch.
"""
import importlib

_EXPORTS = {
    "GpuAttentionBackend": "attention_backend",
    "create_attention_backend": "attention_backend",
    "KVCacheManager": "memory_manager",
    "chunked_prefill": "kernels",
    "paged_attention": "kernels",
    "reshape_and_cache": "kernels",
}

__all__ = sorted(_EXPORTS)


def __getattr__(name):
    mod = _EXPORTS.get(name)
    if mod is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    return getattr(importlib.import_module(f"{__name__}.{mod}"), name)

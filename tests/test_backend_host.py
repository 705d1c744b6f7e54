"""Host-side logic of the gpu backend that needs no device."""
import pytest
import torch

from cloverinfer_amd.attention_backend import _kv_dtype


def test_kv_dtype_names():
    """Pool dtype names: the reference's resident_kv_dtype strings ("fp32",
    "fp16"), bf16, fp8 (OCP e4m3), torch names and dtypes; anything else is
    refused."""
    assert _kv_dtype("fp32") is torch.float32 and _kv_dtype("fp16") is torch.float16
    assert _kv_dtype("bf16") is torch.bfloat16 and _kv_dtype("torch.float16") is torch.float16
    assert _kv_dtype(torch.bfloat16) is torch.bfloat16 and _kv_dtype(None) is None
    assert _kv_dtype("fp8") is torch.float8_e4m3fn
    for bad in ("int8", "fp4", torch.int32, torch.float8_e5m2):
        with pytest.raises(ValueError):
            _kv_dtype(bad)

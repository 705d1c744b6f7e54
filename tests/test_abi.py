"""The C-ABI library (CPU side): it loads, exports every entry point the
header declares, its ctypes mirrors have the C struct layouts, and argument
validation answers without touching a GPU."""
import ctypes
import os
import re
import subprocess

import pytest

from cloverinfer_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "clover_attn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(clv_[a-z_0-9]+)\s*\(", text)))


def test_header_functions_exported(native_lib):
    names = declared_functions()
    assert names, "no functions parsed from the header"
    assert set(names) == set(_native.SIGNATURES), "binding table and header disagree"
    out = subprocess.run(["nm", "-D", "--defined-only", _native.library_path()],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (clv_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, f"not exported: {missing}"


def test_abi_version_and_status_strings(native_lib):
    assert native_lib.clv_abi_version() == _native.ABI_VERSION
    for code in range(6):
        assert native_lib.clv_status_string(code)
    assert b"unknown" in native_lib.clv_status_string(99)


STRUCTS = {
    "clv_decode_args": _native.DecodeArgs,
    "clv_cache_args": _native.CacheArgs,
    "clv_prefill_args": _native.PrefillArgs,
}


def test_ctypes_layouts_match_c(tmp_path):
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "clover_attn.h"',
             "int main(void) {"]
    for cname, cls in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["return 0; }"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True,
                               check=True).stdout.splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, cls in STRUCTS.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert got[(cname, fname)] == getattr(cls, fname).offset, f"{cname}.{fname}"


def _valid_decode():
    a = _native.DecodeArgs()
    a.out = a.q = a.k_cache = a.v_cache = 0x1000
    a.block_tables = a.context_lens = 0x2000
    a.q_stride_seq, a.q_stride_head = 28 * 128, 128
    a.out_stride_seq, a.out_stride_head = 28 * 128, 128
    a.kv_stride_block, a.kv_stride_token, a.kv_stride_head = 16 * 4 * 128, 4 * 128, 128
    a.num_seqs, a.num_heads, a.num_kv_heads, a.head_dim = 0, 28, 4, 128
    a.block_size, a.max_blocks_per_seq, a.max_context_len, a.num_blocks = 16, 4, 64, 16
    a.dtype = _native.CLV_BF16
    a.scale = 0.088
    return a


@pytest.mark.parametrize("field,value,code", [
    ("dtype", 7, _native.CLV_EINVAL),
    ("num_heads", 30, _native.CLV_EINVAL),         # not a multiple of num_kv_heads
    ("head_dim", 96, _native.CLV_EUNSUPPORTED),
    ("block_size", 12, _native.CLV_EUNSUPPORTED),
    ("num_blocks", 0, _native.CLV_EINVAL),
    ("scale", float("nan"), _native.CLV_EINVAL),
])
def test_decode_validation_without_gpu(native_lib, field, value, code):
    a = _valid_decode()
    setattr(a, field, value)
    assert native_lib.clv_paged_decode(ctypes.byref(a), None) == code


def test_null_and_empty_calls(native_lib):
    assert native_lib.clv_paged_decode(None, None) == _native.CLV_EINVAL
    assert native_lib.clv_reshape_and_cache(None, None) == _native.CLV_EINVAL
    assert native_lib.clv_chunked_prefill(None, None) == _native.CLV_EINVAL
    a = _valid_decode()  # zero sequences: valid, nothing to launch
    assert native_lib.clv_paged_decode(ctypes.byref(a), None) == _native.CLV_OK
    a.num_seqs = 1
    a.q = 0x1008  # misaligned
    assert native_lib.clv_paged_decode(ctypes.byref(a), None) == _native.CLV_EINVAL


def test_splitk_workspace_size(native_lib):
    f = native_lib.clv_splitk_workspace_bytes
    # 16 seqs x 32 heads x 64 partitions of 512 over 32768 tokens, D = 128.
    rows = 16 * 32 * 64
    assert f(16, 32, 128, 32768, 512) == rows * 128 * 4 + 2 * rows * 4
    assert f(0, 32, 128, 32768, 512) == 0
    a = _valid_decode()
    a.num_seqs = 1
    assert native_lib.clv_paged_decode_splitk(ctypes.byref(a), 48, None, 0, None) == \
        _native.CLV_EINVAL  # partition not a multiple of 32
    assert native_lib.clv_paged_decode_splitk(ctypes.byref(a), 32, None, 0, None) == \
        _native.CLV_EWORKSPACE


def test_fp8_partials_need_an_explicit_wave_count(native_lib):
    """The partial layout depends on the wave count and the defaults of the
    partials call and of clv_balanced_reduce differ: num_waves <= 0 is
    refused before anything is launched."""
    a = _valid_decode()
    a.num_seqs = 1
    for waves in (0, -1):
        assert native_lib.clv_paged_decode_fp8_partials(
            ctypes.byref(a), 0x3000, 0x3000, waves, None, 0, None) == _native.CLV_EINVAL

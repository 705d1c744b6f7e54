"""Build recipe for the gfx950 shared library ``libclover_attn.so``.

The library is plain HIP + an ``extern "C"`` boundary (include/clover_attn.h);
it links only the HIP runtime, no torch. Objects go to ``_build/`` at the repo
root, the library to ``cloverinfer_amd/_lib/`` (both git-ignored; the library
travels with the source tree to the machine that runs it).

Run ``python -m cloverinfer_amd.build`` or call :func:`build`.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT_DIR = os.path.dirname(PKG_DIR)
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
INCLUDE_DIR = os.path.join(ROOT_DIR, "include")
BUILD_DIR = os.path.join(ROOT_DIR, "_build")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "libclover_attn.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

SOURCES = [
    "clover_attn_abi.hip",
    "cache_ops.hip",
    "decode.hip",
    "decode_stream.hip",
    "prefill.hip",
    "prefill_mfma.hip",
]

ARCH = "gfx950"


def _hipcc() -> str:
    env = os.environ.get("HIPCC")
    if env:
        return env
    found = shutil.which("hipcc")
    return found or "/opt/rocm/bin/hipcc"


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-mcode-object-version=5",
        # Packed fp32 VALU ops stay off: write plain fp32 and let scalar ops run.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA accumulators in VGPRs: the kernels fit in 256 VGPRs, and the
        # AGPR form made the register allocator copy accumulators between the
        # two files on every loop iteration.
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        "-I", INCLUDE_DIR,
        "-I", CSRC_DIR,
        "-Wall",
        "-Wno-unused-function",
    ]


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *compile_flags(), "-c", os.path.join(CSRC_DIR, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the gfx950-only feature flag; drop that note.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every source for gfx950 and link ``libclover_attn.so``; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1, 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)

"""Build recipe for the gfx950 shared library ``libclover_attn.so``.

The library is plain HIP + an ``extern "C"`` boundary (include/clover_attn.h);
it links only the HIP runtime, no torch. Objects go to ``_build/`` at the repo
root, the library to ``cloverinfer_amd/_lib/`` (both git-ignored; the library
travels with the source tree to the machine that runs it).

Run ``python -m cloverinfer_amd.build`` or call :func:`build`.

``python -m cloverinfer_amd.build --sanitize`` builds a second copy whose host
code (the C ABI's validation, sizing and launch set-up) is compiled with
AddressSanitizer and UndefinedBehaviorSanitizer, into ``_lib/sanitize/``
(objects in ``_build/sanitize/``); the device code is built as usual.
``CLV_LIB_PATH`` points the loader at it, and the process must preload the
sanitizer runtime (:func:`sanitizer_runtime`), e.g.::

    LD_PRELOAD=$(python -m cloverinfer_amd.build --print-asan-runtime) \
    ASAN_OPTIONS=detect_leaks=0 CLV_LIB_PATH=cloverinfer_amd/_lib/sanitize/libclover_attn.so \
    python -m pytest tests/test_abi.py tests/test_blocks.py
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

# The node backend's native payload gather (a Python extension on torch's C++
# API, host code only; cloverinfer_amd/host/node_gather.cpp).
HOST_EXT_NAME = "_clv_host"
HOST_EXT_SRC = os.path.join(PKG_DIR, "host", "node_gather.cpp")
HOST_EXT_PATH = os.path.join(LIB_DIR, HOST_EXT_NAME + ".so")

SANITIZE_LIB_PATH = os.path.join(LIB_DIR, "sanitize", LIB_NAME)
# Host-only sanitizer flags: each one behind -Xarch_host, so that the gfx950
# device code is compiled exactly as in the normal build.
SANITIZE_FLAGS = [f for flag in ("-fsanitize=address", "-fsanitize=undefined",
                                 "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer",
                                 "-g")
                  for f in ("-Xarch_host", flag)]


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


def _compile(src: str, verbose: bool, sanitize: bool = False) -> str:
    out_dir = os.path.join(BUILD_DIR, "sanitize") if sanitize else BUILD_DIR
    obj = os.path.join(out_dir, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *compile_flags(), *(SANITIZE_FLAGS if sanitize else []), "-c",
           os.path.join(CSRC_DIR, src), "-o", obj]
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


def build(verbose: bool = False, jobs: int | None = None, sanitize: bool = False) -> str:
    """Compile every source for gfx950 and link ``libclover_attn.so``; returns
    its path. ``sanitize``: the host-sanitized copy at SANITIZE_LIB_PATH."""
    lib_path = SANITIZE_LIB_PATH if sanitize else LIB_PATH
    os.makedirs(os.path.join(BUILD_DIR, "sanitize") if sanitize else BUILD_DIR, exist_ok=True)
    os.makedirs(os.path.dirname(lib_path), exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1, 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, sanitize), SOURCES))
    tmp = lib_path + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if sanitize:
        # The runtime itself comes from the preloaded shared library.
        cmd += ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                "-shared-libasan"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, lib_path)
    return lib_path


def build_host_ext(verbose: bool = False) -> str:
    """Compile the node backend's payload gather (g++, against the installed
    torch) into HOST_EXT_PATH; returns its path."""
    import sysconfig

    import torch
    import torch.utils.cpp_extension as ce

    os.makedirs(LIB_DIR, exist_ok=True)
    inc = [f for p in ce.include_paths() for f in ("-I", p)]
    inc += ["-I", sysconfig.get_paths()["include"]]
    lib = ce.library_paths()[0]
    tmp = HOST_EXT_PATH + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fopenmp", *inc,
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           f"-DTORCH_EXTENSION_NAME={HOST_EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           HOST_EXT_SRC, "-o", tmp, f"-L{lib}", "-lc10", "-ltorch", "-ltorch_cpu",
           "-ltorch_python", f"-Wl,-rpath,{lib}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for {HOST_EXT_SRC}:\n{res.stderr[-4000:]}")
    os.replace(tmp, HOST_EXT_PATH)
    return HOST_EXT_PATH


def sanitizer_runtime() -> str:
    """Path of the AddressSanitizer runtime (which carries the
    UndefinedBehaviorSanitizer checks too) that a process loading the
    sanitized library must preload."""
    res = subprocess.run([_hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"],
                         capture_output=True, text=True)
    path = res.stdout.strip()
    if res.returncode != 0 or not os.path.isabs(path) or not os.path.exists(path):
        llvm = os.path.join(os.path.dirname(os.path.realpath(_hipcc())), "..", "llvm")
        raise RuntimeError(f"AddressSanitizer runtime not found (hipcc said {path!r}; "
                           f"looked under {llvm})")
    return path


if __name__ == "__main__":
    if "--print-asan-runtime" in sys.argv:
        print(sanitizer_runtime())
    else:
        sanitize = "--sanitize" in sys.argv
        path = build(verbose="-v" in sys.argv, sanitize=sanitize)
        print(path)
        if not sanitize:
            print(build_host_ext(verbose="-v" in sys.argv))

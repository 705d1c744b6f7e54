"""The C ABI's host code under AddressSanitizer + UndefinedBehaviorSanitizer.

Builds the host-sanitized copy of libclover_attn.so (device code unchanged;
cloverinfer_amd/build.py --sanitize) and runs the CPU tests that drive the
library's host side (argument validation, workspace sizing, status strings,
exported symbols and struct layouts, and the block bookkeeping around it) in
a child process with the sanitizer runtime preloaded. Any report aborts the
child, which fails this test."""
import os
import subprocess
import sys

from cloverinfer_amd import build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_host_side_under_address_and_ub_sanitizers():
    path = build.build(sanitize=True)
    syms = subprocess.run(["nm", "-D", path], capture_output=True, text=True, check=True).stdout
    assert "__asan_report" in syms and "__ubsan_handle" in syms, "library is not instrumented"
    env = dict(os.environ,
               LD_PRELOAD=build.sanitizer_runtime(),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               CLV_LIB_PATH=path)
    code = ("import sys, pytest; from cloverinfer_amd import _native; "
            f"assert _native.library_path() == {path!r}; "
            "sys.exit(pytest.main(['-q', '-x', '-p', 'no:cacheprovider', '-m', 'not gpu', "
            "'tests/test_abi.py', 'tests/test_blocks.py']))")
    proc = subprocess.run([sys.executable, "-c", code], env=env, cwd=ROOT, capture_output=True,
                          text=True, timeout=600)
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0, out[-4000:]
    assert "passed" in proc.stdout and "ERROR: AddressSanitizer" not in out \
        and "runtime error:" not in out, out[-4000:]

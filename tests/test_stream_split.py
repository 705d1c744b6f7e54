"""The balanced decode's step split (StreamSplit in csrc/decode_stream.hip)
checked on the CPU: tests/host/stream_split_check.hip includes the kernel
source, is built with hipcc for the host side and run there (no GPU call).
Every group must own a non-empty, consecutive span and owner() must invert
start(), for any dispatch-slot count and weights; the merge finds each
segment's partials through owner()."""
import os
import shutil
import subprocess
import tempfile

import pytest

from cloverinfer_amd import build as B

HERE = os.path.dirname(os.path.abspath(__file__))


def test_stream_split_invariants():
    hipcc = B._hipcc()
    if not os.path.exists(hipcc) and not shutil.which(hipcc):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as tmp:
        exe = os.path.join(tmp, "stream_split_check")
        flags = [f for f in B.compile_flags() if f not in ("-fPIC",)]
        res = subprocess.run([hipcc, *flags, os.path.join(HERE, "host", "stream_split_check.hip"),
                              "-o", exe], capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-3000:]
        run = subprocess.run([exe], capture_output=True, text=True, timeout=600)
        assert run.returncode == 0, run.stdout + run.stderr
        assert "bad 0" in run.stdout

"""Work splits of the kernels checked on the CPU: each program under
tests/host/ includes a kernel source, is built with hipcc and runs on the
host (no GPU call).

* stream_split_check.hip: the balanced decode's step split (StreamSplit in
  csrc/decode_stream.hip). Every group must own a non-empty, consecutive
  span and owner() must invert start(), for any dispatch-slot count and
  weights; the merge finds each segment's partials through owner().
* prefill_order_check.hip: the chunked prefill's dispatch order
  (dispatch_slot in csrc/prefill_mfma.hip) is a permutation that keeps every
  work item in its round and dispatches later rounds heaviest tile first."""
import os
import shutil
import subprocess
import tempfile

import pytest

from cloverinfer_amd import build as B

HERE = os.path.dirname(os.path.abspath(__file__))


def _run_host_check(name):
    hipcc = B._hipcc()
    if not os.path.exists(hipcc) and not shutil.which(hipcc):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as tmp:
        exe = os.path.join(tmp, name)
        flags = [f for f in B.compile_flags() if f not in ("-fPIC",)]
        res = subprocess.run([hipcc, *flags, os.path.join(HERE, "host", name + ".hip"),
                              "-o", exe], capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-3000:]
        run = subprocess.run([exe], capture_output=True, text=True, timeout=600)
        assert run.returncode == 0, run.stdout + run.stderr
        assert "bad 0" in run.stdout


def test_stream_split_invariants():
    _run_host_check("stream_split_check")


def test_prefill_dispatch_order():
    _run_host_check("prefill_order_check")

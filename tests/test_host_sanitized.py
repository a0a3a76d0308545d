"""Host-side code of libgdn under AddressSanitizer and UBSan, on the CPU.

Builds the library's host sources (pool and slot allocator, KV page planner,
executor admission/batching/rollback) host-only with ``-fsanitize=address``
and ``-fsanitize=undefined``, with the debug slot-list check compiled in
(``GDN_DEBUG_SLOTS``), links them against a runtime stand-in that backs device
memory with host memory and runs no kernels (``tests/host/fake_hip.cpp``), and
runs the driver ``tests/host/host_test.cpp``. Any sanitizer report (heap
overflow, use after free, leak, undefined behaviour) aborts the run.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
HOST = os.path.join(HERE, "host")


@pytest.mark.skipif(shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="needs make and hipcc")
def test_host_code_clean_under_asan_ubsan():
    r = subprocess.run(["make", "-C", HOST, "-j8", "run"], capture_output=True, text=True,
                       timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-6000:]
    assert "ALL OK" in out, out[-3000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-6000:]

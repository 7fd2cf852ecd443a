"""Runs the C++ GPU tests of the drop-in API (HIP TransferBackend, shared-arena
connector) built by build()."""
import subprocess
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parent.parent / "paged-batch-engine_amd" / "lib"
pytestmark = pytest.mark.gpu


def test_cpp_gpu_suite():
    exe = LIB / "pbe_cpp_gpu_tests"
    assert exe.exists(), "run __graft_entry__.build() first"
    print("[case] pbe_cpp_gpu_tests", flush=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=110)
    print(proc.stdout[-4000:])
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]
    assert "0 failed" in proc.stdout

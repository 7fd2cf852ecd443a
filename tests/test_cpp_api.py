"""Runs the C++ unit tests of the drop-in API (built by build())."""
import subprocess
from pathlib import Path

LIB = Path(__file__).resolve().parent.parent / "paged-batch-engine_amd" / "lib"


def test_cpp_drop_in_api_suite():
    exe = LIB / "pbe_cpp_tests"
    assert exe.exists(), "run __graft_entry__.build() first"
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]
    assert "0 failed" in proc.stdout

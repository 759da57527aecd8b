"""Runs the C++ host test program (transformer-cuda_amd/bin/test_attention), which drives
the reference-named launchers of include/kernels/attention.h through the C ABI."""
import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "transformer-cuda_amd", "bin", "test_attention")


@pytest.mark.gpu
def test_cpp_host_suite():
    assert os.path.exists(BIN), "build first: __graft_entry__.build()"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout[-2000:]
    assert "All host tests passed." in r.stdout

"""bench.py's host side on the CPU: the multi-GPU refusal, and the profile lookups that the
roofline object's `traffic` comes from (profiles/hbm_traffic.md rows for the kernels the
bench lines name as dominant)."""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)

import bench  # noqa: E402  (imports no GPU state at module level)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert r.stdout == ""  # no JSON line
    assert "one GPU" in r.stderr


@pytest.mark.parametrize("config,dtype,kernel", [
    ("c2", "f32", "bwd_dkdv_ds_x3"),       # the headline's dominant kernel
    ("c2", "f32", "bwd_dkdv_ds_packed"),   # --path packed
    ("c3", "bf16", "bwd_dkdv_packed"),
    ("c4", "bf16", "bwd_dkdv_packed"),
    ("c2", "f32", "materialized_gemm_qk"),  # the materialised line
])
def test_traffic_rows_for_the_dominant_kernels(config, dtype, kernel):
    t = bench.measured_traffic(config, dtype, kernel)
    assert isinstance(t, int) and t > 0
    # FETCH_SIZE * 2 + WRITE_SIZE KiB: the copy calibration the file states (factors 2 and
    # 1 to within 0.01%; the KiB cells are rounded for display)
    path = os.path.join(REPO, "profiles", "hbm_traffic.md")
    row = next(ln for ln in open(path) if ln.startswith(f"| {config} | {dtype} |")
               and f"| {kernel} |" in ln)
    cells = [c.strip() for c in row.strip().strip("|").split("|")]
    fetch, write = float(cells[4]), float(cells[5])
    assert abs(t - (2 * fetch + write) * 1024) <= 1e-3 * t
    # and within a few times the kernel's algorithmic bytes (the column beside it)
    alg = int(cells[7])
    assert 0.9 * alg <= t <= 5 * alg


def test_traffic_lookup_misses_are_none():
    assert bench.measured_traffic("c2", "f32", "no_such_kernel") is None
    assert bench.measured_traffic("c9", "f32", "bwd_dkdv_ds_x3") is None

"""The kernels' workgroup -> (head, block) orders and the host's head-group rule, checked on
the CPU by transformer-cuda_amd/bin/sched_check (built from src/sched_check.cpp with the
kernels' own headers): every order is a bijection onto the (head, block) pairs, keeps a
head's blocks on one XCD when the head count allows, takes blocks heaviest first, and
head_group picks the groups measured at the bench shapes."""
import os
import subprocess

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "transformer-cuda_amd")
BIN = os.path.join(PKG, "bin", "sched_check")


def test_block_orders_and_head_groups():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-C", PKG, "bin/sched_check"], check=True,
                       capture_output=True, timeout=300)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-2000:]
    assert "sched_check: all passed" in r.stdout

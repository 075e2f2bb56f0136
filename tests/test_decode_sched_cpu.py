"""The decode kernels' work schedule (powerinfer_x64_amd/csrc/decode_sched.hpp)
walked on the host for well-formed and malformed tables: every page-table read,
pool block and partial slot stays in bounds, and every item, page and merged run
is covered exactly once (tests/cpp/test_decode_sched.cpp).  No GPU is used; the
malformed tables are never sent to one."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "_build", "test_decode_sched")


def test_decode_schedule_bounds_host_walk():
    assert os.path.exists(EXE), "tests/cpp not built (python -m powerinfer_x64_amd.build)"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("0 failures"), r.stdout

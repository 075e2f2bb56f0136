"""The reference's own op tests (src/ops.rs:299-395, tests/smoke.rs:44-61,
src/ssm/mod.rs:164-166, src/bin/layer_trace.rs:180-196), compiled in C++
against the C++ mirror include/pi_ops.hpp, run on the GPU."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP_TEST = os.path.join(ROOT, "tests", "cpp", "_build", "test_ops")


def test_reference_op_tests_on_gpu():
    assert os.path.exists(CPP_TEST), "tests/cpp not built (python -m powerinfer_x64_amd.build)"
    r = subprocess.run([CPP_TEST], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout
    assert r.stdout.count("PASS") == 9


def test_device_layer_cache_cpp():
    """DeviceLayerCache and DeviceGdnLayer (the forward seam in C++): prompt == token loop,
    errors, reset."""
    exe = os.path.join(ROOT, "tests", "cpp", "_build", "test_layer")
    assert os.path.exists(exe), "tests/cpp not built (python -m powerinfer_x64_amd.build)"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("PASS") == 3

"""The C ABI library (no GPU needed): it loads, exports exactly what
include/pi_attn.h declares, and reports errors through status + text."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pi_attn.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pi_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_match_bindings():
    from powerinfer_x64_amd import _abi
    assert _declared() == sorted(_abi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    from powerinfer_x64_amd import _abi
    lib = _abi.load()
    for name in _declared():
        assert hasattr(lib, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True,
                        text=True, check=True).stdout
    exported = set(re.findall(r"\bT (pi_[a-z0-9_]+)$", nm, flags=re.M))
    assert set(_declared()) <= exported


def test_library_is_gfx950_only():
    """The embedded offload bundles name gfx950 and no other GPU target."""
    from powerinfer_x64_amd import _abi
    blob = open(_abi.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", blob))
    assert targets == {b"gfx950"}


def test_abi_version_and_null_handle_errors():
    from powerinfer_x64_amd import _abi
    lib = _abi.load()
    assert lib.pi_abi_version() == 1
    assert lib.pi_sync(None, None) == 1  # PI_ERR_INVALID_ARG
    assert b"null pi_handle" in lib.pi_last_error(None)
    assert lib.pi_attn_decode(None, None, None, None, 1, None, 1, 1, 0, 1.0, None, None,
                              None) == 1
    lib.pi_destroy(None)            # no-ops on null
    lib.pi_kv_pool_destroy(None)
    assert lib.pi_kv_pool_bytes(None) == 0


def test_create_without_device_reports_device_error():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from powerinfer_x64_amd import _abi, runtime
    lib = _abi.load()
    h = ctypes.c_void_p()
    rc = lib.pi_create(0, ctypes.byref(h))
    assert rc == 4 and not h.value  # PI_ERR_DEVICE (BackendError::CudaError analogue)
    assert b"pi_create" in lib.pi_last_error(None)
    with pytest.raises(runtime.DeviceError):
        runtime.Device(0)


CPP_TEST = os.path.join(ROOT, "tests", "cpp", "_build", "test_ops")


def test_cpp_mirror_reports_missing_device():
    """The C++ mirror (include/pi_ops.hpp) returns None from Device::init and the
    test binary exits 2 naming the device error when no GPU is visible."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    assert os.path.exists(CPP_TEST), "tests/cpp not built (python -m powerinfer_x64_amd.build)"
    r = subprocess.run([CPP_TEST], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2, r.stdout + r.stderr
    assert r.stdout.startswith("NO_DEVICE pi_create")


def test_compute_imrope_freqs_host_export_matches_oracle(orc):
    """pi_compute_imrope_freqs is host code in the product; it must equal the
    oracle's restatement of src/ops.rs:78-122 bit for bit."""
    import numpy as np
    from powerinfer_x64_amd import _abi
    lib = _abi.load()
    for base, n_rot, sec in ((1e7, 64, (11, 11, 10, 0)), (1e6, 128, (24, 20, 20, 0)),
                             (1e4, 2, (1, 0, 0, 0))):
        out = np.zeros(n_rot // 2, np.float32)
        s = (ctypes.c_int32 * 4)(*sec)
        assert lib.pi_compute_imrope_freqs(base, n_rot, s, out.ctypes.data_as(ctypes.c_void_p)) == 0
        ref = orc.compute_imrope_freqs(base, n_rot, list(sec))
        assert np.array_equal(out, ref)
    assert lib.pi_compute_imrope_freqs(1e4, 512, s, out.ctypes.data_as(ctypes.c_void_p)) == 5

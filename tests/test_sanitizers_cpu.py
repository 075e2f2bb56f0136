"""AddressSanitizer + UndefinedBehaviorSanitizer builds of the host code, run on the CPU:

- the oracle (oracle/oracle.c) under tests/cpp/san_oracle.cpp, every entry point on small
  and edge shapes with exactly sized buffers;
- the decode schedule's host walk (tests/cpp/test_decode_sched.cpp), which checks the
  indices the decode kernels form, over malformed tables;
- the C ABI's host side (powerinfer_x64_amd/csrc/api.cpp compiled with host sanitizers and
  linked with the library's device objects) under tests/cpp/san_abi_host.cpp: the host-only
  entry points and the argument checks, without a GPU.

Any report fails the test (-fno-sanitize-recover).  Skipped where the compilers or the
library objects are absent.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
OUT = os.path.join(CPP, "_build", "san")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
           UBSAN_OPTIONS="print_stacktrace=1")


def _run(cmd, timeout=300, env=None):
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout, env=env)
    return r.returncode, r.stdout + r.stderr


def _need(tool):
    if shutil.which(tool) is None and not os.path.exists(tool):
        pytest.skip(f"{tool} not found")


def test_oracle_under_asan_ubsan():
    _need("gcc")
    os.makedirs(OUT, exist_ok=True)
    obj = os.path.join(OUT, "oracle_san.o")
    exe = os.path.join(OUT, "san_oracle")
    rc, log = _run(["gcc", "-O1", "-g", "-msse4.1", "-ffp-contract=off", *SAN, "-c",
                    os.path.join(ROOT, "oracle", "oracle.c"), "-o", obj])
    assert rc == 0, log
    rc, log = _run(["g++", "-O1", "-g", "-std=c++17", *SAN, "-I", os.path.join(ROOT, "oracle"),
                    os.path.join(CPP, "san_oracle.cpp"), obj, "-o", exe, "-lm"])
    assert rc == 0, log
    rc, log = _run([exe], env=ENV)
    assert rc == 0 and "san_oracle: ok" in log, log


def test_decode_schedule_walk_under_asan_ubsan():
    _need("g++")
    os.makedirs(OUT, exist_ok=True)
    exe = os.path.join(OUT, "test_decode_sched")
    rc, log = _run(["g++", "-O1", "-g", "-std=c++17", *SAN,
                    "-I", os.path.join(ROOT, "powerinfer_x64_amd", "csrc"),
                    os.path.join(CPP, "test_decode_sched.cpp"), "-o", exe])
    assert rc == 0, log
    rc, log = _run([exe], timeout=600, env=ENV)
    assert rc == 0 and " 0 failures" in log, log[-3000:]


def test_c_abi_host_code_under_asan_ubsan():
    _need(HIPCC)
    build = os.path.join(ROOT, "powerinfer_x64_amd", "_build")
    objs = [os.path.join(build, f) for f in sorted(os.listdir(build)) if f.endswith(".hip.o")] \
        if os.path.isdir(build) else []
    if not objs:
        pytest.skip("library objects not built (python -m powerinfer_x64_amd.build)")
    os.makedirs(OUT, exist_ok=True)
    host_san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                "-Xarch_host", "-fno-sanitize-recover=all"]
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "powerinfer_x64_amd", "csrc")]
    api_o = os.path.join(OUT, "api_san.o")
    drv_o = os.path.join(OUT, "san_abi_host.o")
    exe = os.path.join(OUT, "san_abi_host")
    rc, log = _run([HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC",
                    "-ffp-contract=off", *host_san, *inc, "-c",
                    os.path.join(ROOT, "powerinfer_x64_amd", "csrc", "api.cpp"), "-o", api_o])
    assert rc == 0, log
    rc, log = _run([HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", *host_san, *inc,
                    "-c", os.path.join(CPP, "san_abi_host.cpp"), "-o", drv_o])
    assert rc == 0, log
    rc, log = _run([HIPCC, "--offload-arch=gfx950", *host_san, "-o", exe, drv_o, api_o, *objs])
    assert rc == 0, log
    rc, log = _run([exe], env=ENV)
    assert rc == 0 and "san_abi_host: 0 failed" in log, log[-3000:]

"""Builds libpi_attn.so (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: python -m powerinfer_x64_amd.build   (or __graft_entry__.build()).
Every source is compiled for gfx950 only, with packed-FP32 instruction
generation disabled, then linked into powerinfer_x64_amd/libpi_attn.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libpi_attn.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]


# Per-file additions: the TurboQuant quantizer (device) and its matrix
# generation (host) reproduce the reference's separately rounded multiply and
# add, so nothing in them may fuse into an FMA.
FILE_FLAGS = {"turboquant.hip": ["-ffp-contract=off"], "api.cpp": ["-ffp-contract=off"]}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith(".hip") or f.endswith(".cpp"))


def _compile(src: str) -> str:
    obj = os.path.join(OUT_DIR, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *CFLAGS, *FILE_FLAGS.get(os.path.basename(src), []), *lang, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_cpp_tests(verbose)
    return LIB


CPP_TESTS = os.path.join(HERE, "..", "tests", "cpp")


def build_cpp_tests(verbose: bool = False) -> None:
    """The C++ tests of the C ABI / C++ mirror (host code only, linked against
    the in-tree library through an rpath).  The san_*.cpp drivers are built by
    their own test with sanitizers and are skipped here."""
    out_dir = os.path.join(CPP_TESTS, "_build")
    os.makedirs(out_dir, exist_ok=True)
    for src in sorted(f for f in os.listdir(CPP_TESTS) if f.endswith(".cpp") and not f.startswith("san_")):
        exe = os.path.join(out_dir, src[:-4])
        cmd = ["g++", "-std=c++20", "-O2", "-Wall", "-Wextra", "-I", os.path.join(HERE, "..", "include"),
               "-I", CSRC, os.path.join(CPP_TESTS, src), "-L", HERE, "-lpi_attn",
               "-Wl,-rpath,$ORIGIN/../../../powerinfer_x64_amd", "-o", exe + ".tmp"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"g++ failed on {src}:\n{r.stderr}")
        os.replace(exe + ".tmp", exe)
        if verbose:
            print(f"built {exe}")


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

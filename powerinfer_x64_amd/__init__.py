"""MI355X (gfx950) attention + gated-DeltaNet hot path of PowerInfer_x64.

The product is libpi_attn.so (HIP kernels + the C ABI in include/pi_attn.h).
This package builds it (``build``), binds it (``_abi``) and offers a thin
torch-tensor front end (``runtime``) used by the tests and bench.py.
"""
from . import _abi  # noqa: F401

__all__ = ["_abi", "runtime"]

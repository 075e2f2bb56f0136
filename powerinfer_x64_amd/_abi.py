"""ctypes declarations of every entry point in include/pi_attn.h.

The shared library is loaded from this package directory (built in-tree by
powerinfer_x64_amd.build).  There is no fallback: if the library is missing
or lacks a symbol, loading raises.
"""
from __future__ import annotations

import ctypes
import os

# PI_ATTN_LIB names another build of the same library (an A/B comparison of
# two builds); by default the in-tree build is loaded.
LIB_PATH = os.environ.get("PI_ATTN_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "libpi_attn.so")

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_int = ctypes.c_int

# name -> (restype, argtypes); mirrors include/pi_attn.h one to one.
SIGNATURES = {
    "pi_abi_version": (_int, []),
    "pi_create": (_int, [_int, ctypes.POINTER(_vp)]),
    "pi_destroy": (None, [_vp]),
    "pi_last_error": (ctypes.c_char_p, [_vp]),
    "pi_sync": (_int, [_vp, _vp]),
    "pi_kv_pool_create": (_int, [_vp, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_vp)]),
    "pi_kv_pool_destroy": (None, [_vp]),
    "pi_kv_pool_bytes": (_sz, [_vp]),
    "pi_kv_append": (_int, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i32, _vp]),
    "pi_kv_read": (_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "pi_head_rmsnorm": (_int, [_vp, _vp, _vp, _i32, _i32, _i32, _f32, _vp]),
    "pi_rope": (_int, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _vp]),
    "pi_attn_prologue": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _f32, _i32, _f32, _vp, _vp, _vp,
                                _i32, _vp, _i32, _i32, _i32, _vp]),
    "pi_attn_decode": (_int, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _f32, _vp, _vp,
                              _vp]),
    "pi_attn_decode_noalloc": (_int, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _f32, _vp,
                                      _vp, _vp]),
    "pi_attn_prefill": (_int, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                               _i32, _f32, _vp, _vp]),
    "pi_attn_prefill_paged": (_int, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _f32, _vp,
                                     _vp]),
    "pi_gdn_gates": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "pi_gdn_conv1d": (_int, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "pi_gdn_rmsnorm_gated": (_int, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _f32, _vp]),
    "pi_gdn_decode": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                             _i32, _vp]),
    "pi_gdn_prefill": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                              _i32, _i32, _vp]),
    "pi_ops_attention_head": (_int, [_vp, _vp, _vp, _vp, _vp, _sz, _sz]),
    "pi_ops_rms_norm": (_int, [_vp, _vp, _vp, _vp, _sz, _f32]),
    "pi_ops_softmax": (_int, [_vp, _vp, _sz]),
    "pi_ops_apply_rope": (_int, [_vp, _vp, _vp, _sz, _sz, _sz, _f32]),
    "pi_ops_apply_rope_with_freqs": (_int, [_vp, _vp, _vp, _sz, _sz, _vp, _sz]),
    "pi_compute_imrope_freqs": (_int, [_f32, _sz, _vp, _vp]),
    "pi_ssm_gated_delta_step": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32,
                                       _i32]),
    "pi_ssm_forward": (_int, [_vp, _vp, _vp, _vp, _sz, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _vp,
                              _sz, _sz, _sz]),
    "pi_attn_layer_create": (_int, [_vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _f32, _i32,
                                    _f32, _vp, _i32, ctypes.POINTER(_vp)]),
    "pi_attn_layer_create_dims": (_int, [_vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _vp,
                                         _f32, _i32, _f32, _vp, _i32, ctypes.POINTER(_vp)]),
    "pi_attn_layer_destroy": (None, [_vp]),
    "pi_attn_layer_forward": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp]),
    "pi_attn_layer_forward_dev": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp]),
    "pi_attn_layer_reset": (None, [_vp]),
    "pi_attn_layer_seq_len": (_i32, [_vp]),
    "pi_gdn_layer_create": (_int, [_vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _f32,
                                   ctypes.POINTER(_vp)]),
    "pi_gdn_layer_destroy": (None, [_vp]),
    "pi_gdn_layer_forward": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp]),
    "pi_gdn_layer_forward_dev": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp]),
    "pi_gdn_layer_reset": (_int, [_vp, _vp]),
    "pi_tq_generate": (_int, [_i32, ctypes.c_uint64, _vp, _vp]),
    "pi_tq_pool_create": (_int, [_vp, _i32, _i32, _i32, _i32, ctypes.POINTER(_vp)]),
    "pi_tq_pool_destroy": (None, [_vp]),
    "pi_tq_pool_bytes": (_sz, [_vp]),
    "pi_tq_append": (_int, [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _vp]),
    "pi_tq_read": (_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "pi_tq_attn_decode": (_int, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _vp]),
}

_lib = None


def load():
    """Load libpi_attn.so and bind every symbol; raises if anything is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run `python -m powerinfer_x64_amd.build`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the export is missing
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib

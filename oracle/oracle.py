"""ctypes front end of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg import this module as the parity checker and CPU
baseline.  The product package never imports it.

Each wrapper takes numpy arrays, checks shapes and dtypes, and calls the C
restatement of the reference function named in oracle.h.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_sz = ctypes.c_size_t
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u64p = ctypes.POINTER(ctypes.c_uint64)


def build() -> str:
    """Compile oracle.c with oracle/Makefile; returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "or_dot_product": (ctypes.c_float, [_f32p, _f32p, _sz]),
            "or_sum_squares": (ctypes.c_float, [_f32p, _sz]),
            "or_scale": (None, [_f32p, _f32p, ctypes.c_float, _sz]),
            "or_rms_norm": (None, [_f32p, _f32p, _f32p, _sz, ctypes.c_float]),
            "or_apply_rope": (None, [_f32p, _f32p, _sz, _sz, _sz, ctypes.c_float]),
            "or_compute_imrope_freqs": (None, [ctypes.c_float, _sz, _i32p, _f32p]),
            "or_apply_rope_with_freqs": (None, [_f32p, _f32p, _sz, _sz, _f32p, _sz]),
            "or_softmax": (None, [_f32p, _sz]),
            "or_attention_head": (None, [_f32p, _f32p, _f32p, _f32p, _sz, _sz]),
            "or_attn_decode": (None, [_f32p, _f32p, _sz, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz]),
            "or_apply_gate": (None, [_f32p, _f32p, _sz]),
            "or_attn_layer_tokens": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz,
                                            _sz, _sz, _f32p, _f32p, ctypes.c_float, _sz,
                                            ctypes.c_float, _f32p, _sz, _f32p, _f32p, _sz]),
            "or_attn_prepare": (None, [_f32p, _f32p, _sz, _sz, _sz, _sz, _sz, _f32p, _f32p,
                                       ctypes.c_float, _sz, ctypes.c_float, _f32p, _sz, _sz]),
            "or_gdn_gates": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _sz]),
            "or_gdn_step": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz,
                                   _sz, _sz]),
            "or_gdn_tokens": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz,
                                     _sz, _sz, _sz]),
            "or_rmsnorm_gated": (None, [_f32p, _f32p, _f32p, _sz, _sz, ctypes.c_float]),
            "or_conv1d_silu": (None, [_f32p, _f32p, _f32p, _sz, _sz]),
            "or_ssm_forward": (None, [_f32p, _f32p, _f32p, _sz, _f32p, _f32p, _f32p, _f32p, _sz,
                                      _f32p, _sz, _f32p, _sz, _sz, _sz]),
            "or_splitmix64_next": (ctypes.c_uint64, [_u64p]),
            "or_splitmix64_gaussian": (ctypes.c_float, [_u64p]),
            "or_tq_orthogonal": (None, [_f32p, _sz, ctypes.c_uint64]),
            "or_tq_gaussian_matrix": (None, [_f32p, _sz, _sz, ctypes.c_uint64]),
            "or_tq_compressed_bytes": (_sz, [_sz, _sz, _sz]),
            "or_tq_centroid": (ctypes.c_float, [_sz, _sz]),
            "or_tq_pack": (None, [_u8p, _u8p, _sz, _sz, _u8p, _sz]),
            "or_tq_unpack": (None, [_u8p, _u8p, _u8p, _sz, _sz, _sz]),
            "or_tq_quantize": (None, [_u8p, _f32p, _f32p, _f32p, _sz, _sz, _sz]),
            "or_tq_dequantize": (None, [_f32p, _u8p, _f32p, _sz, _sz]),
            "or_tq_dot": (ctypes.c_float, [_f32p, _u8p, _f32p, _f32p, _sz, _sz, _sz]),
            "or_tq_precompute_query": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz]),
            "or_tq_dot_precomputed": (ctypes.c_float, [_f32p, _f32p, _u8p, _sz, _sz, _sz]),
            "or_tq_cache_append_keys": (None, [_u8p, _f32p, _f32p, _f32p, _f32p, _sz, _sz]),
            "or_tq_cache_attend": (None, [_f32p, _f32p, _u8p, _f32p, _u16p, _f32p, _f32p, _sz,
                                          _sz, _sz, _sz]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(a, writable=False):
    """Return a C-contiguous float32 view (copy if needed) and its pointer."""
    arr = np.ascontiguousarray(a, dtype=np.float32)
    if writable and arr is not a:
        arr = arr.copy()
    return arr


def _p(arr):
    if arr is None:
        return None
    assert arr.dtype == np.float32 and arr.flags.c_contiguous
    return arr.ctypes.data_as(_f32p)


# ---- src/simd.rs -----------------------------------------------------------

def dot_product(a, b) -> float:
    a, b = _f32(a), _f32(b)
    assert a.shape == b.shape
    return float(lib().or_dot_product(_p(a), _p(b), a.size))


def sum_squares(a) -> float:
    a = _f32(a)
    return float(lib().or_sum_squares(_p(a), a.size))


def scale(a, s: float):
    a = _f32(a)
    out = np.empty_like(a)
    lib().or_scale(_p(out), _p(a), float(s), a.size)
    return out


# ---- src/ops.rs ------------------------------------------------------------

def rms_norm(x, w, eps: float):
    x, w = _f32(x), _f32(w)
    assert x.shape == w.shape
    out = np.empty_like(x)
    lib().or_rms_norm(_p(out), _p(x), _p(w), x.size, float(eps))
    return out


def apply_rope(q, k, position: int, head_dim: int, rope_dim: int, base: float):
    """Returns rotated copies of q and k (the reference rotates in place)."""
    q = np.array(q, dtype=np.float32, copy=True)
    k = np.array(k, dtype=np.float32, copy=True)
    lib().or_apply_rope(_p(q), _p(k), position, head_dim, rope_dim, float(base))
    return q, k


def compute_imrope_freqs(base: float, n_rot: int, sections):
    sec = (ctypes.c_int32 * 4)(*[int(s) for s in sections])
    out = np.empty(n_rot // 2, dtype=np.float32)
    lib().or_compute_imrope_freqs(float(base), n_rot, sec, _p(out))
    return out


def apply_rope_with_freqs(q, k, position: int, head_dim: int, freqs):
    q = np.array(q, dtype=np.float32, copy=True)
    k = np.array(k, dtype=np.float32, copy=True)
    f = _f32(freqs)
    lib().or_apply_rope_with_freqs(_p(q), _p(k), position, head_dim, _p(f), f.size)
    return q, k


def softmax(x):
    x = np.array(x, dtype=np.float32, copy=True)
    lib().or_softmax(_p(x), x.size)
    return x


def attention_head(q, k_cache, v_cache, seq_len: int, head_dim: int):
    q, k, v = _f32(q), _f32(k_cache), _f32(v_cache)
    out = np.zeros(head_dim, dtype=np.float32)
    lib().or_attention_head(_p(out), _p(q), _p(k), _p(v), seq_len, head_dim)
    return out


# ---- src/model/mod.rs attention block -------------------------------------

def attn_decode(q, key_cache, value_cache):
    """q [Hq, D]; caches [T, Hkv, D] (already rotated); returns out [Hq, D]."""
    q, kc, vc = _f32(q), _f32(key_cache), _f32(value_cache)
    hq, dq = q.shape
    t, hkv, dk = kc.shape
    dv = vc.shape[2]
    assert vc.shape[:2] == (t, hkv)
    out = np.zeros((hq, dk), dtype=np.float32)
    lib().or_attn_decode(_p(out), _p(q), dq, _p(kc), _p(vc), t, hq, hkv, dk, dv)
    return out


def apply_gate(out, gate):
    out = np.array(out, dtype=np.float32, copy=True)
    g = _f32(gate)
    assert g.size >= out.size
    lib().or_apply_gate(_p(out), _p(g), out.size)
    return out


def attn_layer_tokens(q, k, v, gate=None, q_norm_w=None, k_norm_w=None, eps=1e-6,
                      rope_dim=None, rope_base=10000.0, freqs=None,
                      key_cache=None, value_cache=None, prev_seq_len=0):
    """Per-token attention block for n consecutive tokens of one sequence.

    q [n, Hq, Dq], k [n, Hkv, Dk], v [n, Hkv, Dv] (raw, pre-norm/pre-RoPE),
    optional previous caches [prev, Hkv, D].  Returns (out [n, Hq, Dk],
    key_cache, value_cache) with the caches grown by n tokens.
    """
    q = np.array(q, dtype=np.float32, copy=True)
    k = np.array(k, dtype=np.float32, copy=True)
    v = _f32(v)
    n, hq, dq = q.shape
    _, hkv, dk = k.shape
    dv = v.shape[2]
    total = prev_seq_len + n
    kc = np.zeros((total, hkv, dk), dtype=np.float32)
    vc = np.zeros((total, hkv, dv), dtype=np.float32)
    if prev_seq_len:
        kc[:prev_seq_len] = key_cache[:prev_seq_len]
        vc[:prev_seq_len] = value_cache[:prev_seq_len]
    out = np.zeros((n, hq, dk), dtype=np.float32)
    g = _f32(gate) if gate is not None else None
    qn = _f32(q_norm_w) if q_norm_w is not None else None
    kn = _f32(k_norm_w) if k_norm_w is not None else None
    f = _f32(freqs) if freqs is not None else None
    lib().or_attn_layer_tokens(_p(out), _p(q), _p(g), _p(k), _p(v), n, hq, hkv, dq, dk, dv,
                               _p(qn), _p(kn), float(eps), rope_dim if rope_dim else dk,
                               float(rope_base), _p(f), 0 if f is None else f.size,
                               _p(kc), _p(vc), prev_seq_len)
    return out, kc, vc


def attn_prepare(q, k, n_heads, n_kv_heads, head_dim, q_norm_w=None, k_norm_w=None, eps=1e-6,
                 rope_dim=None, rope_base=10000.0, freqs=None, pos0=0, q_head_dim=None):
    """Q/K norm + RoPE driver for n consecutive tokens (no attention); returns copies.

    q [n, Hq, Dq] or None (Dq = q_head_dim, default head_dim), k [n, Hkv, D] or None;
    token i at position pos0 + i."""
    qq = None if q is None else np.array(q, dtype=np.float32, copy=True)
    kk = None if k is None else np.array(k, dtype=np.float32, copy=True)
    n = (qq if qq is not None else kk).shape[0]
    qn = _f32(q_norm_w) if q_norm_w is not None else None
    kn = _f32(k_norm_w) if k_norm_w is not None else None
    f = _f32(freqs) if freqs is not None else None
    lib().or_attn_prepare(_p(qq), _p(kk), n, n_heads, n_kv_heads,
                          head_dim if q_head_dim is None else q_head_dim, head_dim, _p(qn),
                          _p(kn), float(eps), rope_dim if rope_dim else head_dim,
                          float(rope_base), _p(f), 0 if f is None else f.size, pos0)
    return qq, kk


# ---- src/model/mod.rs gated-DeltaNet block ---------------------------------

def gdn_gates(beta_raw, a_raw, ssm_a, dt_bias):
    br, ar, sa, db = (_f32(x) for x in (beta_raw, a_raw, ssm_a, dt_bias))
    beta = np.empty_like(br)
    g = np.empty_like(br)
    lib().or_gdn_gates(_p(beta), _p(g), _p(br), _p(ar), _p(sa), _p(db), br.size)
    return beta, g


def gdn_tokens(q_raw, k_raw, v, beta, g, state=None):
    """q_raw/k_raw [T, Hk, Dk], v [T, Hv, Dv], beta/g [T, Hv]; state [Hv, Dk, Dv].

    Returns (out [T, Hv, Dv], final state)."""
    q, k, vv, b, gg = (_f32(x) for x in (q_raw, k_raw, v, beta, g))
    t, hk, dk = q.shape
    _, hv, dv = vv.shape
    assert k.shape == q.shape and b.shape == (t, hv) and gg.shape == (t, hv)
    st = (np.zeros((hv, dk, dv), dtype=np.float32) if state is None
          else np.array(state, dtype=np.float32, copy=True))
    out = np.zeros((t, hv, dv), dtype=np.float32)
    lib().or_gdn_tokens(_p(out), _p(st), _p(q), _p(k), _p(vv), _p(b), _p(gg), t, hk, hv, dk, dv)
    return out, st


def rmsnorm_gated(o, z, w, eps):
    o = np.array(o, dtype=np.float32, copy=True)
    zz, ww = _f32(z), _f32(w)
    hv, dv = o.shape[-2], o.shape[-1]
    rows = o.size // (hv * dv)
    lib().or_rmsnorm_gated(_p(o), _p(zz), _p(ww), rows * hv, dv, float(eps))
    return o


def ssm_forward(x, conv1d, ssm_a, dt_bias, alpha, beta, out_w, state, d_inner, d_state, d_conv):
    """ssm::ssm_forward (src/ssm/mod.rs:40-157); returns (y, new state).  conv1d / beta /
    out_w are used at their own lengths, as the reference's branches test them."""
    x, ssm_a, dt_bias, alpha = (_f32(a) for a in (x, ssm_a, dt_bias, alpha))
    conv1d, beta, out_w = (_f32(a) for a in (conv1d, beta, out_w))
    st = np.array(state, dtype=np.float32, copy=True).reshape(-1)
    y = np.zeros(d_inner, np.float32)
    lib().or_ssm_forward(_p(y), _p(x), _p(conv1d), conv1d.size, _p(ssm_a), _p(dt_bias),
                         _p(alpha), _p(beta), beta.size, _p(out_w), out_w.size, _p(st), d_inner,
                         d_state, d_conv)
    return y, st


def conv1d_silu(x, hist, w, d_conv):
    """One token: returns (activation, new history)."""
    x = np.array(x, dtype=np.float32, copy=True)
    h = np.array(hist, dtype=np.float32, copy=True)
    ww = _f32(w)
    lib().or_conv1d_silu(_p(x), _p(h), _p(ww), x.size, d_conv)
    return x, h


# ---- src/turboquant/mod.rs -------------------------------------------------

def _u8(a):
    arr = np.ascontiguousarray(a, dtype=np.uint8)
    return arr, arr.ctypes.data_as(_u8p)


def splitmix64(seed: int, n: int):
    """First n outputs of SplitMix64(seed) (src/turboquant/mod.rs:725-731)."""
    st = ctypes.c_uint64(seed)
    return [int(lib().or_splitmix64_next(ctypes.byref(st))) for _ in range(n)]


def splitmix64_gaussians(seed: int, n: int):
    st = ctypes.c_uint64(seed)
    return np.array([lib().or_splitmix64_gaussian(ctypes.byref(st)) for _ in range(n)],
                    dtype=np.float32)


def tq_orthogonal(dim: int, seed: int):
    out = np.empty((dim, dim), dtype=np.float32)
    lib().or_tq_orthogonal(_p(out), dim, seed)
    return out


def tq_gaussian_matrix(rows: int, cols: int, seed: int):
    out = np.empty((rows, cols), dtype=np.float32)
    lib().or_tq_gaussian_matrix(_p(out), rows, cols, seed)
    return out


def tq_matrices(dim: int, seed: int, qjl_bits: int = None):
    """(rotation, QJL matrix) of TurboQuant::new(bits, dim, qjl_bits, seed) (:76-103)."""
    qjl_bits = dim if qjl_bits is None else qjl_bits
    g = tq_gaussian_matrix(qjl_bits, dim, seed ^ 0xDEADBEEF) if qjl_bits else None
    return tq_orthogonal(dim, seed), g


def tq_centroids(bits: int):
    return np.array([lib().or_tq_centroid(bits, j) for j in range(1 << bits)], dtype=np.float32)


def tq_compressed_bytes(bits: int, dim: int, qjl_bits: int) -> int:
    return int(lib().or_tq_compressed_bytes(bits, dim, qjl_bits))


def tq_pack(idx, bits: int, signs=()):
    idx, pi = _u8(idx)
    sg, ps = _u8(np.asarray(signs, dtype=np.uint8).reshape(-1))
    out = np.zeros((idx.size * bits + sg.size + 7) // 8, dtype=np.uint8)
    lib().or_tq_pack(out.ctypes.data_as(_u8p), pi, idx.size, bits, ps, sg.size)
    return out


def tq_unpack(packed, n: int, bits: int, n_signs: int = 0):
    pk, pp = _u8(packed)
    idx = np.zeros(n, dtype=np.uint8)
    sg = np.zeros(max(n_signs, 1), dtype=np.uint8)
    lib().or_tq_unpack(idx.ctypes.data_as(_u8p), sg.ctypes.data_as(_u8p), pp, n, bits, n_signs)
    return idx, sg[:n_signs]


def tq_quantize(x, R, G, bits: int, qjl_bits: int):
    x, R = _f32(x), _f32(R)
    G = _f32(G) if G is not None else None
    dim = x.size
    out = np.zeros(tq_compressed_bytes(bits, dim, qjl_bits), dtype=np.uint8)
    lib().or_tq_quantize(out.ctypes.data_as(_u8p), _p(x), _p(R), _p(G), dim, bits, qjl_bits)
    return out


def tq_dequantize(packed, R, bits: int):
    R = _f32(R)
    dim = R.shape[0]
    pk, pp = _u8(packed)
    out = np.empty(dim, dtype=np.float32)
    lib().or_tq_dequantize(_p(out), pp, _p(R), dim, bits)
    return out


def tq_dot(q, packed, R, G, bits: int, qjl_bits: int) -> float:
    q, R = _f32(q), _f32(R)
    G = _f32(G) if G is not None else None
    pk, pp = _u8(packed)
    return float(lib().or_tq_dot(_p(q), pp, _p(R), _p(G), q.size, bits, qjl_bits))


def tq_cache_append_keys(keys, R, G):
    """keys [n_kv, dim] of one token -> (packed [n_kv, ceil(4 dim / 8)-byte records], norms [n_kv]);
    R, G [n_kv, dim, dim] (CompressedKVCache::append, :455-486)."""
    k, R, G = _f32(keys), _f32(R), _f32(G)
    n_kv, dim = k.shape
    nb = tq_compressed_bytes(3, dim, dim)
    packed = np.zeros((n_kv, nb), dtype=np.uint8)
    norms = np.zeros(n_kv, dtype=np.float32)
    lib().or_tq_cache_append_keys(packed.ctypes.data_as(_u8p), _p(norms), _p(k), _p(R), _p(G),
                                  n_kv, dim)
    return packed, norms


def tq_cache_attend(q_head, packed, norms, values_f16, R, G, kv_h: int):
    """One query head over a compressed cache: packed [T, n_kv, nb] uint8, norms [T, n_kv],
    values_f16 [T, n_kv, dim] float16, R, G [dim, dim] of KV head kv_h."""
    q, nm, R, G = _f32(q_head), _f32(norms), _f32(R), _f32(G)
    pk, pp = _u8(packed)
    vals = np.ascontiguousarray(values_f16, dtype=np.float16).view(np.uint16)
    T, n_kv, dim = vals.shape
    out = np.zeros(dim, dtype=np.float32)
    lib().or_tq_cache_attend(_p(out), _p(q), pp, _p(nm), vals.ctypes.data_as(_u16p), _p(R),
                             _p(G), T, n_kv, kv_h, dim)
    return out


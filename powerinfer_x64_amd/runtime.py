"""torch-tensor front end of libpi_attn.so (include/pi_attn.h).

torch provides device memory and the stream; every computation runs in the
library's HIP kernels.  Calls are issued on torch's current stream so they
order with surrounding torch work.  Errors raise PiError subclasses that
mirror the reference's BackendError (src/runtime/mod.rs:6-18).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence

import numpy as np
import torch

from . import _abi

F32, F16, BF16 = 0, 1, 2
MODULO, GROUPED = 0, 1
PAGE_TOKENS = 16

_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}


class PiError(RuntimeError):
    code = -1


class InvalidArg(PiError):
    code = 1


class OutOfMemory(PiError):
    code = 2


class InvalidKernel(PiError):
    code = 3


class DeviceError(PiError):
    code = 4


class Unsupported(PiError):
    code = 5


_ERRORS = {c.code: c for c in (InvalidArg, OutOfMemory, InvalidKernel, DeviceError, Unsupported)}


def _vp(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need(t: torch.Tensor, name: str, dtype=None, shape=None, dev=None):
    if not isinstance(t, torch.Tensor):
        raise InvalidArg(f"{name}: expected a torch.Tensor")
    if dev is not None and t.device != dev:
        raise InvalidArg(f"{name}: on {t.device}, expected {dev}")
    if dtype is not None and t.dtype != dtype:
        raise InvalidArg(f"{name}: dtype {t.dtype}, expected {dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise InvalidArg(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    if not t.is_contiguous():
        raise InvalidArg(f"{name}: must be contiguous")


class Device:
    """One pi_handle bound to a GPU (GpuDevice / GpuResources, src/cuda/mod.rs:141-460)."""

    def __init__(self, device: int = 0):
        self.lib = _abi.load()
        self.index = device
        self.torch_device = torch.device("cuda", device)
        h = ctypes.c_void_p()
        rc = self.lib.pi_create(device, ctypes.byref(h))
        if rc != 0:
            raise _ERRORS.get(rc, PiError)(self.lib.pi_last_error(None).decode())
        self.h = h

    def close(self):
        if self.h:
            self.lib.pi_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def stream(self):
        return ctypes.c_void_p(torch.cuda.current_stream(self.torch_device).cuda_stream)

    def check(self, rc: int):
        if rc != 0:
            raise _ERRORS.get(rc, PiError)(self.lib.pi_last_error(self.h).decode())

    def sync(self):
        self.check(self.lib.pi_sync(self.h, self.stream()))


class KvPool:
    """Paged KV cache in HBM: 16-token pages, one K and one V block per (page, kv head)."""

    def __init__(self, dev: Device, n_pages: int, n_kv_heads: int, head_dim: int,
                 dtype: torch.dtype = torch.float16, page_tokens: int = PAGE_TOKENS):
        self.dev = dev
        self.n_pages, self.n_kv_heads, self.head_dim = n_pages, n_kv_heads, head_dim
        self.dtype = dtype
        p = ctypes.c_void_p()
        code = _DTYPE_CODE.get(dtype, -1)
        dev.check(dev.lib.pi_kv_pool_create(dev.h, n_pages, page_tokens, n_kv_heads, head_dim,
                                            code, ctypes.byref(p)))
        self.p = p

    @property
    def nbytes(self) -> int:
        return int(self.dev.lib.pi_kv_pool_bytes(self.p))

    def close(self):
        if self.p:
            self.dev.lib.pi_kv_pool_destroy(self.p)
            self.p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def append(self, k: torch.Tensor, v: torch.Tensor, page_table: torch.Tensor,
               start_pos: torch.Tensor):
        """k, v: [n_seq, n_tok, n_kv_heads, head_dim] (f32/f16/bf16)."""
        d = self.dev
        if k.dim() != 4 or k.shape[2:] != (self.n_kv_heads, self.head_dim):
            raise InvalidArg(f"k: shape {tuple(k.shape)}")
        for name, t in (("k", k), ("v", v)):
            _need(t, name, dtype=k.dtype, shape=k.shape, dev=d.torch_device)
        n_seq, n_tok = k.shape[:2]
        _need(page_table, "page_table", torch.int32, dev=d.torch_device)
        _need(start_pos, "start_pos", torch.int32, (n_seq,), d.torch_device)
        if page_table.dim() != 2 or page_table.shape[0] < n_seq:
            raise InvalidArg(f"page_table: shape {tuple(page_table.shape)}")
        d.check(d.lib.pi_kv_append(d.h, self.p, _vp(k), _vp(v), _DTYPE_CODE.get(k.dtype, -1),
                                   _vp(page_table), page_table.shape[1], _vp(start_pos), n_seq,
                                   n_tok, d.stream()))

    def read(self, page_table: torch.Tensor, seq: int, start: int, n_tok: int):
        d = self.dev
        _need(page_table, "page_table", torch.int32, dev=d.torch_device)
        ko = torch.empty((n_tok, self.n_kv_heads, self.head_dim), dtype=torch.float32,
                         device=d.torch_device)
        vo = torch.empty_like(ko)
        d.check(d.lib.pi_kv_read(d.h, self.p, _vp(page_table), page_table.shape[1], seq, start,
                                 n_tok, _vp(ko), _vp(vo), d.stream()))
        return ko, vo


class AttnLayer:
    """LayerCache of one attention layer for one sequence, on the device
    (src/model/mod.rs:73-106), with the forward step of src/model/mod.rs:1035-1196 on host
    slices (numpy float32), as the reference's InferenceContext::forward hands them over."""

    def __init__(self, dev: Device, max_tokens: int, n_heads: int, n_kv_heads: int,
                 head_dim: int, kv_dtype: torch.dtype = torch.float16, q_norm_w=None,
                 k_norm_w=None, eps: float = 1e-6, rope_dim: int = None,
                 rope_base: float = 1e6, sections=None, gqa_mode: int = MODULO,
                 q_head_dim: int = None, v_head_dim: int = None):
        """head_dim is the key head width; q_head_dim (>= head_dim) and v_head_dim default to
        it (src/model/mod.rs:976-982: the three may differ)."""
        self.dev = dev
        self.n_heads, self.n_kv_heads, self.head_dim = n_heads, n_kv_heads, head_dim
        self.q_head_dim = head_dim if q_head_dim is None else q_head_dim
        self.v_head_dim = head_dim if v_head_dim is None else v_head_dim
        qn = None if q_norm_w is None else np.ascontiguousarray(q_norm_w, np.float32).reshape(-1)
        kn = None if k_norm_w is None else np.ascontiguousarray(k_norm_w, np.float32).reshape(-1)
        for name, w in (("q_norm_w", qn), ("k_norm_w", kn)):
            if w is not None and w.size != head_dim:
                raise InvalidArg(f"{name}: expected {head_dim} values, got {w.size}")
        sec = None if sections is None else (ctypes.c_int32 * 4)(*[int(x) for x in sections])
        p = ctypes.c_void_p()
        dev.check(dev.lib.pi_attn_layer_create_dims(
            dev.h, max_tokens, n_heads, n_kv_heads, self.q_head_dim, head_dim, self.v_head_dim,
            _DTYPE_CODE.get(kv_dtype, -1),
            None if qn is None else qn.ctypes.data_as(ctypes.c_void_p),
            None if kn is None else kn.ctypes.data_as(ctypes.c_void_p), float(eps),
            head_dim if rope_dim is None else rope_dim, float(rope_base), sec, gqa_mode,
            ctypes.byref(p)))
        self.p = p

    def close(self):
        if self.p:
            self.dev.lib.pi_attn_layer_destroy(self.p)
            self.p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def seq_len(self) -> int:
        return int(self.dev.lib.pi_attn_layer_seq_len(self.p))

    def reset(self):
        self.dev.lib.pi_attn_layer_reset(self.p)

    def forward(self, q: np.ndarray, k: np.ndarray, v: np.ndarray, gate=None):
        """q [n, Hq, Dq], k [n, Hkv, D], v [n, Hkv, Dv] float32 (q, k normalised / rotated in
        place); gate like q; returns out [n, Hq, D]."""
        n = q.shape[0]
        for name, a, h, d in (("q", q, self.n_heads, self.q_head_dim),
                              ("k", k, self.n_kv_heads, self.head_dim),
                              ("v", v, self.n_kv_heads, self.v_head_dim)):
            if (not isinstance(a, np.ndarray) or a.dtype != np.float32 or
                    not a.flags.c_contiguous or a.shape != (n, h, d)):
                raise InvalidArg(f"{name}: expected C-contiguous float32 [{n}, {h}, {d}]")
        g = None
        if gate is not None:
            g = np.ascontiguousarray(gate, np.float32)
            if g.shape != q.shape:
                raise InvalidArg(f"gate: shape {g.shape}")
        out = np.empty((n, self.n_heads, self.head_dim), np.float32)
        vp = lambda a: None if a is None else a.ctypes.data_as(ctypes.c_void_p)
        self.dev.check(self.dev.lib.pi_attn_layer_forward(self.dev.h, self.p, vp(q), vp(k), vp(v),
                                                          vp(g), n, vp(out)))
        return out

    def forward_dev(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    gate: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
        """The same step on device tensors (f32, q / gate [n, Hq, Dq], k [n, Hkv, D],
        v [n, Hkv, Dv]; q and k normalised / rotated in place), enqueued on torch's current
        stream; returns out [n, Hq, D]."""
        d = self.dev
        n = q.shape[0]
        _need(q, "q", torch.float32, (n, self.n_heads, self.q_head_dim), d.torch_device)
        _need(k, "k", torch.float32, (n, self.n_kv_heads, self.head_dim), d.torch_device)
        _need(v, "v", torch.float32, (n, self.n_kv_heads, self.v_head_dim), d.torch_device)
        if gate is not None:
            _need(gate, "gate", torch.float32, q.shape, d.torch_device)
        shp = (n, self.n_heads, self.head_dim)
        if out is None:
            out = torch.empty(shp, dtype=torch.float32, device=q.device)
        _need(out, "out", torch.float32, shp, d.torch_device)
        d.check(d.lib.pi_attn_layer_forward_dev(d.h, self.p, _vp(q), _vp(k), _vp(v), _vp(gate), n,
                                                _vp(out), d.stream()))
        return out


class GdnLayer:
    """Gated-DeltaNet layer of one sequence, on the device: the rolling conv state and the
    recurrent state (src/model/mod.rs:122-127), with the step of src/model/mod.rs:750-932 on
    host slices (numpy float32): conv1d + SiLU, q / k / v split, gates, the delta rule and
    RMSNormGated."""

    def __init__(self, dev: Device, n_k_heads: int, n_v_heads: int, k_hd: int, v_hd: int,
                 conv_w, ssm_a, dt_bias, norm_w, eps: float = 1e-6):
        self.dev = dev
        self.hk, self.hv, self.dk, self.dv = n_k_heads, n_v_heads, k_hd, v_hd
        self.conv_dim = 2 * n_k_heads * k_hd + n_v_heads * v_hd
        w = np.ascontiguousarray(conv_w, np.float32)
        if w.ndim != 2 or w.shape[0] != self.conv_dim:
            raise InvalidArg(f"conv_w: expected [{self.conv_dim}, d_conv], got {w.shape}")
        arrs = [np.ascontiguousarray(a, np.float32).reshape(-1) for a in (ssm_a, dt_bias, norm_w)]
        for name, a, m in zip(("ssm_a", "dt_bias", "norm_w"), arrs, (n_v_heads, n_v_heads, v_hd)):
            if a.size != m:
                raise InvalidArg(f"{name}: expected {m} values, got {a.size}")
        vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        p = ctypes.c_void_p()
        dev.check(dev.lib.pi_gdn_layer_create(dev.h, n_k_heads, n_v_heads, k_hd, v_hd,
                                              w.shape[1], vp(w), vp(arrs[0]), vp(arrs[1]),
                                              vp(arrs[2]), float(eps), ctypes.byref(p)))
        self.p = p

    def close(self):
        if self.p:
            self.dev.lib.pi_gdn_layer_destroy(self.p)
            self.p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        self.dev.check(self.dev.lib.pi_gdn_layer_reset(self.dev.h, self.p))

    def forward(self, qkv: np.ndarray, z: np.ndarray, beta_raw: np.ndarray, a_raw: np.ndarray):
        """qkv [n, conv_dim], z [n, Hv, Dv], beta_raw, a_raw [n, Hv] float32; returns the
        gated, normalised output [n, Hv, Dv]."""
        n = qkv.shape[0]
        for name, a, shp in (("qkv", qkv, (n, self.conv_dim)), ("z", z, (n, self.hv, self.dv)),
                             ("beta_raw", beta_raw, (n, self.hv)), ("a_raw", a_raw, (n, self.hv))):
            if (not isinstance(a, np.ndarray) or a.dtype != np.float32 or
                    not a.flags.c_contiguous or a.shape != shp):
                raise InvalidArg(f"{name}: expected C-contiguous float32 {list(shp)}")
        out = np.empty((n, self.hv, self.dv), np.float32)
        vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        self.dev.check(self.dev.lib.pi_gdn_layer_forward(self.dev.h, self.p, vp(qkv), vp(z),
                                                         vp(beta_raw), vp(a_raw), n, vp(out)))
        return out

    def forward_dev(self, qkv: torch.Tensor, z: torch.Tensor, beta_raw: torch.Tensor,
                    a_raw: torch.Tensor, out: Optional[torch.Tensor] = None):
        """The same step on device f32 tensors, enqueued on torch's current stream."""
        d = self.dev
        n = qkv.shape[0]
        for name, t, shp in (("qkv", qkv, (n, self.conv_dim)), ("z", z, (n, self.hv, self.dv)),
                             ("beta_raw", beta_raw, (n, self.hv)), ("a_raw", a_raw, (n, self.hv))):
            _need(t, name, torch.float32, shp, d.torch_device)
        if out is None:
            out = torch.empty((n, self.hv, self.dv), dtype=torch.float32, device=qkv.device)
        _need(out, "out", torch.float32, (n, self.hv, self.dv), d.torch_device)
        d.check(d.lib.pi_gdn_layer_forward_dev(d.h, self.p, _vp(qkv), _vp(z), _vp(beta_raw),
                                               _vp(a_raw), n, _vp(out), d.stream()))
        return out


class TqPool:
    """TurboQuant compressed KV cache (CompressedKVCache, src/turboquant/mod.rs:408-566) in
    16-token pages: ceil(head_dim/2)-byte 3-bit + QJL key records with f32 norms, f16
    values; head_dim 1..256."""

    def __init__(self, dev: Device, n_pages: int, n_kv_heads: int, head_dim: int = 128,
                 page_tokens: int = PAGE_TOKENS):
        self.dev = dev
        self.n_pages, self.n_kv_heads, self.head_dim = n_pages, n_kv_heads, head_dim
        self.KEY_BYTES = (4 * head_dim + 7) // 8
        p = ctypes.c_void_p()
        dev.check(dev.lib.pi_tq_pool_create(dev.h, n_pages, page_tokens, n_kv_heads, head_dim,
                                            ctypes.byref(p)))
        self.p = p

    @property
    def nbytes(self) -> int:
        return int(self.dev.lib.pi_tq_pool_bytes(self.p))

    def close(self):
        if self.p:
            self.dev.lib.pi_tq_pool_destroy(self.p)
            self.p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def append(self, k: torch.Tensor, v: torch.Tensor, page_table: torch.Tensor,
               start_pos: torch.Tensor):
        """k, v: [n_seq, n_tok, n_kv_heads, head_dim] f32."""
        d = self.dev
        if k.dim() != 4 or k.shape[2:] != (self.n_kv_heads, self.head_dim):
            raise InvalidArg(f"k: shape {tuple(k.shape)}")
        for name, t in (("k", k), ("v", v)):
            _need(t, name, dtype=torch.float32, shape=k.shape, dev=d.torch_device)
        n_seq, n_tok = k.shape[:2]
        _need(page_table, "page_table", torch.int32, dev=d.torch_device)
        _need(start_pos, "start_pos", torch.int32, (n_seq,), d.torch_device)
        if page_table.dim() != 2 or page_table.shape[0] < n_seq:
            raise InvalidArg(f"page_table: shape {tuple(page_table.shape)}")
        d.check(d.lib.pi_tq_append(d.h, self.p, _vp(k), _vp(v), _vp(page_table),
                                   page_table.shape[1], _vp(start_pos), n_seq, n_tok, d.stream()))

    def read(self, page_table: torch.Tensor, seq: int, start: int, n_tok: int):
        """(keys [n_tok, Hkv, ceil(head_dim/2)] uint8, norms [n_tok, Hkv] f32, values
        [n_tok, Hkv, head_dim] f16)."""
        d = self.dev
        _need(page_table, "page_table", torch.int32, dev=d.torch_device)
        ko = torch.empty((n_tok, self.n_kv_heads, self.KEY_BYTES), dtype=torch.uint8,
                         device=d.torch_device)
        no = torch.empty((n_tok, self.n_kv_heads), dtype=torch.float32, device=d.torch_device)
        vo = torch.empty((n_tok, self.n_kv_heads, self.head_dim), dtype=torch.float16,
                         device=d.torch_device)
        d.check(d.lib.pi_tq_read(d.h, self.p, _vp(page_table), page_table.shape[1], seq, start,
                                 n_tok, _vp(ko), _vp(no), _vp(vo), d.stream()))
        return ko, no, vo


def tq_generate(dim: int, seed: int):
    """Host only: (rotation, QJL matrix) of TurboQuant::new(bits, dim, dim, seed)."""
    lib = _abi.load()
    rot = np.empty((dim, dim), dtype=np.float32)
    qjl = np.empty((dim, dim), dtype=np.float32)
    rc = lib.pi_tq_generate(dim, seed, rot.ctypes.data_as(ctypes.c_void_p),
                            qjl.ctypes.data_as(ctypes.c_void_p))
    if rc != 0:
        raise _ERRORS.get(rc, PiError)(lib.pi_last_error(None).decode())
    return rot, qjl


def tq_attn_decode(dev: Device, q: torch.Tensor, pool: TqPool, page_table: torch.Tensor,
                   ctx_len: torch.Tensor, gqa_mode: int = MODULO,
                   gate: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
    """q [B, Hq, D] f32 -> out [B, Hq, D] f32 over each sequence's compressed cache."""
    _need(q, "q", torch.float32, dev=dev.torch_device)
    b, hq, dh = q.shape
    if dh != pool.head_dim:
        raise InvalidArg(f"q head_dim {dh} != pool head_dim {pool.head_dim}")
    _need(page_table, "page_table", torch.int32, dev=dev.torch_device)
    if page_table.dim() != 2 or page_table.shape[0] != b:
        raise InvalidArg(f"page_table: shape {tuple(page_table.shape)}")
    _need(ctx_len, "ctx_len", torch.int32, (b,), dev.torch_device)
    if gate is not None:
        _need(gate, "gate", torch.float32, q.shape, dev.torch_device)
    if out is None:
        out = torch.empty_like(q)
    _need(out, "out", torch.float32, q.shape, dev.torch_device)
    dev.check(dev.lib.pi_tq_attn_decode(dev.h, _vp(q), pool.p, _vp(page_table),
                                        page_table.shape[1], _vp(ctx_len), b, hq, gqa_mode,
                                        _vp(gate), _vp(out), dev.stream()))
    return out


def head_rmsnorm(dev: Device, x: torch.Tensor, w: torch.Tensor, eps: float):
    """In place: every row of the last dimension of x (f32) is RMS-normalised and scaled by w."""
    _need(x, "x", torch.float32, dev=dev.torch_device)
    dim = x.shape[-1]
    _need(w, "w", torch.float32, (dim,), dev.torch_device)
    dev.check(dev.lib.pi_head_rmsnorm(dev.h, _vp(x), _vp(w), x.numel() // dim, dim, dim,
                                      float(eps), dev.stream()))
    return x


def rope(dev: Device, q: torch.Tensor, k: Optional[torch.Tensor], pos: torch.Tensor,
         rope_dim: int, base: float, sections: Optional[Sequence[int]] = None):
    """In place on q [n_tok, Hq, D] and k [n_tok, Hkv, D] (f32) at positions pos [n_tok]."""
    _need(q, "q", torch.float32, dev=dev.torch_device)
    n_tok, hq, dh = q.shape
    hkv = 1
    if k is not None:
        _need(k, "k", torch.float32, dev=dev.torch_device)
        if k.shape[0] != n_tok or k.shape[2] != dh:
            raise InvalidArg(f"k: shape {tuple(k.shape)}")
        hkv = k.shape[1]
    _need(pos, "pos", torch.int32, (n_tok,), dev.torch_device)
    sec = None
    if sections is not None:
        sec = (ctypes.c_int32 * 4)(*[int(s) for s in sections])
    dev.check(dev.lib.pi_rope(dev.h, _vp(q), _vp(k), _vp(pos), n_tok, hq, hkv, dh, rope_dim,
                              float(base), sec, dev.stream()))
    return q, k


def attn_decode(dev: Device, q: torch.Tensor, pool: KvPool, page_table: torch.Tensor,
                ctx_len: torch.Tensor, gqa_mode: int = MODULO, scale: Optional[float] = None,
                gate: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
    """q [B, Hq, D] f32 -> out [B, Hq, D] f32 over each sequence's ctx_len[b] cached tokens."""
    _need(q, "q", torch.float32, dev=dev.torch_device)
    b, hq, dh = q.shape
    if dh != pool.head_dim:
        raise InvalidArg(f"q head_dim {dh} != pool head_dim {pool.head_dim}")
    _need(page_table, "page_table", torch.int32, dev=dev.torch_device)
    if page_table.dim() != 2 or page_table.shape[0] != b:
        raise InvalidArg(f"page_table: shape {tuple(page_table.shape)}")
    _need(ctx_len, "ctx_len", torch.int32, (b,), dev.torch_device)
    if gate is not None:
        _need(gate, "gate", torch.float32, q.shape, dev.torch_device)
    if out is None:
        out = torch.empty_like(q)
    _need(out, "out", torch.float32, q.shape, dev.torch_device)
    if scale is None:
        scale = 1.0 / math.sqrt(dh)
    dev.check(dev.lib.pi_attn_decode(dev.h, _vp(q), pool.p, _vp(page_table), page_table.shape[1],
                                     _vp(ctx_len), b, hq, gqa_mode, float(scale), _vp(gate),
                                     _vp(out), dev.stream()))
    return out


def attn_prefill(dev: Device, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 causal: bool = True, gqa_mode: int = MODULO, scale: Optional[float] = None,
                 out: Optional[torch.Tensor] = None):
    """q [B, S, Hq, D], k/v [B, S, Hkv, D] (bf16/f16) -> out [B, S, Hq, D] f32."""
    _need(q, "q", dev=dev.torch_device)
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise Unsupported(f"q: dtype {q.dtype} (bf16 or f16)")
    bsz, s, hq, dh = q.shape
    _need(k, "k", q.dtype, dev=dev.torch_device)
    hkv = k.shape[2]
    _need(k, "k", q.dtype, (bsz, s, hkv, dh), dev.torch_device)
    _need(v, "v", q.dtype, (bsz, s, hkv, dh), dev.torch_device)
    if out is None:
        out = torch.empty((bsz, s, hq, dh), dtype=torch.float32, device=q.device)
    _need(out, "out", torch.float32, (bsz, s, hq, dh), dev.torch_device)
    if scale is None:
        scale = 1.0 / math.sqrt(dh)
    dev.check(dev.lib.pi_attn_prefill(dev.h, _vp(q), _vp(k), _vp(v), _DTYPE_CODE[q.dtype], bsz,
                                      s, hq, hkv, dh, 1 if causal else 0, gqa_mode, float(scale),
                                      _vp(out), dev.stream()))
    return out


def attn_prefill_paged(dev: Device, q: torch.Tensor, pool: KvPool, page_row: torch.Tensor,
                       start_pos: int, gqa_mode: int = MODULO, scale: Optional[float] = None,
                       out: Optional[torch.Tensor] = None):
    """A chunk continuing a sequence: q [n, Hq, D] at positions start_pos .. start_pos + n - 1
    over the sequence's pages (page_row: int32 [max_pages]; the chunk's K/V appended first)
    -> out [n, Hq, D] f32.  q is f16 for an f16 pool, f32 for an f32 pool."""
    _need(q, "q", pool.dtype, dev=dev.torch_device)
    n, hq, dh = q.shape
    if dh != pool.head_dim:
        raise InvalidArg(f"q head_dim {dh} != pool head_dim {pool.head_dim}")
    _need(page_row, "page_row", torch.int32, dev=dev.torch_device)
    if out is None:
        out = torch.empty((n, hq, dh), dtype=torch.float32, device=q.device)
    _need(out, "out", torch.float32, (n, hq, dh), dev.torch_device)
    if scale is None:
        scale = 1.0 / math.sqrt(dh)
    dev.check(dev.lib.pi_attn_prefill_paged(dev.h, _vp(q), pool.p, _vp(page_row), page_row.numel(),
                                            int(start_pos), n, hq, gqa_mode, float(scale), _vp(out),
                                            dev.stream()))
    return out


def gdn_gates(dev: Device, beta_raw, a_raw, ssm_a, dt_bias):
    """beta_raw/a_raw [n_tok, Hv], ssm_a/dt_bias [Hv] (f32) -> (beta, g)."""
    n_tok, hv = beta_raw.shape
    for name, t, shp in (("beta_raw", beta_raw, (n_tok, hv)), ("a_raw", a_raw, (n_tok, hv)),
                         ("ssm_a", ssm_a, (hv,)), ("dt_bias", dt_bias, (hv,))):
        _need(t, name, torch.float32, shp, dev.torch_device)
    beta = torch.empty_like(beta_raw)
    g = torch.empty_like(beta_raw)
    dev.check(dev.lib.pi_gdn_gates(dev.h, _vp(beta_raw), _vp(a_raw), _vp(ssm_a), _vp(dt_bias),
                                   _vp(beta), _vp(g), n_tok, hv, dev.stream()))
    return beta, g


def _gdn_check(dev, q, k, v, beta, g, state, lead):
    hk, dk = q.shape[-2:]
    hv, dv = v.shape[-2:]
    _need(q, "q", torch.float32, (lead, hk, dk), dev.torch_device)
    _need(k, "k", torch.float32, (lead, hk, dk), dev.torch_device)
    _need(v, "v", torch.float32, (lead, hv, dv), dev.torch_device)
    _need(beta, "beta", torch.float32, (lead, hv), dev.torch_device)
    _need(g, "g", torch.float32, (lead, hv), dev.torch_device)
    return hk, hv, dk, dv


def gdn_decode(dev: Device, q, k, v, beta, g, state, out=None):
    """One step per sequence: q/k [B, Hk, Dk] raw, v [B, Hv, Dv], beta/g [B, Hv],
    state [B, Hv, Dk, Dv] (in/out)."""
    b = q.shape[0]
    hk, hv, dk, dv = _gdn_check(dev, q, k, v, beta, g, state, b)
    _need(state, "state", torch.float32, (b, hv, dk, dv), dev.torch_device)
    if out is None:
        out = torch.empty((b, hv, dv), dtype=torch.float32, device=q.device)
    _need(out, "out", torch.float32, (b, hv, dv), dev.torch_device)
    dev.check(dev.lib.pi_gdn_decode(dev.h, _vp(q), _vp(k), _vp(v), _vp(beta), _vp(g), _vp(state),
                                    _vp(out), b, hk, hv, dk, dv, dev.stream()))
    return out


def gdn_prefill(dev: Device, q, k, v, beta, g, state, out=None, chunk: int = 64):
    """n_tok tokens of one sequence: q/k [T, Hk, Dk], v [T, Hv, Dv], beta/g [T, Hv],
    state [Hv, Dk, Dv] (in/out)."""
    t = q.shape[0]
    hk, hv, dk, dv = _gdn_check(dev, q, k, v, beta, g, state, t)
    _need(state, "state", torch.float32, (hv, dk, dv), dev.torch_device)
    if out is None:
        out = torch.empty((t, hv, dv), dtype=torch.float32, device=q.device)
    _need(out, "out", torch.float32, (t, hv, dv), dev.torch_device)
    dev.check(dev.lib.pi_gdn_prefill(dev.h, _vp(q), _vp(k), _vp(v), _vp(beta), _vp(g),
                                     _vp(state), _vp(out), t, hk, hv, dk, dv, chunk,
                                     dev.stream()))
    return out


def ssm_forward(dev: Device, x, ssm_conv1d, ssm_a, ssm_dt_bias, ssm_alpha, ssm_beta, ssm_out,
                state: np.ndarray, d_inner: int, d_state: int, d_conv: int) -> np.ndarray:
    """ssm::ssm_forward (src/ssm/mod.rs:40-157) on host slices, computed on the GPU: returns
    y [d_inner] and updates `state` (float32 [d_state * d_inner], C-contiguous) in place.
    ssm_conv1d, ssm_beta and ssm_out pick the reference's branches by their lengths."""
    f = lambda a: np.ascontiguousarray(np.asarray(a, np.float32).reshape(-1))  # noqa: E731
    x, w, a, bias, alpha, beta, out_w = (f(v) for v in (x, ssm_conv1d, ssm_a, ssm_dt_bias,
                                                        ssm_alpha, ssm_beta, ssm_out))
    if (not isinstance(state, np.ndarray) or state.dtype != np.float32 or
            not state.flags.c_contiguous or state.size != d_state * d_inner):
        raise InvalidArg(f"state: expected C-contiguous float32 of {d_state * d_inner} values")
    for name, arr, n in (("x", x, d_inner), ("ssm_dt_bias", bias, d_inner),
                         ("ssm_a", a, d_state * d_inner), ("ssm_alpha", alpha, d_inner * d_inner)):
        if arr.size != n:
            raise InvalidArg(f"{name}: expected {n} values, got {arr.size}")
    y = np.empty(d_inner, np.float32)
    vp = lambda arr: arr.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    dev.check(dev.lib.pi_ssm_forward(dev.h, vp(y), vp(x), vp(w), w.size, vp(a), vp(bias),
                                     vp(alpha), vp(beta), beta.size, vp(out_w), out_w.size,
                                     vp(state), d_inner, d_state, d_conv))
    return y


def attention_head(dev: Device, q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                   seq_len: int, head_dim: int) -> np.ndarray:
    """ops::attention_head (src/ops.rs:213-247) on host slices, computed on the GPU."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k_cache, dtype=np.float32)
    v = np.ascontiguousarray(v_cache, dtype=np.float32)
    if q.size < head_dim or k.size < seq_len * head_dim or v.size < seq_len * head_dim:
        raise InvalidArg("attention_head: slice shorter than seq_len * head_dim")
    out = np.zeros(head_dim, dtype=np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    dev.check(dev.lib.pi_ops_attention_head(dev.h, out.ctypes.data_as(fp), q.ctypes.data_as(fp),
                                            k.ctypes.data_as(fp), v.ctypes.data_as(fp), seq_len,
                                            head_dim))
    return out


def gdn_conv1d(dev: Device, x, conv_state, w, out=None):
    """Depthwise causal conv1d + SiLU: x [n_seq, n_tok, conv_dim], conv_state
    [n_seq, d_conv-1, conv_dim] (in/out), w [conv_dim, d_conv] -> out like x."""
    n_seq, n_tok, conv_dim = x.shape
    d_conv = w.shape[1]
    _need(x, "x", torch.float32, dev=dev.torch_device)
    _need(conv_state, "conv_state", torch.float32, (n_seq, d_conv - 1, conv_dim), dev.torch_device)
    _need(w, "w", torch.float32, (conv_dim, d_conv), dev.torch_device)
    if out is None:
        out = torch.empty_like(x)
    _need(out, "out", torch.float32, x.shape, dev.torch_device)
    dev.check(dev.lib.pi_gdn_conv1d(dev.h, _vp(x), _vp(conv_state), _vp(w), _vp(out), n_seq, n_tok,
                                    conv_dim, d_conv, dev.stream()))
    return out


def gdn_rmsnorm_gated(dev: Device, o, z, w, eps: float):
    """In place on o [..., n_v_heads, v_hd]: o * rsqrt(mean(o^2) + eps) * w * silu(z)."""
    hv, dv = o.shape[-2:]
    _need(o, "o", torch.float32, dev=dev.torch_device)
    _need(z, "z", torch.float32, o.shape, dev.torch_device)
    _need(w, "w", torch.float32, (dv,), dev.torch_device)
    rows = o.numel() // (hv * dv)
    dev.check(dev.lib.pi_gdn_rmsnorm_gated(dev.h, _vp(o), _vp(z), _vp(w), rows, hv, dv, float(eps),
                                           dev.stream()))
    return o


def attn_prologue(dev: Device, q, k, v, pool: KvPool, page_table, start_pos, q_norm_w=None,
                  k_norm_w=None, eps: float = 1e-6, rope_dim: int = 0, rope_base: float = 10000.0,
                  sections: Optional[Sequence[int]] = None):
    """Norm + RoPE + append for q [n_seq, n_tok, Hq, D], k/v [n_seq, n_tok, Hkv, D]
    (f32; q and k rewritten in place, k and v appended at start_pos[s] + t)."""
    n_seq, n_tok, hq, dh = q.shape
    _need(q, "q", torch.float32, dev=dev.torch_device)
    _need(k, "k", torch.float32, (n_seq, n_tok, pool.n_kv_heads, pool.head_dim), dev.torch_device)
    _need(v, "v", torch.float32, k.shape, dev.torch_device)
    if dh != pool.head_dim:
        raise InvalidArg(f"q head_dim {dh} != pool head_dim {pool.head_dim}")
    _need(page_table, "page_table", torch.int32, dev=dev.torch_device)
    _need(start_pos, "start_pos", torch.int32, (n_seq,), dev.torch_device)
    for name, w in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w)):
        if w is not None:
            _need(w, name, torch.float32, (dh,), dev.torch_device)
    sec = None if sections is None else (ctypes.c_int32 * 4)(*[int(s) for s in sections])
    dev.check(dev.lib.pi_attn_prologue(dev.h, _vp(q), _vp(k), _vp(v), _vp(q_norm_w), _vp(k_norm_w),
                                       float(eps), int(rope_dim), float(rope_base), sec, pool.p,
                                       _vp(page_table), page_table.shape[1], _vp(start_pos), n_seq,
                                       n_tok, hq, dev.stream()))
    return q, k

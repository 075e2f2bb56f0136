"""Helpers shared by the GPU parity tests: seeded inputs, paged-cache setup,
the oracle-side cache preparation, and the parity metrics."""
from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from oracle import oracle as orc

_DEV = None


def device():
    """One pi_handle for the whole test session (cuda:0)."""
    global _DEV
    if _DEV is None:
        from powerinfer_x64_amd import runtime
        assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
        _DEV = runtime.Device(0)
    return _DEV


def to_dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def oracle_workers():
    """Threads for oracle work (ctypes releases the GIL): the GPU box's CPU share is 16."""
    return max(1, min(16, os.cpu_count() or 1))


def parallel_map(fn, items):
    """fn over items on oracle_workers() threads, results in order."""
    with ThreadPoolExecutor(max_workers=oracle_workers()) as ex:
        return list(ex.map(fn, items))


def row_rel_err(out, ref):
    """max over rows (last dim) of ||out - ref||_2 / ||ref||_2, in float64."""
    o = np.asarray(out, np.float64).reshape(-1, np.shape(ref)[-1])
    r = np.asarray(ref, np.float64).reshape(-1, np.shape(ref)[-1])
    num = np.linalg.norm(o - r, axis=1)
    den = np.maximum(np.linalg.norm(r, axis=1), 1e-30)
    return float((num / den).max())


def argmax_agreement(out, ref, vocab=8192, seed=99):
    """Synthetic logits W . vec(row) in float64 for both outputs (W ~ N(0,1)/sqrt(n)).

    Returns (n_rows, n_mismatch, n_ties): a mismatching row whose reference
    top-2 margin is below 2*max||W_i||*||out-ref|| is counted as a tie."""
    o = np.asarray(out, np.float64).reshape(out.shape[0], -1)
    r = np.asarray(ref, np.float64).reshape(ref.shape[0], -1)
    n = o.shape[1]
    w = np.random.default_rng(seed).standard_normal((vocab, n)) / math.sqrt(n)
    lo, lr = o @ w.T, r @ w.T
    wn = np.linalg.norm(w, axis=1).max()
    mism = ties = 0
    for i in range(o.shape[0]):
        a, b = int(lo[i].argmax()), int(lr[i].argmax())
        if a != b:
            top2 = np.sort(lr[i])[-2:]
            if top2[1] - top2[0] <= 2 * wn * np.linalg.norm(o[i] - r[i]):
                ties += 1
            else:
                mism += 1
    return o.shape[0], mism, ties


class PagedCase:
    """A batch of sequences with raw (pre-RoPE) K/V in a randomly permuted page table."""

    def __init__(self, rng, lens, hq, hkv, d, theta=1e6, rope_dim=None, sections=None,
                 q_norm_w=None, k_norm_w=None, eps=1e-6, extra_pages=3, f32_draws=False):
        self.lens = [int(x) for x in lens]
        self.hq, self.hkv, self.d = hq, hkv, d
        self.theta, self.sections = theta, sections
        self.rope_dim = rope_dim or d
        self.q_norm_w, self.k_norm_w, self.eps = q_norm_w, k_norm_w, eps
        self.freqs = (orc.compute_imrope_freqs(theta, self.rope_dim, sections)
                      if sections is not None else None)
        b = len(self.lens)
        self.max_pages = max(1, max((x + 15) // 16 for x in self.lens))
        n_used = sum((x + 15) // 16 for x in self.lens)
        self.n_pages = n_used + extra_pages
        perm = rng.permutation(self.n_pages).astype(np.int32)
        self.page_table = np.full((b, self.max_pages), -1, np.int32)
        off = 0
        for i, x in enumerate(self.lens):
            np_ = (x + 15) // 16
            self.page_table[i, :np_] = perm[off:off + np_]
            off += np_
        if f32_draws:  # float32 draws directly (large caches)
            draw = lambda shape: rng.standard_normal(shape, dtype=np.float32)  # noqa: E731
        else:
            draw = lambda shape: rng.standard_normal(shape).astype(np.float32)  # noqa: E731
        self.k = [draw((x, hkv, d)) for x in self.lens]
        self.v = [draw((x, hkv, d)) for x in self.lens]
        self.q = draw((b, hq, d))

    # ---- oracle side (the reference's functions on the same raw inputs) ----
    def oracle_caches(self, i, kv_round=None):
        """K (normed + rotated at 0..L-1) and V of sequence i, optionally rounded."""
        _, kr = orc.attn_prepare(None, self.k[i], self.hq, self.hkv, self.d,
                                 k_norm_w=self.k_norm_w, eps=self.eps, rope_dim=self.rope_dim,
                                 rope_base=self.theta, freqs=self.freqs, pos0=0)
        v = self.v[i]
        if kv_round is not None:
            kr = kr.astype(kv_round).astype(np.float32)
            v = v.astype(kv_round).astype(np.float32)
        return kr, v

    def oracle_q(self, i):
        qr, _ = orc.attn_prepare(self.q[i][None], None, self.hq, self.hkv, self.d,
                                 q_norm_w=self.q_norm_w, eps=self.eps, rope_dim=self.rope_dim,
                                 rope_base=self.theta, freqs=self.freqs,
                                 pos0=max(self.lens[i] - 1, 0))
        return qr[0]

    def oracle_out(self, i, kv_round=None, gate=None):
        if self.lens[i] == 0:
            return np.zeros((self.hq, self.d), np.float32)
        kc, vc = self.oracle_caches(i, kv_round)
        out = orc.attn_decode(self.oracle_q(i), kc, vc)
        if gate is not None:
            out = orc.apply_gate(out, gate)
        return out

    # ---- GPU side (norm, RoPE, append and decode all in the HIP library) ----
    def gpu_build(self, dev, pool_dtype):
        from powerinfer_x64_amd import runtime as rt
        pool = rt.KvPool(dev, self.n_pages, self.hkv, self.d, dtype=pool_dtype)
        pt = to_dev(self.page_table)
        nw = to_dev(self.k_norm_w) if self.k_norm_w is not None else None
        for i, x in enumerate(self.lens):
            if x == 0:
                continue
            k = to_dev(self.k[i])
            v = to_dev(self.v[i])
            if nw is not None:
                rt.head_rmsnorm(dev, k, nw, self.eps)
            pos = torch.arange(x, dtype=torch.int32, device=k.device)
            # K heads rotate like query heads; pass them as the q operand.
            rt.rope(dev, k, None, pos, self.rope_dim, self.theta, self.sections)
            row = pt[i:i + 1].contiguous()
            pool.append(k[None].contiguous(), v[None].contiguous(), row,
                        torch.zeros(1, dtype=torch.int32, device=k.device))
        self.pool, self.pt = pool, pt
        return pool

    def gpu_q(self, dev):
        from powerinfer_x64_amd import runtime as rt
        q = to_dev(self.q)
        if self.q_norm_w is not None:
            rt.head_rmsnorm(dev, q, to_dev(self.q_norm_w), self.eps)
        pos = to_dev(np.array([max(x - 1, 0) for x in self.lens], np.int32))
        rt.rope(dev, q, None, pos, self.rope_dim, self.theta, self.sections)
        return q

    def gpu_decode(self, dev, gqa_mode=0, gate=None):
        from powerinfer_x64_amd import runtime as rt
        q = self.gpu_q(dev)
        ctx = to_dev(np.array(self.lens, np.int32))
        g = to_dev(gate) if gate is not None else None
        out = rt.attn_decode(dev, q, self.pool, self.pt, ctx, gqa_mode=gqa_mode, gate=g)
        torch.cuda.synchronize()
        return out.cpu().numpy()

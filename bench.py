"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline (BASELINE.json metric "decode-attn HBM GB/s (% of peak) at 32k ctx;
prefill attn TFLOP/s"): one decode step of config 2 -- Qwen3-8B GQA
(32 q / 8 kv heads, head_dim 128), 32 sequences with context lengths drawn
uniformly from [1024, 32768], f16 KV in 16-token pages under a randomly
permuted page table.  A step is one pi_attn_decode launch over the whole
batch with K/V already resident in HBM.  `value` is algorithmic bytes (K and V
of every cached token once, q, out, page-table entries) per second.

Also reported (same line, "prefill"/"workloads"): config 3 causal prefill
TFLOP/s, the all-32k variant of config 2, config 4 gated decode, config 1,
and the gated-DeltaNet decode step.  Inputs are synthetic N(0,1) generated on
the GPU from fixed seeds; RoPE is applied by the library's own kernel.

Timing: after `warmup` calls and a synchronize, one HIP event pair on the
library's stream brackets `steps` back-to-back calls, followed by a
synchronize; ms_per_step is that interval / steps.  A second pass with an
event pair per call gives the median and minimum.

cpu_baseline: the oracle (a C restatement of the reference's CPU loops,
single core) on the same decode inputs read back from the pool.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16/bf16
PAGE = 16


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--cpu-seconds", type=float, default=20.0,
                   help="budget of the single-core CPU baseline sample")
    p.add_argument("--only-headline", action="store_true")
    p.add_argument("--workload", default=None,
                   choices=["c1", "c2", "c2_32k", "c3", "c4", "gdn", "gdn_prefill", "tq", "copy",
                            "rows_f"],
                   help="time one workload only and print its figures (for sweeps)")
    return p.parse_args()


class Timer:
    """HIP events on the stream the library launches on (torch's current stream)."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, fn, steps, warmup):
        """ms_avg: one event pair around `steps` back-to-back calls (the timed
        region, host submission overlapped with the GPU); ms_median / ms_min:
        a second pass with an event pair around each call."""
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        avg = a.elapsed_time(b) / steps
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
        for x, y in ev:
            x.record()
            fn()
            y.record()
        torch.cuda.synchronize()
        per = [x.elapsed_time(y) for x, y in ev]  # ms
        return {"ms_avg": float(avg), "ms_median": float(np.median(per)),
                "ms_min": float(np.min(per)), "wall_s": wall}


def _paged_decode_setup(torch, rt, dev, lens, hq, hkv, d, theta, seed, sections=None,
                        rope_dim=None, qk_norm=False, eps=1e-6, pool_dtype=None):
    """Builds a pool holding RoPE'd K and V for every sequence (generated on the GPU)."""
    rng = np.random.default_rng(seed)
    n_pages_seq = [(int(x) + PAGE - 1) // PAGE for x in lens]
    total = sum(n_pages_seq)
    max_pages = max(n_pages_seq)
    perm = rng.permutation(total).astype(np.int32)
    pt = np.full((len(lens), max_pages), -1, np.int32)
    off = 0
    for i, n in enumerate(n_pages_seq):
        pt[i, :n] = perm[off:off + n]
        off += n
    pool_dtype = pool_dtype or torch.float16
    pool = rt.KvPool(dev, total, hkv, d, dtype=pool_dtype)
    kv_bytes = 2 if pool_dtype == torch.float16 else 4
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    tpt = torch.from_numpy(pt).cuda()
    rd = rope_dim or d
    qn = kn = None
    if qk_norm:
        qn = torch.rand(d, generator=g, device="cuda") + 0.5
        kn = torch.rand(d, generator=g, device="cuda") + 0.5
    zero = torch.zeros(1, dtype=torch.int32, device="cuda")
    for i, x in enumerate(lens):
        x = int(x)
        k = torch.randn((x, hkv, d), generator=g, device="cuda")
        v = torch.randn((x, hkv, d), generator=g, device="cuda")
        if kn is not None:
            rt.head_rmsnorm(dev, k, kn, eps)
        rt.rope(dev, k, None, torch.arange(x, dtype=torch.int32, device="cuda"), rd, theta,
                sections)
        pool.append(k[None], v[None], tpt[i:i + 1].contiguous(), zero)
        del k, v
    q = torch.randn((len(lens), hq, d), generator=g, device="cuda")
    if qn is not None:
        rt.head_rmsnorm(dev, q, qn, eps)
    ctx = torch.tensor([int(x) for x in lens], dtype=torch.int32, device="cuda")
    rt.rope(dev, q, None, ctx - 1, rd, theta, sections)
    torch.cuda.synchronize()
    algo = (sum(int(x) for x in lens) * hkv * d * 2 * kv_bytes  # K and V
            + 2 * len(lens) * hq * d * 4                # q in, out
            + total * 4 + len(lens) * 4)                # page-table entries, lengths
    return pool, tpt, ctx, q, algo


def _decode_fn(dev, pool, tpt, ctx, q, out, gate=None):
    lib = dev.lib
    args = (dev.h, ctypes.c_void_p(q.data_ptr()), pool.p, ctypes.c_void_p(tpt.data_ptr()),
            tpt.shape[1], ctypes.c_void_p(ctx.data_ptr()), q.shape[0], q.shape[1], 0,
            1.0 / math.sqrt(q.shape[2]),
            None if gate is None else ctypes.c_void_p(gate.data_ptr()),
            ctypes.c_void_p(out.data_ptr()), None)

    def fn():
        rc = lib.pi_attn_decode(*args)
        if rc:
            raise RuntimeError(lib.pi_last_error(dev.h).decode())
    return fn


def bench_decode(torch, rt, dev, timer, lens, hq, hkv, d, theta, seed, steps, warmup, **kw):
    gate_on = kw.pop("gate", False)
    pool, tpt, ctx, q, algo = _paged_decode_setup(torch, rt, dev, lens, hq, hkv, d, theta, seed,
                                                  **kw)
    out = torch.empty_like(q)
    gate = torch.randn(q.shape, device="cuda") if gate_on else None
    if gate is not None:
        algo += gate.numel() * 4
    t = timer.run(_decode_fn(dev, pool, tpt, ctx, q, out, gate), steps, warmup)
    gbs = algo / (t["ms_avg"] * 1e-3) / 1e9
    res = {"GB_s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS, "ms_per_step": t["ms_avg"],
           "ms_median": t["ms_median"], "bytes_per_launch": algo,
           "tokens": int(sum(int(x) for x in lens))}
    return res, (pool, tpt, ctx, q, out, gate)


def bench_tq_decode(torch, rt, dev, timer, lens, hq, hkv, seed, steps, warmup):
    """TurboQuant compressed-KV decode (pi_tq_attn_decode) over the config 2 shape: the
    cache is appended through pi_tq_append (K, V ~ N(0,1) generated on the GPU); the timed
    call includes the per-query precompute and the merge."""
    d = 128
    rng = np.random.default_rng(seed)
    n_pages_seq = [(int(x) + PAGE - 1) // PAGE for x in lens]
    total = sum(n_pages_seq)
    perm = rng.permutation(total).astype(np.int32)
    pt = np.full((len(lens), max(n_pages_seq)), -1, np.int32)
    off = 0
    for i, n in enumerate(n_pages_seq):
        pt[i, :n] = perm[off:off + n]
        off += n
    pool = rt.TqPool(dev, total, hkv)
    tpt = torch.from_numpy(pt).cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    zero = torch.zeros(1, dtype=torch.int32, device="cuda")
    t0 = time.perf_counter()
    for i, x in enumerate(lens):
        k = torch.randn((1, int(x), hkv, d), generator=g, device="cuda")
        v = torch.randn((1, int(x), hkv, d), generator=g, device="cuda")
        pool.append(k, v, tpt[i:i + 1].contiguous(), zero)
        del k, v
    torch.cuda.synchronize()
    append_s = time.perf_counter() - t0
    q = torch.randn((len(lens), hq, d), generator=g, device="cuda")
    ctx = torch.tensor([int(x) for x in lens], dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    lib = dev.lib
    args = (dev.h, ctypes.c_void_p(q.data_ptr()), pool.p, ctypes.c_void_p(tpt.data_ptr()),
            tpt.shape[1], ctypes.c_void_p(ctx.data_ptr()), len(lens), hq, 0, None,
            ctypes.c_void_p(out.data_ptr()), None)

    def fn():
        rc = lib.pi_tq_attn_decode(*args)
        if rc:
            raise RuntimeError(lib.pi_last_error(dev.h).decode())
    t = timer.run(fn, steps, warmup)
    tokens = sum(int(x) for x in lens)
    # per token and KV head: 64-byte key record + f32 norm + 128 f16 values
    algo = (tokens * hkv * (64 + 4 + d * 2) + 2 * len(lens) * hq * d * 4
            + total * 4 + len(lens) * 4 + 2 * hkv * d * d * 4)
    gbs = algo / (t["ms_avg"] * 1e-3) / 1e9
    f16_equiv = tokens * hkv * d * 2 * 2
    res = {"GB_s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS, "ms_per_step": t["ms_avg"],
           "ms_median": t["ms_median"], "bytes_per_launch": algo, "tokens": tokens,
           "kv_bytes_vs_f16_pool": round(tokens * hkv * (68 + d * 2) / f16_equiv, 4),
           "append_tokens_per_s": tokens / append_s}
    del pool
    return res


def cpu_baseline_decode(torch, rt, dev, state, lens, hq, hkv, d, budget_s):
    """Oracle (single core) on sequences of the same workload until the budget is spent."""
    from oracle import oracle as orc
    pool, tpt, ctx, q, out, _ = state
    qh = q.cpu().numpy()
    oh = out.cpu().numpy()
    t_cpu = 0.0
    nbytes = 0
    done = 0
    max_rel = 0.0
    for i, x in enumerate(lens):
        x = int(x)
        ko, vo = pool.read(tpt, i, 0, x)
        torch.cuda.synchronize()
        kh, vh = ko.cpu().numpy(), vo.cpu().numpy()
        t0 = time.perf_counter()
        ref = orc.attn_decode(qh[i], kh, vh)
        t_cpu += time.perf_counter() - t0
        nbytes += x * hkv * d * 2 * 2 + 2 * hq * d * 4
        done += 1
        rel = np.linalg.norm(oh[i] - ref, axis=1) / np.linalg.norm(ref, axis=1)
        max_rel = max(max_rel, float(rel.max()))
        if t_cpu >= budget_s:
            break
    return {"value": nbytes / t_cpu / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle or_attn_decode (C restatement of src/model/mod.rs:1154-1190, "
                      f"gcc -O3 -msse4.1, 1 thread) on {done} of {len(lens)} sequences "
                      f"({sum(int(x) for x in lens[:done])} tokens) read back from the pool as "
                      f"f32; {t_cpu:.1f} s",
            "parity_max_row_rel_err": max_rel}


def bench_prefill(torch, rt, dev, timer, s, hq, hkv, d, theta, seed, steps, warmup):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    q = torch.randn((s, hq, d), generator=g, device="cuda")
    k = torch.randn((s, hkv, d), generator=g, device="cuda")
    v = torch.randn((s, hkv, d), generator=g, device="cuda")
    pos = torch.arange(s, dtype=torch.int32, device="cuda")
    rt.rope(dev, q, k, pos, d, theta)
    qb, kb, vb = (t.to(torch.bfloat16)[None].contiguous() for t in (q, k, v))
    out = torch.empty((1, s, hq, d), device="cuda")
    lib = dev.lib
    args = (dev.h, ctypes.c_void_p(qb.data_ptr()), ctypes.c_void_p(kb.data_ptr()),
            ctypes.c_void_p(vb.data_ptr()), 2, 1, s, hq, hkv, d, 1, 0, 1.0 / math.sqrt(d),
            ctypes.c_void_p(out.data_ptr()), None)

    def fn():
        rc = lib.pi_attn_prefill(*args)
        if rc:
            raise RuntimeError(lib.pi_last_error(dev.h).decode())

    t = timer.run(fn, steps, warmup)
    flops = 4.0 * hq * d * s * (s + 1) / 2
    tf = flops / (t["ms_avg"] * 1e-3) / 1e12
    return {"TFLOP_s": tf, "mfma_frac": tf / MFMA_F16_PEAK_TFLOPS, "ms_per_step": t["ms_avg"],
            "flops_per_launch": flops, "tokens_per_s": s / (t["ms_avg"] * 1e-3)}


def bench_gdn_decode(torch, rt, dev, timer, steps, warmup):
    hk, hv, dk, dv = 16, 32, 128, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(0x5EED0004)
    q = torch.randn((1, hk, dk), generator=g, device="cuda")
    k = torch.randn((1, hk, dk), generator=g, device="cuda")
    v = torch.randn((1, hv, dv), generator=g, device="cuda")
    beta = torch.sigmoid(torch.randn((1, hv), generator=g, device="cuda"))
    gg = -torch.nn.functional.softplus(torch.randn((1, hv), generator=g, device="cuda"))
    state = torch.zeros((1, hv, dk, dv), device="cuda")
    out = torch.empty((1, hv, dv), device="cuda")
    lib = dev.lib
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    args = (dev.h, P(q), P(k), P(v), P(beta), P(gg), P(state), P(out), 1, hk, hv, dk, dv, None)

    def fn():
        rc = lib.pi_gdn_decode(*args)
        if rc:
            raise RuntimeError(lib.pi_last_error(dev.h).decode())

    t = timer.run(fn, steps, warmup)
    algo = 2 * hv * dk * dv * 4 + (2 * hk * dk + 2 * hv * dv + 2 * hv) * 4
    gbs = algo / (t["ms_avg"] * 1e-3) / 1e9
    return {"us_per_step": t["ms_avg"] * 1e3, "tokens_per_s": 1e3 / t["ms_avg"], "GB_s": gbs,
            "hbm_frac": gbs / HBM_PEAK_GBS, "bytes_per_launch": algo}


def bench_gdn_prefill(torch, rt, dev, timer, steps, warmup, t=4096):
    """Config 5 prefill: 4096 tokens, chunk 64, from a zero state."""
    hk, hv, dk, dv = 16, 32, 128, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(0x5EED0005)
    q = torch.randn((t, hk, dk), generator=g, device="cuda")
    k = torch.randn((t, hk, dk), generator=g, device="cuda")
    v = torch.randn((t, hv, dv), generator=g, device="cuda")
    beta = torch.sigmoid(torch.randn((t, hv), generator=g, device="cuda"))
    gg = -torch.nn.functional.softplus(torch.randn((t, hv), generator=g, device="cuda"))
    state = torch.zeros((hv, dk, dv), device="cuda")
    out = torch.empty((t, hv, dv), device="cuda")
    lib = dev.lib
    P = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    args = (dev.h, P(q), P(k), P(v), P(beta), P(gg), P(state), P(out), t, hk, hv, dk, dv, 64,
            None)

    def fn():
        rc = lib.pi_gdn_prefill(*args)
        if rc:
            raise RuntimeError(lib.pi_last_error(dev.h).decode())

    r = timer.run(fn, steps, warmup)
    nc = (t + 63) // 64
    # algorithmic bytes: f32 q, k, v, beta, g in; out and state in + out
    algo = (2 * t * hk * dk + t * hv * dv + 2 * t * hv + t * hv * dv + 2 * hv * dk * dv) * 4
    c = 64
    flops = nc * hv * (6 * c * dk * dv + 6 * c * c * dk + 4 * c * c * dv + (2 / 3) * c ** 3)
    s = r["ms_avg"] * 1e-3
    return {"ms_per_step": r["ms_avg"], "tokens_per_s": t / s, "GB_s": algo / s / 1e9,
            "hbm_frac": algo / s / 1e9 / HBM_PEAK_GBS, "TFLOP_s": flops / s / 1e12,
            "bytes_per_launch": algo, "flops_per_launch": flops}


def _lib_fn(dev, entry, args):
    """A timed call of one C entry point with prepared ctypes arguments."""
    lib = dev.lib

    def fn():
        rc = entry(*args)
        if rc:
            raise RuntimeError(lib.pi_last_error(dev.h).decode())
    return fn


def _hbm(r, algo):
    s = r["ms_avg"] * 1e-3
    return {"us_per_call": r["ms_avg"] * 1e3, "GB_s": algo / s / 1e9,
            "hbm_frac": algo / s / 1e9 / HBM_PEAK_GBS, "bytes_per_launch": algo}


def bench_rows_f(torch, rt, dev, timer, steps, warmup):
    """The steps either side of the path: the fused attention prologue (row f1:
    per-head RMSNorm, RoPE, paged append in one launch) and the GDN conv1d and
    RMSNormGated (row f2), at a prompt shape (HBM-bound) and a decode step."""
    P = lambda x: None if x is None else ctypes.c_void_p(x.data_ptr())  # noqa: E731
    lib = dev.lib
    res = {}
    g = torch.Generator(device="cuda")
    g.manual_seed(0x5EED00F1)

    def prologue(n_seq, n_tok, hq, hkv, d, rope_dim, base, sections, norm, start):
        pages = (start + n_tok + 15) // 16
        pool = rt.KvPool(dev, n_seq * pages, hkv, d, torch.float16)
        pt = torch.arange(n_seq * pages, dtype=torch.int32, device="cuda").view(n_seq, pages)
        sp = torch.full((n_seq,), start, dtype=torch.int32, device="cuda")
        q = torch.randn((n_seq, n_tok, hq, d), generator=g, device="cuda")
        k = torch.randn((n_seq, n_tok, hkv, d), generator=g, device="cuda")
        v = torch.randn((n_seq, n_tok, hkv, d), generator=g, device="cuda")
        wq = torch.rand((d,), generator=g, device="cuda") + 0.5 if norm else None
        wk = torch.rand((d,), generator=g, device="cuda") + 0.5 if norm else None
        sec = None if sections is None else (ctypes.c_int32 * 4)(*sections)
        args = (dev.h, P(q), P(k), P(v), P(wq), P(wk), 1e-6, rope_dim, base, sec, pool.p, P(pt),
                pages, P(sp), n_seq, n_tok, hq, None)
        r = timer.run(_lib_fn(dev, lib.pi_attn_prologue, args), steps, warmup)
        # q and k read and rewritten (f32), v read, k and v appended (f16)
        algo = n_seq * n_tok * d * (4 * (2 * hq + 3 * hkv) + 2 * 2 * hkv)
        pool.close()
        return _hbm(r, algo)

    res["f1_prologue_prompt_c3"] = prologue(1, 4096, 32, 8, 128, 128, 1e6, None, False, 0)
    res["f1_prologue_decode_c4"] = prologue(8, 1, 16, 2, 256, 64, 1e7, [11, 11, 10, 0], True,
                                            65535)

    hk, hv, dk, dv, d_conv = 16, 32, 128, 128, 4
    conv_dim = 2 * hk * dk + hv * dv
    w = torch.randn((conv_dim, d_conv), generator=g, device="cuda") * 0.5
    nw = torch.rand((dv,), generator=g, device="cuda") + 0.5
    for name, t in (("prompt_c5", 4096), ("decode_step", 1)):
        x = torch.randn((1, t, conv_dim), generator=g, device="cuda")
        cs = torch.randn((1, d_conv - 1, conv_dim), generator=g, device="cuda")
        xo = torch.empty_like(x)
        args = (dev.h, P(x), P(cs), P(w), P(xo), 1, t, conv_dim, d_conv, None)
        r = timer.run(_lib_fn(dev, lib.pi_gdn_conv1d, args), steps, warmup)
        # x read, out written, state read and written, weights read
        res["f2_gdn_conv1d_" + name] = _hbm(
            r, (2 * t * conv_dim + 2 * (d_conv - 1) * conv_dim + conv_dim * d_conv) * 4)
        o = torch.randn((t, hv, dv), generator=g, device="cuda")
        z = torch.randn((t, hv, dv), generator=g, device="cuda")
        args = (dev.h, P(o), P(z), P(nw), t, hv, dv, 1e-6, None)
        r = timer.run(_lib_fn(dev, lib.pi_gdn_rmsnorm_gated, args), steps, warmup)
        res["f2_gdn_rmsnorm_gated_" + name] = _hbm(r, (3 * t * hv * dv + dv) * 4)

    # row f3: one layer of `forward` through the host-slice seam (synchronous,
    # host <-> device copies of the slices included): wall clock per call
    rng = np.random.default_rng(0x5EED00F3)
    f32 = np.float32
    prompt, n_dec = 1024, 50

    def layer_times(reset, step_prompt, step_token):
        for _ in range(2):  # warm-up
            reset()
            step_prompt()
        reps = []
        for _ in range(3):
            reset()
            t0 = time.perf_counter()
            step_prompt()
            reps.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        for _ in range(n_dec):
            step_token()
        dec = (time.perf_counter() - t0) / n_dec
        tp = float(np.median(reps))
        return ({"ms_per_call": tp * 1e3, "tokens_per_s": prompt / tp},
                {"us_per_token": dec * 1e6, "tokens_per_s": 1.0 / dec})

    hq, hkv, d = 16, 2, 256
    lay = rt.AttnLayer(dev, prompt + n_dec + 16, hq, hkv, d, torch.float16,
                       q_norm_w=rng.uniform(0.5, 1.5, d).astype(f32),
                       k_norm_w=rng.uniform(0.5, 1.5, d).astype(f32), rope_dim=64,
                       rope_base=1e7, sections=[11, 11, 10, 0])
    qa, ka, va, ga = (rng.standard_normal((prompt, h, d)).astype(f32)
                      for h in (hq, hkv, hkv, hq))
    q1, k1, v1, g1 = (np.ascontiguousarray(x[:1]) for x in (qa, ka, va, ga))
    pr, dc = layer_times(lay.reset, lambda: lay.forward(qa, ka, va, ga),
                         lambda: lay.forward(q1, k1, v1, g1))
    res["f3_attn_layer_prompt_1024_c4"] = pr
    res["f3_attn_layer_decode_token_c4"] = dc
    lay.close()
    gl = rt.GdnLayer(dev, hk, hv, dk, dv, (rng.standard_normal((conv_dim, d_conv)) * 0.5).astype(f32),
                     -np.exp(rng.standard_normal(hv)).astype(f32),
                     rng.standard_normal(hv).astype(f32), rng.uniform(0.5, 1.5, dv).astype(f32))
    xa = rng.standard_normal((prompt, conv_dim)).astype(f32)
    za = rng.standard_normal((prompt, hv, dv)).astype(f32)
    ba, aa = (rng.standard_normal((prompt, hv)).astype(f32) for _ in range(2))
    x1, z1, b1, a1 = (np.ascontiguousarray(x[:1]) for x in (xa, za, ba, aa))
    pr, dc = layer_times(gl.reset, lambda: gl.forward(xa, za, ba, aa),
                         lambda: gl.forward(x1, z1, b1, a1))
    res["f3_gdn_layer_prompt_1024_c5"] = pr
    res["f3_gdn_layer_decode_token_c5"] = dc
    gl.close()
    return res


def bench_copy(torch, timer, steps, warmup, nbytes=1 << 30):
    """A plain device copy of known size: the calibration kernel for the
    FETCH_SIZE / WRITE_SIZE counters, and the practical HBM ceiling."""
    src = torch.randn(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    t = timer.run(lambda: dst.copy_(src), steps, warmup)
    moved = 2 * nbytes
    return {"bytes_read": nbytes, "bytes_written": nbytes, "ms_per_step": t["ms_avg"],
            "GB_s": moved / (t["ms_avg"] * 1e-3) / 1e9,
            "hbm_frac": moved / (t["ms_avg"] * 1e-3) / 1e9 / HBM_PEAK_GBS}


def _traffic(summary, kernels):
    """HBM bytes per launch (read + write, copy-calibrated FETCH_SIZE / WRITE_SIZE)
    summed over `kernels`, from the committed rocprofv3 PMC table in
    profiles/<summary>.txt; None when the summary has no such table."""
    p = os.path.join(ROOT, "profiles", f"{summary}.txt")
    if not os.path.exists(p):
        return None
    total, seen, in_table = 0, set(), False
    for line in open(p):
        f = line.split()
        if f[:3] == ["kernel", "FETCH_KiB", "WRITE_KiB"]:
            in_table = True
            continue
        if in_table and len(f) == 5 and f[0] in kernels:
            total += int(float(f[3])) + int(float(f[4]))
            seen.add(f[0])
    return total if seen == set(kernels) else None


def _single(torch, rt, dev, timer, a):
    w, st, wu = a.workload, a.steps, a.warmup
    if w == "c2":
        rng = np.random.default_rng(0x5EED0001)
        lens = [int(x) for x in rng.integers(1024, 32769, size=32)]
        return bench_decode(torch, rt, dev, timer, lens, 32, 8, 128, 1e6, 0x5EED0001, st, wu)[0]
    if w == "c2_32k":
        return bench_decode(torch, rt, dev, timer, [32768] * 32, 32, 8, 128, 1e6, 0x5EED0011, st,
                            wu)[0]
    if w == "c4":
        return bench_decode(torch, rt, dev, timer, [65536] * 8, 16, 2, 256, 1e7, 0x5EED0003, st,
                            wu, sections=[11, 11, 10, 0], rope_dim=64, qk_norm=True,
                            gate=True)[0]
    if w == "c1":
        return bench_decode(torch, rt, dev, timer, [513], 32, 32, 128, 1e4, 0x5EED0000, st, wu,
                            pool_dtype=torch.float32)[0]
    if w == "c3":
        return bench_prefill(torch, rt, dev, timer, 4096, 32, 8, 128, 1e6, 0x5EED0002, st, wu)
    if w == "gdn_prefill":
        return bench_gdn_prefill(torch, rt, dev, timer, st, wu)
    if w == "tq":
        rng = np.random.default_rng(0x5EED0001)
        lens = [int(x) for x in rng.integers(1024, 32769, size=32)]
        return bench_tq_decode(torch, rt, dev, timer, lens, 32, 8, 0x5EED0004, st, wu)
    if w == "copy":
        return bench_copy(torch, timer, st, wu)
    if w == "rows_f":
        return bench_rows_f(torch, rt, dev, timer, st, wu)
    return bench_gdn_decode(torch, rt, dev, timer, st, wu)


def main():
    a = _args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {a.gpus} is not supported "
              f"(the hot path's sharding is described in DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch
    from powerinfer_x64_amd import runtime as rt

    dev = rt.Device(0)
    timer = Timer(torch)
    if a.workload:
        print(json.dumps({"workload": a.workload, "pps_env": os.environ.get("PI_DECODE_PPS"),
                          **_single(torch, rt, dev, timer, a)}), flush=True)
        return

    # ---- headline: config 2 decode ----
    rng = np.random.default_rng(0x5EED0001)
    lens = [int(x) for x in rng.integers(1024, 32769, size=32)]
    c2, state = bench_decode(torch, rt, dev, timer, lens, 32, 8, 128, 1e6, 0x5EED0001, a.steps,
                             a.warmup)
    t_cpu0 = time.perf_counter()
    cpu = cpu_baseline_decode(torch, rt, dev, state, lens, 32, 8, 128, a.cpu_seconds)
    cpu_wall = time.perf_counter() - t_cpu0
    del state
    torch.cuda.empty_cache()

    line = {
        "metric": "decode-attn HBM GB/s (% of peak) at 32k ctx; prefill attn TFLOP/s",
        "value": round(c2["GB_s"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(c2["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "config 2: Qwen3-8B GQA decode, 32 q / 8 kv heads, head_dim "
                               "128, batch 32, ctx ~ U[1024, 32768] (seeded), f16 KV in "
                               "16-token pages, permuted page table, RoPE theta 1e6",
                   "batch": 32, "ctx_tokens_total": c2["tokens"], "max_ctx": max(lens),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(c2["GB_s"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(c2["hbm_frac"], 4),
                     "traffic": _traffic("decode_kernel_c2",
                                         ["decode_kernel<f16,128,2>", "decode_merge_kernel"])},
        "cpu_baseline": {k: (round(v, 4) if isinstance(v, float) else v)
                         for k, v in cpu.items()},
    }

    if not a.only_headline:
        wl = {}
        # config 2 with every context at 32768 (the "at 32k ctx" reading of the metric)
        r32, st = bench_decode(torch, rt, dev, timer, [32768] * 32, 32, 8, 128, 1e6,
                               0x5EED0011, a.steps, a.warmup)
        del st
        torch.cuda.empty_cache()
        wl["c2_all_32k_decode"] = r32
        pf = bench_prefill(torch, rt, dev, timer, 4096, 32, 8, 128, 1e6, 0x5EED0002, a.steps,
                           a.warmup)
        torch.cuda.empty_cache()
        line["prefill"] = {"workload": "config 3: Qwen3-8B causal prefill, S 4096, 32/8 heads, "
                                       "head_dim 128, bf16 in, f32 softmax/accumulate",
                           "TFLOP_s": round(pf["TFLOP_s"], 2),
                           "roofline": {"bound": "mfma", "achieved": round(pf["TFLOP_s"], 2),
                                        "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                        "frac": round(pf["mfma_frac"], 4)},
                           "ms_per_step": round(pf["ms_per_step"], 4),
                           "tokens_per_s": round(pf["tokens_per_s"], 1)}
        r4, st = bench_decode(torch, rt, dev, timer, [65536] * 8, 16, 2, 256, 1e7, 0x5EED0003,
                              a.steps, a.warmup, sections=[11, 11, 10, 0], rope_dim=64,
                              qk_norm=True, gate=True)
        del st
        torch.cuda.empty_cache()
        wl["c4_gated_decode_64k"] = r4
        r1, st = bench_decode(torch, rt, dev, timer, [513], 32, 32, 128, 1e4, 0x5EED0000,
                              a.steps, a.warmup, pool_dtype=torch.float32)
        del st
        wl["c1_mha_decode_513"] = r1
        wl["c5_gdn_decode_step"] = bench_gdn_decode(torch, rt, dev, timer, a.steps, a.warmup)
        wl["c5_gdn_prefill_4096"] = bench_gdn_prefill(torch, rt, dev, timer, a.steps, a.warmup)
        torch.cuda.empty_cache()
        # TurboQuant compressed-KV decode on the config 2 shape (3-bit + QJL keys, f16 values)
        wl["c2_turboquant_decode"] = bench_tq_decode(torch, rt, dev, timer, lens, 32, 8, 0x5EED0004,
                                                     a.steps, a.warmup)
        wl.update(bench_rows_f(torch, rt, dev, timer, a.steps, a.warmup))
        line["workloads"] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                                 for kk, vv in v.items()} for k, v in wl.items()}
    line["cpu_baseline_wall_s"] = round(cpu_wall, 2)
    print(json.dumps(line), flush=True)
    dev.close()


if __name__ == "__main__":
    main()

"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline (BASELINE.json metric "decode-attn HBM GB/s (% of peak) at 32k ctx;
prefill attn TFLOP/s"): one decode step of config 2 -- Qwen3-8B GQA
(32 q / 8 kv heads, head_dim 128), 32 sequences with context lengths drawn
uniformly from [1024, 32768], f16 KV in 16-token pages under a randomly
permuted page table.  A step is one pi_attn_decode launch over the whole
batch with K/V already resident in HBM.  `value` is algorithmic bytes (K and V
of every cached token once, q, out, page-table entries) per second.

Also reported (same line, "prefill"/"workloads"): config 3 causal prefill
TFLOP/s, the config-4 layer's prefill at head dim 256, the all-32k variant of
config 2, config 4 gated decode, config 1, and the gated-DeltaNet decode step.  Inputs are synthetic N(0,1) generated on
the GPU from fixed seeds; RoPE is applied by the library's own kernel.

Timing: after `warmup` calls and a synchronize, one HIP event pair on the
library's stream brackets `steps` back-to-back calls, followed by a
synchronize; ms_per_step is that interval / steps.  A second pass with an
event pair per call gives the median and minimum.

cpu_baseline: beside every entry, the oracle (a C restatement of the reference's
single-threaded CPU loops) on one pinned core, on a bounded sample of that
entry's own inputs (about --cpu-seconds in total), in the entry's unit.
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
MFMA_F32_PEAK_TFLOPS = 157.3  # dense fp32 MFMA
PAGE = 16


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--cpu-seconds", type=float, default=20.0,
                   help="budget of the single-core CPU baseline sample")
    p.add_argument("--only-headline", action="store_true")
    p.add_argument("--no-graph-replays", action="store_true",
                   help="leave out the layer-token figures replayed from HIP graphs (thousands of "
                        "dispatches: slow under a per-dispatch counter profiler)")
    p.add_argument("--workload", default=None,
                   choices=["c1", "c2", "c2_32k", "c3", "c4", "gdn", "gdn_prefill", "tq", "copy",
                            "rows_f", "chunk", "tq_c4", "c4_prefill"],
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


def _decode_fn(dev, pool, tpt, ctx, q, out, gate=None, torch=None):
    """One pi_attn_decode call; with `torch`, on torch's current stream (as a graph capture
    needs), else on the handle's stream."""
    lib = dev.lib
    args = [dev.h, ctypes.c_void_p(q.data_ptr()), pool.p, ctypes.c_void_p(tpt.data_ptr()),
            tpt.shape[1], ctypes.c_void_p(ctx.data_ptr()), q.shape[0], q.shape[1], 0,
            1.0 / math.sqrt(q.shape[2]),
            None if gate is None else ctypes.c_void_p(gate.data_ptr()),
            ctypes.c_void_p(out.data_ptr()), None]

    def fn():
        if torch is not None:
            args[-1] = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.pi_attn_decode(*args)
        if rc:
            raise RuntimeError(lib.pi_last_error(dev.h).decode())
    return fn


def bench_decode(torch, rt, dev, timer, lens, hq, hkv, d, theta, seed, steps, warmup,
                 cpu_s=0.0, **kw):
    gate_on = kw.pop("gate", False)
    graph = kw.pop("graph", False)
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
    if graph:
        # the same call (decode + merge kernels) replayed from a captured graph of 64 calls:
        # what a serving loop that launches its layers from graphs pays per step
        us = graph_us_per_call(torch, _decode_fn(dev, pool, tpt, ctx, q, out, gate, torch=torch))
        res.update({"us_per_step_graph": us, "GB_s_graph": algo / us / 1e3,
                    "hbm_frac_graph": algo / us / 1e3 / HBM_PEAK_GBS})
    if cpu_s > 0:
        torch.cuda.synchronize()
        qh, oh = q.cpu().numpy(), out.cpu().numpy()
        gh = None if gate is None else gate.cpu().numpy()
        elem = 4 if kw.get("pool_dtype") == torch.float32 else 2

        def load(i):
            ko, vo = pool.read(tpt, i, 0, int(lens[i]))
            torch.cuda.synchronize()
            return ko.cpu().numpy(), vo.cpu().numpy()
        with OneCore():
            res["cpu_baseline"] = cpu_decode(qh, load, lens, hkv, d, elem, cpu_s, oh, gh)
    return res, (pool, tpt, ctx, q, out, gate)


def bench_tq_decode(torch, rt, dev, timer, lens, hq, hkv, seed, steps, warmup, cpu_s=0.0,
                    d=128, gated=False):
    """TurboQuant compressed-KV decode (pi_tq_attn_decode) over a paged cache appended through
    pi_tq_append (K, V ~ N(0,1) generated on the GPU); the timed call includes the per-query
    precompute and the merge (and the sigmoid gate when `gated`)."""
    rng = np.random.default_rng(seed)
    n_pages_seq = [(int(x) + PAGE - 1) // PAGE for x in lens]
    total = sum(n_pages_seq)
    perm = rng.permutation(total).astype(np.int32)
    pt = np.full((len(lens), max(n_pages_seq)), -1, np.int32)
    off = 0
    for i, n in enumerate(n_pages_seq):
        pt[i, :n] = perm[off:off + n]
        off += n
    pool = rt.TqPool(dev, total, hkv, head_dim=d)
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
    gate = torch.randn(q.shape, generator=g, device="cuda") if gated else None
    lib = dev.lib
    args = (dev.h, ctypes.c_void_p(q.data_ptr()), pool.p, ctypes.c_void_p(tpt.data_ptr()),
            tpt.shape[1], ctypes.c_void_p(ctx.data_ptr()), len(lens), hq, 0,
            None if gate is None else ctypes.c_void_p(gate.data_ptr()),
            ctypes.c_void_p(out.data_ptr()), None)

    def fn():
        rc = lib.pi_tq_attn_decode(*args)
        if rc:
            raise RuntimeError(lib.pi_last_error(dev.h).decode())
    t = timer.run(fn, steps, warmup)
    tokens = sum(int(x) for x in lens)
    cpu = None
    if cpu_s > 0:
        cpu = cpu_tq_decode(torch, pool, tpt, q, out, lens, hq, hkv, cpu_s, d, gate)
    # per token and KV head: d/2-byte key record + f32 norm + d f16 values
    rec = d // 2 + 4 + d * 2
    algo = (tokens * hkv * rec + (3 if gated else 2) * len(lens) * hq * d * 4
            + total * 4 + len(lens) * 4 + 2 * hkv * d * d * 4)
    gbs = algo / (t["ms_avg"] * 1e-3) / 1e9
    f16_equiv = tokens * hkv * d * 2 * 2
    res = {"head_dim": d, "GB_s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS, "ms_per_step": t["ms_avg"],
           "ms_median": t["ms_median"], "bytes_per_launch": algo, "tokens": tokens,
           "kv_bytes_vs_f16_pool": round(tokens * hkv * rec / f16_equiv, 4),
           "append_tokens_per_s": tokens / append_s}
    if cpu is not None:
        res["cpu_baseline"] = cpu
    del pool
    return res


def cpu_tq_decode(torch, pool, tpt, q, out, lens, hq, hkv, budget_s, d=128, gate=None):
    """or_tq_cache_attend (the compressed-cache attention of src/turboquant/mod.rs:489-535 with
    the precomputed query) per query head, over the stored records read back from the pool,
    sequence by sequence until the budget is spent (then the gate, :1192-1196)."""
    from oracle import oracle as orc
    torch.cuda.synchronize()
    qh, oh = q.cpu().numpy(), out.cpu().numpy()
    gh = None if gate is None else gate.cpu().numpy()
    mats = [orc.tq_matrices(d, 0xCAFEBABE + h) for h in range(hkv)]
    t = 0.0
    nbytes = toks = done = 0
    err = 0.0
    with OneCore():
        for i, L in enumerate(int(x) for x in lens):
            ko, no, vo = pool.read(tpt, i, 0, L)
            torch.cuda.synchronize()
            kh, nh, vh = ko.cpu().numpy(), no.cpu().numpy(), vo.cpu().numpy()
            t0 = time.perf_counter()
            ref = np.stack([orc.tq_cache_attend(qh[i, h], kh, nh, vh, *mats[h % hkv], h % hkv)
                            for h in range(hq)])
            if gh is not None:
                ref = orc.apply_gate(ref, gh[i])
            t += time.perf_counter() - t0
            nbytes += L * hkv * (d // 2 + 4 + d * 2) + 2 * hq * d * 4
            toks += L
            done += 1
            err = max(err, _row_rel(oh[i], ref))
            if t >= budget_s:
                break
    return _cpu(nbytes / t / 1e9, "GB/s",
                f"or_tq_cache_attend per query head on {done} of {len(lens)} sequences ({toks} "
                f"tokens) of stored records read back from the pool; bytes counted as the GPU "
                f"entry's ({d // 2 + 4 + d * 2} B per token and KV head)", round(t, 3),
                parity_max_row_rel_err=round(err, 6))


# ---- CPU baselines ------------------------------------------------------------
# The oracle (oracle/oracle.c: a C restatement of the reference's single-threaded CPU
# loops, built gcc -O3 -msse4.1) timed on one pinned core on a bounded sample of each
# workload's own inputs, copied back from the GPU outside the timed region.  Each
# figure is in the unit of the GPU entry it sits beside (the workload's algorithmic
# bytes, flops or tokens per second), so the two read side by side.

def cpu_info():
    """Host CPU model (from /proc/cpuinfo) and how many cores this process may use."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "host_cpus": os.cpu_count(),
            "allowed_cpus": len(os.sched_getaffinity(0))}


class OneCore:
    """Pins the process to one core (the lowest it may use) and restores the mask."""

    def __enter__(self):
        self.mask = os.sched_getaffinity(0)
        self.core = min(self.mask)
        os.sched_setaffinity(0, {self.core})
        return self

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.mask)


def _cpu(value, unit, sample, seconds, **extra):
    return {"value": value, "unit": unit, "cores": 1, "kind": "port", "sample": sample,
            "cpu_seconds": seconds, **extra}


def _row_rel(a, b):
    a = np.asarray(a, np.float64).reshape(-1, np.shape(b)[-1])
    b = np.asarray(b, np.float64).reshape(-1, np.shape(b)[-1])
    return float((np.linalg.norm(a - b, axis=1) / np.maximum(np.linalg.norm(b, axis=1), 1e-30)).max())


def cpu_decode(qh, load, lens, hkv, d, elem_bytes, budget_s, out_gpu, gate=None, order=None):
    """or_attn_decode (src/model/mod.rs:1154-1190, + the gate :1192-1196) per sequence until
    the budget is spent; load(i) -> (K, V) f32 [L, Hkv, D] is untimed."""
    from oracle import oracle as orc
    t = 0.0
    nbytes = tokens = calls = 0
    err = 0.0
    order = list(order if order is not None else range(len(lens)))
    kept = {}  # a workload that fits the budget more than once is repeated from memory
    seen = set()
    while t < budget_s:
        for i in order:
            kh, vh = kept[i] if i in kept else load(i)
            if sum(int(lens[j]) for j in order) <= (1 << 20):
                kept[i] = (kh, vh)
            t0 = time.perf_counter()
            ref = orc.attn_decode(qh[i], kh, vh)
            if gate is not None:
                ref = orc.apply_gate(ref, gate[i])
            t += time.perf_counter() - t0
            L = int(lens[i])
            nbytes += L * hkv * d * 2 * elem_bytes + 2 * qh.shape[1] * d * 4
            tokens += L
            calls += 1
            seen.add(i)
            err = max(err, _row_rel(out_gpu[i], ref))
            if t >= budget_s:
                break
    rep_mb = sum(k.nbytes + v.nbytes for k, v in kept.values()) / 1e6
    note = ""
    if calls > len(seen):  # a repeat re-reads its K/V; only a few MB can stay in a CCD's L3
        where = "can stay in the CPU caches" if rep_mb <= 16 else "is re-read from DRAM on each repeat"
        note = f"; the {len(kept)} sequence(s) were repeated from host memory ({rep_mb:.1f} MB, which {where})"
    return _cpu(nbytes / t / 1e9, "GB/s",
                f"or_attn_decode{' + or_apply_gate' if gate is not None else ''} on {len(seen)} "
                f"of {len(lens)} sequences ({calls} calls, {tokens} tokens) read back from the "
                f"pool as f32; bytes counted as the GPU entry's ({elem_bytes}-byte K/V){note}",
                round(t, 3), parity_max_row_rel_err=round(err, 6))


def cpu_prefill(qf, kf, vf, out_gpu, budget_s, stride=97):
    """The reference's prefill: or_attn_decode for row i over keys 0..i (src/model/mod.rs:668
    token loop).  Rows go from the last down in steps of `stride` (mod S), so the sample
    spreads over the triangle; flops per row are 4 * Hq * D * (i + 1)."""
    from oracle import oracle as orc
    s, hq, d = qf.shape
    t = flops = 0.0
    done = 0
    err = 0.0
    i = s - 1
    while done < s:
        t0 = time.perf_counter()
        ref = orc.attn_decode(qf[i], kf[:i + 1], vf[:i + 1])
        t += time.perf_counter() - t0
        flops += 4.0 * hq * d * (i + 1)
        err = max(err, _row_rel(out_gpu[i], ref))
        done += 1
        i = (i - stride) % s
        if t >= budget_s:
            break
    full = 4.0 * hq * d * s * (s + 1) / 2
    return _cpu(flops / t / 1e12, "TFLOP/s",
                f"or_attn_decode rows i = {s - 1}, {s - 1 - stride}, ... (mod {s}): {done} of "
                f"{s} rows, {flops / 1e9:.2f} of {full / 1e9:.1f} GFLOP", round(t, 3),
                full_prompt_s_estimate=round(full / (flops / t), 1),
                parity_max_row_rel_err=round(err, 6))


def cpu_gdn_tokens(q, k, v, beta, g, out_gpu, budget_s, state=None, chunk=32):
    """or_gdn_tokens (src/model/mod.rs:841-916, one token at a time) over the first tokens of
    the workload, `chunk` tokens per call continuing the state, until the budget is spent.
    Returns (figures, tokens done, seconds)."""
    from oracle import oracle as orc
    n_all = q.shape[0]
    st = state
    t = 0.0
    n = 0
    err = 0.0
    while n < n_all:
        m = min(chunk, n_all - n)
        t0 = time.perf_counter()
        o, st = orc.gdn_tokens(q[n:n + m], k[n:n + m], v[n:n + m], beta[n:n + m], g[n:n + m], st)
        t += time.perf_counter() - t0
        err = max(err, float(np.abs(o - out_gpu[n:n + m]).max()))
        n += m
        if t >= budget_s:
            break
    return n, t, err


def bench_prefill(torch, rt, dev, timer, s, hq, hkv, d, theta, seed, steps, warmup, cpu_s=0.0):
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
    res = {"TFLOP_s": tf, "mfma_frac": tf / MFMA_F16_PEAK_TFLOPS, "ms_per_step": t["ms_avg"],
           "flops_per_launch": flops, "tokens_per_s": s / (t["ms_avg"] * 1e-3)}
    if cpu_s > 0:
        torch.cuda.synchronize()
        qf, kf, vf = (x[0].float().cpu().numpy() for x in (qb, kb, vb))
        with OneCore():
            res["cpu_baseline"] = cpu_prefill(qf, kf, vf, out[0].cpu().numpy(), cpu_s)
    return res


def graph_us_per_call(torch, fn, n_calls=64, replays=50):
    """Microseconds per call of `fn` when n_calls of it are captured in one HIP graph and
    the graph is replayed (the launch cost a serving loop with graphs pays per step)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(gr, stream=side):
            for _ in range(n_calls):
                fn()
    torch.cuda.synchronize()
    for _ in range(3):
        gr.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        gr.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (replays * n_calls) * 1e3


def bench_gdn_decode(torch, rt, dev, timer, steps, warmup, cpu_s=0.0, batch=1, graph=True):
    """Config 5 decode step(s): pi_gdn_decode on `batch` sequences (one token each)."""
    hk, hv, dk, dv = 16, 32, 128, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(0x5EED0004)
    q = torch.randn((batch, hk, dk), generator=g, device="cuda")
    k = torch.randn((batch, hk, dk), generator=g, device="cuda")
    v = torch.randn((batch, hv, dv), generator=g, device="cuda")
    beta = torch.sigmoid(torch.randn((batch, hv), generator=g, device="cuda"))
    gg = -torch.nn.functional.softplus(torch.randn((batch, hv), generator=g, device="cuda"))
    state = torch.zeros((batch, hv, dk, dv), device="cuda")
    out = torch.empty((batch, hv, dv), device="cuda")
    lib = dev.lib
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    args = [dev.h, P(q), P(k), P(v), P(beta), P(gg), P(state), P(out), batch, hk, hv, dk, dv,
            None]

    def fn():
        rc = lib.pi_gdn_decode(*args)
        if rc:
            raise RuntimeError(lib.pi_last_error(dev.h).decode())

    t = timer.run(fn, steps, warmup)
    algo = batch * (2 * hv * dk * dv * 4 + (2 * hk * dk + 2 * hv * dv + 2 * hv) * 4)
    gbs = algo / (t["ms_avg"] * 1e-3) / 1e9
    res = {"batch": batch, "us_per_step": t["ms_avg"] * 1e3,
           "tokens_per_s": batch * 1e3 / t["ms_avg"], "GB_s": gbs,
           "hbm_frac": gbs / HBM_PEAK_GBS, "bytes_per_launch": algo}
    if graph:
        # the same step launched from a captured graph of 64 steps, on the capture stream
        args[-1] = ctypes.c_void_p(0)

        def fn_cur():
            args[-1] = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            fn()
        us = graph_us_per_call(torch, fn_cur)
        args[-1] = None
        # the per-launch floor of a graph on this box: torch's fill of one element, replayed the same way
        one = torch.empty(1, device="cuda")
        floor_us = graph_us_per_call(torch, lambda: one.fill_(1.0))
        res.update({"us_per_step_graph": us, "GB_s_graph": algo / us / 1e3,
                    "hbm_frac_graph": algo / us / 1e3 / HBM_PEAK_GBS,
                    "graph_launch_floor_us": floor_us})
    if cpu_s > 0:
        # the timed calls advanced the state: one GPU step from zero for the parity figure
        state.zero_()
        fn()
        torch.cuda.synchronize()
        # sequence 0's token as 256 consecutive steps (the reference's per-token loop); every
        # sequence of a batch costs the reference the same, one after another
        h = [x[:1].cpu().numpy() for x in (q, k, v, beta, gg)]
        o_gpu = out[:1].cpu().numpy()
        reps = 256
        with OneCore():
            n, sec, _ = cpu_gdn_tokens(*[np.repeat(x, reps, axis=0) for x in h],
                                       np.repeat(o_gpu, reps, axis=0), cpu_s)
        from oracle import oracle as orc
        o1, _ = orc.gdn_tokens(*h)
        res["cpu_baseline"] = _cpu(
            n * (algo / batch) / sec / 1e9, "GB/s",
            f"or_gdn_tokens: {n} steps of one sequence from a zero state, per sequence step "
            f"{sec / n * 1e6:.1f} us ({n / sec:.1f} tokens/s); bytes counted as the GPU entry's "
            f"per sequence (state read + write, q, k, v, beta, g, out)", round(sec, 3),
            us_per_step=round(sec / n * 1e6 * batch, 2),
            parity_max_abs_err=float(np.abs(o1 - o_gpu).max()))
    return res


def bench_gdn_prefill(torch, rt, dev, timer, steps, warmup, t=4096, cpu_s=0.0):
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
    res = {"ms_per_step": r["ms_avg"], "tokens_per_s": t / s, "GB_s": algo / s / 1e9,
           "hbm_frac": algo / s / 1e9 / HBM_PEAK_GBS, "TFLOP_s": flops / s / 1e12,
           "bytes_per_launch": algo, "flops_per_launch": flops}
    if cpu_s > 0:
        state.zero_()  # the timed calls advanced the state: one call from zero for parity
        fn()
        torch.cuda.synchronize()
        h = [x.cpu().numpy() for x in (q, k, v, beta, gg)]
        with OneCore():
            n, sec, err = cpu_gdn_tokens(*h, out.cpu().numpy(), cpu_s)
        per_tok = (2 * hk * dk + 2 * hv * dv + 2 * hv) * 4
        res["cpu_baseline"] = _cpu(
            (n * per_tok + 2 * hv * dk * dv * 4) / sec / 1e9, "GB/s",
            f"or_gdn_tokens (the reference's per-token recurrence) over the first {n} of {t} "
            f"tokens from a zero state ({n / sec:.1f} tokens/s); bytes counted as the GPU "
            f"entry's for those tokens", round(sec, 3), tokens_per_s=round(n / sec, 1),
            full_prompt_s_estimate=round(t * sec / n, 1), parity_max_abs_err=err)
    return res


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


def _fp(a, offset=0):
    """float* into a C-contiguous float32 array, `offset` floats in."""
    return ctypes.cast(ctypes.c_void_p(a.ctypes.data + 4 * offset), ctypes.POINTER(ctypes.c_float))


def _nan_max(a, b):
    """max(a, b), except that a NaN on either side gives NaN (and stays NaN after)."""
    return float("nan") if (a != a or b != b) else max(a, b)


def _cpu_repeat(fn, budget_s):
    """Calls fn() until budget_s seconds of it (at least once); returns (seconds, calls)."""
    t, n = 0.0, 0
    while n == 0 or t < budget_s:
        t0 = time.perf_counter()
        fn()
        t += time.perf_counter() - t0
        n += 1
    return t, n


def _cpu_hbm(name, sec, units, unit_bytes, sample, **extra):
    """A CPU figure in the GPU entry's unit (algorithmic bytes per second)."""
    return _cpu(units * unit_bytes / sec / 1e9, "GB/s", sample, round(sec, 3),
                us_per_unit=round(sec / units * 1e6, 3), **extra)


def bench_rows_f(torch, rt, dev, timer, steps, warmup, cpu_s=0.0, graphs=True):
    """The steps either side of the path: the fused attention prologue (row f1:
    per-head RMSNorm, RoPE, paged append in one launch) and the GDN conv1d and
    RMSNormGated (row f2), at a prompt shape (HBM-bound) and a decode step; and row
    f3, one layer of `forward` through the host-slice seam.  With cpu_s > 0 every
    entry also gets the oracle's figure for the same step (cpu_s / 10 seconds each)."""
    from oracle import oracle as orc  # only for the CPU legs
    P = lambda x: None if x is None else ctypes.c_void_p(x.data_ptr())  # noqa: E731
    lib = dev.lib
    res = {}
    g = torch.Generator(device="cuda")
    g.manual_seed(0x5EED00F1)
    leg_s = cpu_s / 10.0
    host = lambda x: None if x is None else x.cpu().numpy()  # noqa: E731

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
        hq_, hk_, wq_, wk_ = host(q), host(k), host(wq), host(wk)  # before the in-place calls
        args = (dev.h, P(q), P(k), P(v), P(wq), P(wk), 1e-6, rope_dim, base, sec, pool.p, P(pt),
                pages, P(sp), n_seq, n_tok, hq, None)
        r = timer.run(_lib_fn(dev, lib.pi_attn_prologue, args), steps, warmup)
        # q and k read and rewritten (f32), v read, k and v appended (f16)
        per_tok = d * (4 * (2 * hq + 3 * hkv) + 2 * 2 * hkv)
        out = _hbm(r, n_seq * n_tok * per_tok)
        pool.close()
        if leg_s > 0:
            freqs = orc.compute_imrope_freqs(base, rope_dim, sections) if sections else None
            chunk = min(n_tok, 256)
            done = [0]

            def step():  # or_attn_prepare (src/model/mod.rs:1035-1138) on the next chunk
                s0 = done[0] % (n_seq * n_tok)
                b, t0 = divmod(s0, n_tok)
                m = min(chunk, n_tok - t0)
                orc.attn_prepare(hq_[b, t0:t0 + m], hk_[b, t0:t0 + m], hq, hkv, d, q_norm_w=wq_,
                                 k_norm_w=wk_, rope_dim=rope_dim, rope_base=base, freqs=freqs,
                                 pos0=start + t0)
                done[0] += m
            with OneCore():
                sec_, _ = _cpu_repeat(step, leg_s)
            out["cpu_baseline"] = _cpu_hbm(
                "prologue", sec_, done[0], per_tok,
                f"or_attn_prepare (norm + RoPE) over {done[0]} tokens in chunks of {chunk}; bytes "
                f"counted as the GPU entry's per token (the reference's append is a Vec copy)")
        return out

    res["f1_prologue_prompt_c3"] = prologue(1, 4096, 32, 8, 128, 128, 1e6, None, False, 0)
    res["f1_prologue_decode_c4"] = prologue(8, 1, 16, 2, 256, 64, 1e7, [11, 11, 10, 0], True,
                                            65535)

    hk, hv, dk, dv, d_conv = 16, 32, 128, 128, 4
    conv_dim = 2 * hk * dk + hv * dv
    w = torch.randn((conv_dim, d_conv), generator=g, device="cuda") * 0.5
    nw = torch.rand((dv,), generator=g, device="cuda") + 0.5
    wh, nwh = host(w), host(nw)
    for name, t in (("prompt_c5", 4096), ("decode_step", 1)):
        x = torch.randn((1, t, conv_dim), generator=g, device="cuda")
        cs = torch.randn((1, d_conv - 1, conv_dim), generator=g, device="cuda")
        xo = torch.empty_like(x)
        xh, csh = host(x), host(cs)
        args = (dev.h, P(x), P(cs), P(w), P(xo), 1, t, conv_dim, d_conv, None)
        r = timer.run(_lib_fn(dev, lib.pi_gdn_conv1d, args), steps, warmup)
        # x read, out written, state read and written, weights read
        per_call = (2 * t * conv_dim + 2 * (d_conv - 1) * conv_dim + conv_dim * d_conv) * 4
        res["f2_gdn_conv1d_" + name] = _hbm(r, per_call)
        if leg_s > 0:
            xa = xh.reshape(t, conv_dim).copy()
            hist = csh.reshape(d_conv - 1, conv_dim).copy()
            c_lib = orc.lib()
            pos = [0]

            def conv_tok():  # or_conv1d_silu (src/model/mod.rs:750-776), one token in place
                c_lib.or_conv1d_silu(_fp(xa, (pos[0] % t) * conv_dim), _fp(hist), _fp(wh),
                                     conv_dim, d_conv)
                pos[0] += 1
            with OneCore():
                sec_, n = _cpu_repeat(conv_tok, leg_s)
            res["f2_gdn_conv1d_" + name]["cpu_baseline"] = _cpu_hbm(
                "conv1d", sec_, n, per_call / t,
                f"or_conv1d_silu over {n} tokens, one call per token as the reference's loop; "
                f"bytes counted as the GPU entry's per token")
        o = torch.randn((t, hv, dv), generator=g, device="cuda")
        z = torch.randn((t, hv, dv), generator=g, device="cuda")
        oh, zh = host(o), host(z)
        args = (dev.h, P(o), P(z), P(nw), t, hv, dv, 1e-6, None)
        r = timer.run(_lib_fn(dev, lib.pi_gdn_rmsnorm_gated, args), steps, warmup)
        per_call = (3 * t * hv * dv + dv) * 4
        res["f2_gdn_rmsnorm_gated_" + name] = _hbm(r, per_call)
        if leg_s > 0:
            oa = oh.copy()
            c_lib = orc.lib()

            def norm_call():  # or_rmsnorm_gated (src/model/mod.rs:918-932) over every row
                c_lib.or_rmsnorm_gated(_fp(oa), _fp(zh), _fp(nwh), t * hv, dv, 1e-6)
            with OneCore():
                sec_, n = _cpu_repeat(norm_call, leg_s)
            res["f2_gdn_rmsnorm_gated_" + name]["cpu_baseline"] = _cpu_hbm(
                "rmsnorm_gated", sec_, n, per_call,
                f"or_rmsnorm_gated over the {t} x {hv} rows, {n} calls; bytes counted as the "
                f"GPU entry's")

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
    qn_w = rng.uniform(0.5, 1.5, d).astype(f32)
    kn_w = rng.uniform(0.5, 1.5, d).astype(f32)
    lay = rt.AttnLayer(dev, prompt + n_dec + 16, hq, hkv, d, torch.float16, q_norm_w=qn_w,
                       k_norm_w=kn_w, rope_dim=64, rope_base=1e7, sections=[11, 11, 10, 0])
    qa, ka, va, ga = (rng.standard_normal((prompt, h, d)).astype(f32)
                      for h in (hq, hkv, hkv, hq))
    q1, k1, v1, g1 = (np.ascontiguousarray(x[:1]) for x in (qa, ka, va, ga))
    raw = [x.copy() for x in (qa, ka, va, ga, q1, k1, v1, g1)]  # the seam rotates q, k in place
    pr, dc = layer_times(lay.reset, lambda: lay.forward(qa, ka, va, ga),
                         lambda: lay.forward(q1, k1, v1, g1))
    res["f3_attn_layer_prompt_1024_c4"] = pr
    res["f3_attn_layer_decode_token_c4"] = dc
    lay.close()
    # the decode token on device tensors (pi_attn_layer_forward_dev: prologue, decode over the
    # prompt's pages and the gate), HIP events over 200 tokens after the 1024-token prompt
    # timer.run (warm-up, the timed pass, the per-call pass), then one call and a capture of 64
    n_tok_dev = 2 * 200 + 20 + 65
    lay = rt.AttnLayer(dev, prompt + n_tok_dev + 16, hq, hkv, d, torch.float16, q_norm_w=qn_w,
                       k_norm_w=kn_w, rope_dim=64, rope_base=1e7, sections=[11, 11, 10, 0])
    dev_t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda")  # noqa: E731
    lay.forward_dev(dev_t(raw[0]), dev_t(raw[1]), dev_t(raw[2]), gate=dev_t(raw[3]))
    qd, kd1, vd1, gd1 = (dev_t(x) for x in raw[4:])
    od = torch.empty((1, hq, d), dtype=torch.float32, device="cuda")
    tok = lambda: lay.forward_dev(qd, kd1, vd1, gate=gd1, out=od)  # noqa: E731
    r = timer.run(tok, 200, 20)
    # back to back from Python the host's per-call cost sets the pace; 64 tokens captured in
    # one HIP graph and replayed give the device time per token (each replay recomputes the
    # captured positions)
    res["f3_attn_layer_decode_token_c4_device"] = {
        "us_per_token": r["ms_avg"] * 1e3, "us_median": r["ms_median"] * 1e3,
        "tokens_per_s": 1e3 / r["ms_avg"]}
    if graphs:
        res["f3_attn_layer_decode_token_c4_device"]["us_per_token_graph"] = graph_us_per_call(torch, tok)
    lay.close()
    if leg_s > 0:
        freqs = orc.compute_imrope_freqs(1e7, 64, [11, 11, 10, 0])
        kw = dict(q_norm_w=qn_w, k_norm_w=kn_w, rope_dim=64, rope_base=1e7, freqs=freqs)
        rq, rk, rv, rg = raw[:4]
        kc = vc = None
        n, t = 0, 0.0
        with OneCore():
            while n < prompt and t < leg_s:  # or_attn_layer_tokens in chunks of 128 tokens
                m = min(128, prompt - n)
                t0 = time.perf_counter()
                _, kc, vc = orc.attn_layer_tokens(rq[n:n + m], rk[n:n + m], rv[n:n + m],
                                                  gate=rg[n:n + m], key_cache=kc, value_cache=vc,
                                                  prev_seq_len=n, **kw)
                t += time.perf_counter() - t0
                n += m
        res["f3_attn_layer_prompt_1024_c4"]["cpu_baseline"] = _cpu(
            n / t, "tokens/s", f"or_attn_layer_tokens (norm, IMRoPE, append, attention over "
            f"every cached key, gate; src/model/mod.rs:1035-1196) over the first {n} of "
            f"{prompt} prompt tokens, 128 per call", round(t, 3))
        # one decode token after those n: the C loop into caches with room for it
        kcap = np.zeros((n + 1, hkv, d), f32)
        vcap = np.zeros((n + 1, hkv, d), f32)
        kcap[:n], vcap[:n] = kc[:n], vc[:n]
        o1 = np.zeros((1, hq, d), f32)
        qx, kx = raw[4].copy(), raw[5].copy()
        fr = np.ascontiguousarray(freqs, f32)
        c_lib = orc.lib()

        def dec_tok():
            qx[:], kx[:] = raw[4], raw[5]
            c_lib.or_attn_layer_tokens(_fp(o1), _fp(qx), _fp(raw[7]), _fp(kx), _fp(raw[6]), 1, hq,
                                       hkv, d, d, d, _fp(qn_w), _fp(kn_w), 1e-6, 64, 1e7, _fp(fr),
                                       fr.size, _fp(kcap), _fp(vcap), n)
        with OneCore():
            sec_, m = _cpu_repeat(dec_tok, leg_s)
        res["f3_attn_layer_decode_token_c4"]["cpu_baseline"] = _cpu(
            m / sec_, "tokens/s", f"or_attn_layer_tokens for one token after {n} cached, {m} "
            f"calls", round(sec_, 3), us_per_token=round(sec_ / m * 1e6, 2))
        res["f3_attn_layer_decode_token_c4_device"]["cpu_baseline"] = dict(
            res["f3_attn_layer_decode_token_c4"]["cpu_baseline"])

    conv_w = (rng.standard_normal((conv_dim, d_conv)) * 0.5).astype(f32)
    ssm_a = -np.exp(rng.standard_normal(hv)).astype(f32)
    dt_b = rng.standard_normal(hv).astype(f32)
    gn_w = rng.uniform(0.5, 1.5, dv).astype(f32)
    gl = rt.GdnLayer(dev, hk, hv, dk, dv, conv_w, ssm_a, dt_b, gn_w)
    xa = rng.standard_normal((prompt, conv_dim)).astype(f32)
    za = rng.standard_normal((prompt, hv, dv)).astype(f32)
    ba, aa = (rng.standard_normal((prompt, hv)).astype(f32) for _ in range(2))
    x1, z1, b1, a1 = (np.ascontiguousarray(x[:1]) for x in (xa, za, ba, aa))
    pr, dc = layer_times(gl.reset, lambda: gl.forward(xa, za, ba, aa),
                         lambda: gl.forward(x1, z1, b1, a1))
    res["f3_gdn_layer_prompt_1024_c5"] = pr
    res["f3_gdn_layer_decode_token_c5"] = dc
    # the same one-token step on device tensors (pi_gdn_layer_forward_dev), HIP events
    dev_t = lambda a: torch.from_numpy(a).to("cuda")  # noqa: E731
    xd, zd, bd, ad = dev_t(x1), dev_t(z1), dev_t(b1), dev_t(a1)
    od = torch.empty((1, hv, dv), dtype=torch.float32, device="cuda")
    gl.reset()
    gl.forward_dev(dev_t(xa), dev_t(za), dev_t(ba), dev_t(aa))  # a prompt's state and conv rows
    gtok = lambda: gl.forward_dev(xd, zd, bd, ad, out=od)  # noqa: E731
    r = timer.run(gtok, 200, 20)
    res["f3_gdn_layer_decode_token_c5_device"] = {
        "us_per_token": r["ms_avg"] * 1e3, "us_median": r["ms_median"] * 1e3,
        "tokens_per_s": 1e3 / r["ms_avg"]}
    if graphs:
        res["f3_gdn_layer_decode_token_c5_device"]["us_per_token_graph"] = graph_us_per_call(torch, gtok)
    gl.close()
    if leg_s > 0:
        kd, vd = hk * dk, hv * dv
        c_lib = orc.lib()

        def gdn_chain(x, z, br, ar, hist, state):
            """src/model/mod.rs:750-932 for x.shape[0] tokens: conv1d + SiLU per token, the
            q / k / v split, gates, the per-token recurrence, RMSNormGated x SiLU(z)."""
            act = x.copy()
            for i in range(act.shape[0]):
                c_lib.or_conv1d_silu(_fp(act, i * conv_dim), _fp(hist), _fp(conv_w), conv_dim,
                                     d_conv)
            m = act.shape[0]
            q = act[:, :kd].reshape(m, hk, dk)
            k = act[:, kd:2 * kd].reshape(m, hk, dk)
            v = act[:, 2 * kd:].reshape(m, hv, dv)
            beta, gg = orc.gdn_gates(br, ar, ssm_a, dt_b)
            o, state = orc.gdn_tokens(q, k, v, beta, gg, state)
            return orc.rmsnorm_gated(o, z, gn_w, 1e-6), state

        hist = np.zeros((d_conv - 1, conv_dim), f32)
        state = None
        n, t = 0, 0.0
        with OneCore():
            while n < prompt and t < leg_s:
                m = min(64, prompt - n)
                t0 = time.perf_counter()
                _, state = gdn_chain(xa[n:n + m], za[n:n + m], ba[n:n + m], aa[n:n + m], hist,
                                     state)
                t += time.perf_counter() - t0
                n += m
            res["f3_gdn_layer_prompt_1024_c5"]["cpu_baseline"] = _cpu(
                n / t, "tokens/s", f"the oracle's GDN layer chain (or_conv1d_silu per token, "
                f"or_gdn_gates, or_gdn_tokens, or_rmsnorm_gated) over the first {n} of {prompt} "
                f"prompt tokens, 64 per call", round(t, 3))
            sec_, m = _cpu_repeat(lambda: gdn_chain(x1, z1, b1, a1, hist.copy(), state), leg_s)
        res["f3_gdn_layer_decode_token_c5"]["cpu_baseline"] = _cpu(
            m / sec_, "tokens/s", f"the oracle's GDN layer chain for one token, {m} calls",
            round(sec_, 3), us_per_token=round(sec_ / m * 1e6, 2))
        res["f3_gdn_layer_decode_token_c5_device"]["cpu_baseline"] = dict(
            res["f3_gdn_layer_decode_token_c5"]["cpu_baseline"])
    return res


def bench_chunk(torch, rt, dev, timer, steps, warmup, cpu_s=0.0):
    """Row f3's continued chunk: a 1024-token chunk of an attention layer (config-4 layer
    shape: 16/2 heads, D 256, q/k RMSNorm, IMRoPE, gate, f16 cache) continuing an 8192-token
    sequence, against a fresh 1024-token prompt.  Timed as device steps (pi_attn_layer_forward_dev,
    HIP events) and through the host-slice seam (wall clock, copies included); plus the
    paged prefill kernel alone on the config-2 heads (gather included)."""
    from oracle import oracle as orc  # only for the CPU leg
    rng = np.random.default_rng(0x5EED0C4)
    f32 = np.float32
    hq, hkv, d, hist, n = 16, 2, 256, 8192, 1024
    qn_w = rng.uniform(0.5, 1.5, d).astype(f32)
    kn_w = rng.uniform(0.5, 1.5, d).astype(f32)
    kw = dict(q_norm_w=qn_w, k_norm_w=kn_w, rope_dim=64, rope_base=1e7, sections=[11, 11, 10, 0])
    lay = rt.AttnLayer(dev, hist + n + 16, hq, hkv, d, torch.float16, **kw)
    g = torch.Generator(device="cuda")
    g.manual_seed(0x5EED0C5)
    rnd = lambda *shape: torch.randn(shape, generator=g, device="cuda")  # noqa: E731
    hq_, hk_, hv_ = rnd(hist, hq, d), rnd(hist, hkv, d), rnd(hist, hkv, d)
    cq, ck, cv, cg = rnd(n, hq, d), rnd(n, hkv, d), rnd(n, hkv, d), rnd(n, hq, d)
    out = torch.empty((n, hq, d), device="cuda")
    res = {}

    def dev_time(prefix):  # GPU time of one chunk step after a prefix of `prefix` tokens
        ts = []
        for rep in range(warmup + steps):
            lay.reset()
            if prefix:
                lay.forward_dev(hq_[:prefix].clone(), hk_[:prefix].clone(), hv_[:prefix])
            q, k = cq.clone(), ck.clone()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            # ~50 us of GPU spin ahead of the start event: the host has enqueued the step's
            # launches before the GPU reaches it, as when layers run back to back, so the
            # figure is the step's device time, not the host's launch latency
            torch.cuda._sleep(100_000)
            a.record()
            lay.forward_dev(q, k, cv, gate=cg, out=out)
            b.record()
            torch.cuda.synchronize()
            if rep >= warmup:
                ts.append(a.elapsed_time(b))
        return float(np.median(ts))
    fresh_ms = dev_time(0)
    chunk_ms = dev_time(hist)
    flops_chunk = 4.0 * hq * d * n * (hist + (n + 1) / 2)
    flops_fresh = 4.0 * hq * d * n * (n + 1) / 2
    res["f3_attn_layer_prompt_1024_c4_device"] = {
        "ms_per_call": fresh_ms, "tokens_per_s": n / fresh_ms * 1e3,
        "attn_TFLOP_s": flops_fresh / fresh_ms / 1e9}
    res["f3_attn_layer_chunk_1024_over_8192_c4_device"] = {
        "ms_per_call": chunk_ms, "tokens_per_s": n / chunk_ms * 1e3,
        "attn_TFLOP_s": flops_chunk / chunk_ms / 1e9, "vs_fresh_prompt": chunk_ms / fresh_ms,
        "flops_vs_fresh_prompt": flops_chunk / flops_fresh}
    # through the host-slice seam (copies of the slices both ways, synchronous)
    hh = [x.cpu().numpy() for x in (hq_, hk_, hv_)]
    ch = [x.cpu().numpy() for x in (cq, ck, cv, cg)]
    walls = {}
    for name, prefix in (("fresh", 0), ("chunk", hist)):
        ts = []
        for rep in range(4):
            lay.reset()
            if prefix:
                lay.forward(hh[0].copy(), hh[1].copy(), hh[2])
            q, k = ch[0].copy(), ch[1].copy()
            t0 = time.perf_counter()
            lay.forward(q, k, ch[2], gate=ch[3])
            if rep >= 1:
                ts.append(time.perf_counter() - t0)
        walls[name] = float(np.median(ts)) * 1e3
    res["f3_attn_layer_chunk_1024_over_8192_c4"] = {
        "ms_per_call": walls["chunk"], "tokens_per_s": n / walls["chunk"] * 1e3,
        "fresh_prompt_ms_per_call": walls["fresh"], "vs_fresh_prompt": walls["chunk"] / walls["fresh"]}
    if cpu_s > 0:
        # the reference's per-token loop (the oracle's C entry on caches allocated once, so no
        # call copies a cache), 4 tokens per call for the first tokens of the chunk over the
        # 8192 history
        c_lib = orc.lib()
        freqs = orc.compute_imrope_freqs(1e7, 64, [11, 11, 10, 0])
        fr = np.ascontiguousarray(freqs, np.float32)
        # the history's cache: K normalised and rotated at 0 .. 8191 (no attention needed)
        _, kc = orc.attn_prepare(None, hh[1], hq, hkv, d, k_norm_w=kn_w, rope_dim=64,
                                 rope_base=1e7, freqs=freqs, pos0=0)
        kcap = np.zeros((hist + n, hkv, d), f32)
        vcap = np.zeros((hist + n, hkv, d), f32)
        kcap[:hist], vcap[:hist] = kc, hh[2]

        def tokens(i0, m_, prev, kc_, vc_):
            qx = np.array(ch[0][i0:i0 + m_], f32)  # normalised / rotated in place
            kx = np.array(ch[1][i0:i0 + m_], f32)
            o = np.empty((m_, hq, d), f32)
            c_lib.or_attn_layer_tokens(_fp(o), _fp(qx), _fp(np.ascontiguousarray(ch[3][i0:i0 + m_])),
                                       _fp(kx), _fp(np.ascontiguousarray(ch[2][i0:i0 + m_])), m_,
                                       hq, hkv, d, d, d, _fp(qn_w), _fp(kn_w), 1e-6, 64, 1e7,
                                       _fp(fr), fr.size, _fp(kc_), _fp(vc_), prev)
        m, t = 0, 0.0
        with OneCore():
            while m < n and t < cpu_s:
                t0 = time.perf_counter()
                tokens(m, 4, hist + m, kcap, vcap)
                t += time.perf_counter() - t0
                m += 4
        cpu = _cpu(m / t, "tokens/s", f"or_attn_layer_tokens for the first {m} tokens of the "
                   f"chunk over the {hist}-token history, 4 per call", round(t, 3))
        res["f3_attn_layer_chunk_1024_over_8192_c4"]["cpu_baseline"] = cpu
        res["f3_attn_layer_chunk_1024_over_8192_c4_device"]["cpu_baseline"] = cpu
        # the fresh prompt: tokens at positions spread evenly over it, each attending its own
        # prefix (the prompt's keys normalised and rotated once, as the cache holds them)
        _, kp = orc.attn_prepare(None, ch[1], hq, hkv, d, k_norm_w=kn_w, rope_dim=64,
                                 rope_base=1e7, freqs=freqs, pos0=0)
        kpc, vpc = np.ascontiguousarray(kp, f32), np.array(ch[2], f32)
        stride = 37
        m, t, i = 0, 0.0, 0
        with OneCore():
            while i < n and t < cpu_s:
                t0 = time.perf_counter()
                tokens(i, 1, i, kpc, vpc)
                t += time.perf_counter() - t0
                m += 1
                i += stride
        res["f3_attn_layer_prompt_1024_c4_device"]["cpu_baseline"] = _cpu(
            m / t, "tokens/s", f"or_attn_layer_tokens for {m} tokens of a fresh {n}-token prompt "
            f"(positions 0, {stride}, {2 * stride}, ...: each attends its own prefix), one per "
            f"call", round(t, 3))
    lay.close()

    # the paged prefill kernel alone: config-2 heads, 1024 queries over 8192 + 1024 keys
    hq, hkv, d = 32, 8, 128
    pages = (hist + n) // 16
    pool = rt.KvPool(dev, pages + 8, hkv, d, torch.float16)
    row = torch.from_numpy(np.random.default_rng(1).permutation(pages + 8)[:pages].astype(np.int32)).cuda()
    k = rnd(hist + n, hkv, d)
    v = rnd(hist + n, hkv, d)
    pool.append(k[None], v[None], row[None].contiguous(), torch.zeros(1, dtype=torch.int32, device="cuda"))
    q16 = rnd(n, hq, d).half()
    o = torch.empty((n, hq, d), device="cuda")
    P = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    args = (dev.h, P(q16), pool.p, P(row), pages, hist, n, hq, 0, 1.0 / math.sqrt(d), P(o), None)
    r = timer.run(_lib_fn(dev, dev.lib.pi_attn_prefill_paged, args), steps, warmup)
    fl = 4.0 * hq * d * n * (hist + (n + 1) / 2)
    tf = fl / (r["ms_avg"] * 1e-3) / 1e12
    res["c2_prefill_paged_1024_over_8192"] = {"TFLOP_s": tf, "mfma_frac": tf / MFMA_F16_PEAK_TFLOPS,
                                              "ms_per_step": r["ms_avg"], "flops_per_launch": fl}
    if cpu_s > 0:
        kf = k.cpu().numpy().astype(np.float16).astype(np.float32)
        vf = v.cpu().numpy().astype(np.float16).astype(np.float32)
        qf = q16.float().cpu().numpy()
        oh = o.cpu().numpy()
        t, fl_done, i, err = 0.0, 0.0, n - 1, 0.0
        with OneCore():
            while i >= 0 and t < cpu_s:
                t0 = time.perf_counter()
                ref = orc.attn_decode(qf[i], kf[:hist + i + 1], vf[:hist + i + 1])
                t += time.perf_counter() - t0
                fl_done += 4.0 * hq * d * (hist + i + 1)
                err = max(err, _row_rel(oh[i], ref))
                i -= 97
        res["c2_prefill_paged_1024_over_8192"]["cpu_baseline"] = _cpu(
            fl_done / t / 1e12, "TFLOP/s", f"or_attn_decode on rows {n - 1}, {n - 98}, ... of the "
            f"chunk over their {hist}+ keys", round(t, 3), parity_max_row_rel_err=round(err, 6))
    pool.close()

    # the f32-cache prefill straight from the pages: config-1 heads (32/32, D 128, f32 cache),
    # 1024 queries over 8192 + 1024 keys, f32-accurate products (bf16 hi / lo splits)
    hq, hkv = 32, 32
    pool = rt.KvPool(dev, pages + 8, hkv, d, torch.float32)
    k = rnd(hist + n, hkv, d)
    v = rnd(hist + n, hkv, d)
    pool.append(k[None], v[None], row[None].contiguous(), torch.zeros(1, dtype=torch.int32, device="cuda"))
    q32 = rnd(n, hq, d)
    o = torch.empty((n, hq, d), device="cuda")
    args = (dev.h, P(q32), pool.p, P(row), pages, hist, n, hq, 0, 1.0 / math.sqrt(d), P(o), None)
    r = timer.run(_lib_fn(dev, dev.lib.pi_attn_prefill_paged, args), steps, warmup)
    fl = 4.0 * hq * d * n * (hist + (n + 1) / 2)
    tf = fl / (r["ms_avg"] * 1e-3) / 1e12
    res["c1_prefill_paged_f32_1024_over_8192"] = {
        "TFLOP_s": tf, "mfma_frac_bf16_peak": tf / MFMA_F16_PEAK_TFLOPS,
        "vs_f32_mfma_peak": tf / MFMA_F32_PEAK_TFLOPS, "ms_per_step": r["ms_avg"],
        "flops_per_launch": fl}
    if cpu_s > 0:
        kf, vf, qf, oh = k.cpu().numpy(), v.cpu().numpy(), q32.cpu().numpy(), o.cpu().numpy()
        t, fl_done, i, err, rows = 0.0, 0.0, n - 1, 0.0, 0
        with OneCore():
            while i >= 0 and t < cpu_s:
                t0 = time.perf_counter()
                ref = orc.attn_decode(qf[i], kf[:hist + i + 1], vf[:hist + i + 1])
                t += time.perf_counter() - t0
                fl_done += 4.0 * hq * d * (hist + i + 1)
                e = float(np.abs(oh[i].astype(np.float64) - ref).max())
                err = _nan_max(err, e)
                rows += 1
                i -= 97
        res["c1_prefill_paged_f32_1024_over_8192"]["cpu_baseline"] = _cpu(
            fl_done / t / 1e12, "TFLOP/s", f"or_attn_decode on {rows} rows ({n - 1}, {n - 98}, ...) "
            f"of the f32 chunk over their {hist}+ keys", round(t, 3),
            parity_max_abs_err=float(f"{err:.3e}"), gpu_out_finite=bool(np.isfinite(oh).all()))
    pool.close()
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
    # table rows: kernel, workgroups, FETCH_KiB, WRITE_KiB, read_B(cal), write_B(cal)[, algo, ratio]
    total, seen, in_table = 0, set(), False
    for line in open(p):
        f = line.split()
        if f[:4] == ["kernel", "wgs", "FETCH_KiB", "WRITE_KiB"]:
            in_table = True
            continue
        if in_table and len(f) >= 6 and f[0] in kernels and f[0] not in seen:
            total += int(float(f[4])) + int(float(f[5]))
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
                            pool_dtype=torch.float32, graph=True)[0]
    if w == "c3":
        return bench_prefill(torch, rt, dev, timer, 4096, 32, 8, 128, 1e6, 0x5EED0002, st, wu)
    if w == "c4_prefill":  # a 4096-token prompt of the config-4 layer (16/2 heads, D 256)
        return bench_prefill(torch, rt, dev, timer, 4096, 16, 2, 256, 1e7, 0x5EED0007, st, wu)
    if w == "gdn_prefill":
        return bench_gdn_prefill(torch, rt, dev, timer, st, wu)
    if w == "tq":
        rng = np.random.default_rng(0x5EED0001)
        lens = [int(x) for x in rng.integers(1024, 32769, size=32)]
        return bench_tq_decode(torch, rt, dev, timer, lens, 32, 8, 0x5EED0004, st, wu)
    if w == "tq_c4":
        return bench_tq_decode(torch, rt, dev, timer, [65536] * 8, 16, 2, 0x5EED0014, st, wu,
                               d=256, gated=True)
    if w == "copy":
        return bench_copy(torch, timer, st, wu)
    if w == "rows_f":
        return bench_rows_f(torch, rt, dev, timer, st, wu, graphs=not a.no_graph_replays)
    if w == "chunk":
        return bench_chunk(torch, rt, dev, timer, st, wu)
    return bench_gdn_decode(torch, rt, dev, timer, st, wu)


def _round_num(v):
    # 4 decimals, but 3 significant digits below 0.01 so small errors do not print as 0
    return round(v, 4) if v == 0 or abs(v) >= 1e-2 or v != v else float(f"{v:.3g}")


def _rounded(d):
    return {k: (_round_num(v) if isinstance(v, float) else _rounded(v) if isinstance(v, dict) else v)
            for k, v in d.items()}


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

    # CPU baseline budget (seconds of single-core oracle work) per workload
    cs = a.cpu_seconds
    share = {"c2": 0.25, "c2_32k": 0.04, "c3": 0.15, "c4": 0.1, "c1": 0.03, "gdn_dec": 0.04,
             "gdn_pre": 0.1, "tq": 0.07, "rows_f": 0.2, "chunk": 0.04, "c4_pre": 0.05}
    budget = {k: v * cs for k, v in share.items()}
    t_all0 = time.perf_counter()

    # ---- headline: config 2 decode ----
    rng = np.random.default_rng(0x5EED0001)
    lens = [int(x) for x in rng.integers(1024, 32769, size=32)]
    c2, state = bench_decode(torch, rt, dev, timer, lens, 32, 8, 128, 1e6, 0x5EED0001, a.steps,
                             a.warmup, cpu_s=budget["c2"])
    cpu = c2.pop("cpu_baseline")
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
                                         ["decode_kernel<f16,128,2>", "decode_merge_kernel<4>"])},
        "cpu_baseline": {**{k: (round(v, 4) if isinstance(v, float) else v)
                            for k, v in cpu.items()}, **cpu_info(),
                         "pinned": "os.sched_setaffinity to one core for the oracle calls"},
    }

    if not a.only_headline:
        wl = {}
        # config 2 with every context at 32768 (the "at 32k ctx" reading of the metric)
        r32, st = bench_decode(torch, rt, dev, timer, [32768] * 32, 32, 8, 128, 1e6,
                               0x5EED0011, a.steps, a.warmup, cpu_s=budget["c2_32k"])
        del st
        torch.cuda.empty_cache()
        wl["c2_all_32k_decode"] = r32
        pf = bench_prefill(torch, rt, dev, timer, 4096, 32, 8, 128, 1e6, 0x5EED0002, a.steps,
                           a.warmup, cpu_s=budget["c3"])
        torch.cuda.empty_cache()
        line["prefill"] = {"workload": "config 3: Qwen3-8B causal prefill, S 4096, 32/8 heads, "
                                       "head_dim 128, bf16 in, f32 softmax/accumulate",
                           "TFLOP_s": round(pf["TFLOP_s"], 2),
                           "roofline": {"bound": "mfma", "achieved": round(pf["TFLOP_s"], 2),
                                        "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                        "frac": round(pf["mfma_frac"], 4)},
                           "ms_per_step": round(pf["ms_per_step"], 4),
                           "tokens_per_s": round(pf["tokens_per_s"], 1),
                           "cpu_baseline": pf["cpu_baseline"]}
        # the config-4 attention layer's prompt: causal prefill at head dim 256, S 4096, 16/2 heads
        wl["c4_layer_prefill_4096_d256"] = bench_prefill(torch, rt, dev, timer, 4096, 16, 2, 256, 1e7,
                                                         0x5EED0007, a.steps, a.warmup,
                                                         cpu_s=budget["c4_pre"])
        torch.cuda.empty_cache()
        r4, st = bench_decode(torch, rt, dev, timer, [65536] * 8, 16, 2, 256, 1e7, 0x5EED0003,
                              a.steps, a.warmup, sections=[11, 11, 10, 0], rope_dim=64,
                              qk_norm=True, gate=True, cpu_s=budget["c4"])
        del st
        torch.cuda.empty_cache()
        wl["c4_gated_decode_64k"] = r4
        r1, st = bench_decode(torch, rt, dev, timer, [513], 32, 32, 128, 1e4, 0x5EED0000,
                              a.steps, a.warmup, pool_dtype=torch.float32, cpu_s=budget["c1"],
                              graph=True)
        del st
        wl["c1_mha_decode_513"] = r1
        wl["c5_gdn_decode_step"] = bench_gdn_decode(torch, rt, dev, timer, a.steps, a.warmup,
                                                    cpu_s=budget["gdn_dec"])
        # 32 sequences per step: the state stream of a serving batch
        wl["c5_gdn_decode_step_batch32"] = bench_gdn_decode(torch, rt, dev, timer, a.steps,
                                                            a.warmup, batch=32, graph=False,
                                                            cpu_s=budget["gdn_dec"] / 2)
        wl["c5_gdn_prefill_4096"] = bench_gdn_prefill(torch, rt, dev, timer, a.steps, a.warmup,
                                                      cpu_s=budget["gdn_pre"])
        torch.cuda.empty_cache()
        # TurboQuant compressed-KV decode on the config 2 shape (3-bit + QJL keys, f16 values)
        wl["c2_turboquant_decode"] = bench_tq_decode(torch, rt, dev, timer, lens, 32, 8, 0x5EED0004,
                                                     a.steps, a.warmup, cpu_s=budget["tq"] / 2)
        torch.cuda.empty_cache()
        # TurboQuant on config 4's attention layer shape: 16/2 heads, D 256, gated, 8 x 65536
        wl["c4_turboquant_decode_64k"] = bench_tq_decode(torch, rt, dev, timer, [65536] * 8, 16, 2,
                                                         0x5EED0014, a.steps, a.warmup,
                                                         cpu_s=budget["tq"] / 2, d=256, gated=True)
        torch.cuda.empty_cache()
        wl.update(bench_rows_f(torch, rt, dev, timer, a.steps, a.warmup,
                               cpu_s=budget["rows_f"], graphs=not a.no_graph_replays))
        wl.update(bench_chunk(torch, rt, dev, timer, min(a.steps, 10), min(a.warmup, 3),
                              cpu_s=budget["chunk"]))
        line["workloads"] = {k: _rounded(v) for k, v in wl.items()}
        line["prefill"] = _rounded(line["prefill"])
    line["bench_wall_s"] = round(time.perf_counter() - t_all0, 2)
    print(json.dumps(line), flush=True)
    dev.close()


if __name__ == "__main__":
    main()

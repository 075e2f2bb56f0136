"""Library calls captured in a HIP graph and replayed, against the same calls run eagerly.

A serving loop captures its decode step once and replays it; the calls it captures must not
allocate or synchronise (pi_gdn_decode, pi_attn_decode_noalloc).  Each graph is replayed
several times with eager work and synchronisations in between, and every replay is compared
with the eager result bit for bit (same kernels, same launch shapes).
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from tests.gpu_util import PagedCase, device, to_dev

pytestmark = pytest.mark.gpu


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(gr, stream=side):
            fn()
    torch.cuda.synchronize()
    return gr


def test_gdn_decode_steps_graph_replay():
    """8 consecutive decode steps (config-5 heads) captured once; each replay from a reset
    state equals the eager steps."""
    dev = device()
    hk, hv, dk, dv, n = 16, 32, 128, 128, 8
    rng = np.random.default_rng(0x6A1)
    q = to_dev(rng.standard_normal((n, 1, hk, dk)).astype(np.float32))
    k = to_dev(rng.standard_normal((n, 1, hk, dk)).astype(np.float32))
    v = to_dev(rng.standard_normal((n, 1, hv, dv)).astype(np.float32))
    beta = to_dev((1 / (1 + np.exp(-rng.standard_normal((n, 1, hv))))).astype(np.float32))
    g = to_dev((-np.log1p(np.exp(rng.standard_normal((n, 1, hv))))).astype(np.float32))
    s0 = to_dev(rng.standard_normal((1, hv, dk, dv)).astype(np.float32) * 0.1)
    state = torch.empty_like(s0)
    out = torch.empty((n, 1, hv, dv), device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def steps():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for i in range(n):
            rc = dev.lib.pi_gdn_decode(dev.h, P(q[i]), P(k[i]), P(v[i]), P(beta[i]), P(g[i]),
                                       P(state), P(out[i]), 1, hk, hv, dk, dv, st)
            assert rc == 0

    state.copy_(s0)
    steps()
    torch.cuda.synchronize()
    ref_out, ref_state = out.clone(), state.clone()
    state.copy_(s0)
    gr = _capture(steps)
    for rep in range(3):
        state.copy_(s0)   # eager work between replays
        out.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), f"replay {rep}: outputs differ"
        assert torch.equal(state, ref_state), f"replay {rep}: states differ"


def test_decode_noalloc_graph_replay():
    """pi_attn_decode_noalloc (config-2 heads, f16 pages, ragged batch) captured once; each
    replay equals eager pi_attn_decode, with a different eager decode run in between."""
    dev = device()
    rng = np.random.default_rng(0x6A2)
    lens = [int(x) for x in rng.integers(1, 6000, size=10)]
    case = PagedCase(rng, lens, 32, 8, 128, theta=1e6)
    case.gpu_build(dev, torch.float16)
    q = case.gpu_q(dev)
    ctx = to_dev(np.array(lens, np.int32))
    out = torch.zeros_like(q)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    scale = 1.0 / math.sqrt(128)

    def call(entry, o, c):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = getattr(dev.lib, entry)(dev.h, P(q), case.pool.p, P(case.pt), case.pt.shape[1],
                                     P(c), q.shape[0], 32, 0, scale, None, P(o), st)
        assert rc == 0, dev.lib.pi_last_error(dev.h)

    ref = torch.empty_like(q)
    call("pi_attn_decode", ref, ctx)
    torch.cuda.synchronize()
    gr = _capture(lambda: call("pi_attn_decode_noalloc", out, ctx))
    other = torch.empty_like(q)
    short = to_dev(np.minimum(np.array(lens, np.int32), 17))
    for rep in range(3):
        out.zero_()
        call("pi_attn_decode_noalloc", other, short)  # eager use of the same scratch between
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}: outputs differ"

"""TurboQuant at head widths without an MFMA tile (head_dim 1..256 but 128 and 256;
src/turboquant/mod.rs:430-437 takes any head_dim, and its own cache test uses 16).

These widths run the in-order kernels: the key records are the reference's bit stream
(3-bit codes, then the QJL signs, ceil(4 d / 8) bytes) and must equal the oracle's byte
for byte; the decode follows attention_scores, the softmax and weighted_value_sum in the
reference's order, skipping weights below 1e-7 (:519-536), so its rows match
or_tq_cache_attend to 2e-5 relative (the device's expf and the parallel sums of the
softmax are the only differences), and a token whose weight is below 1e-7 contributes
exactly nothing.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as o
from powerinfer_x64_amd import runtime as rt
from tests.gpu_util import device, row_rel_err, to_dev
from tests.test_gpu_turboquant import TqCase, _check_records

pytestmark = pytest.mark.gpu


def test_reference_cache_test_shape():
    """test_compressed_kv_cache (src/turboquant/mod.rs:868-893): 2 KV heads of 16 dims, 10
    tokens of sin / cos data, the query sin(0.1 i): records and the attention output of every
    query head against the oracle."""
    dev = device()
    n_kv, d, n = 2, 16, 10
    case = TqCase(np.random.default_rng(0), [n], n_kv, d=d)
    case.k = [np.array([[[math.sin((t * 100 + h * d + i) * 0.01) for i in range(d)]
                         for h in range(n_kv)] for t in range(n)], np.float32)]
    case.v = [np.array([[[math.cos((t * 100 + h * d + i) * 0.02) for i in range(d)]
                         for h in range(n_kv)] for t in range(n)], np.float32)]
    case.build(dev)
    _check_records(case, 0)
    q1 = np.array([math.sin(i * 0.1) for i in range(d)], np.float32)
    q = np.stack([q1, 2 * q1])[None]  # two query heads, one per KV head (modulo map)
    out = rt.tq_attn_decode(dev, to_dev(q), case.pool, case.pt_d,
                            to_dev(np.array([n], np.int32))).cpu().numpy()
    ref = case.oracle_out(0, q[0])
    assert row_rel_err(out[0], ref) <= 2e-5


@pytest.mark.parametrize("d,hq,hkv,gqa_mode", [(16, 4, 2, 0), (33, 3, 3, 0), (64, 8, 2, 1),
                                               (96, 6, 2, 0), (200, 4, 1, 1)])
def test_any_width_records_and_decode(d, hq, hkv, gqa_mode):
    """Ragged contexts (an empty one among them) appended in chunks into permuted pages, a
    sigmoid gate, both head maps."""
    dev = device()
    rng = np.random.default_rng(0x7D00 + d)
    lens = [1, 37, 300, 0, 129]
    case = TqCase(rng, lens, hkv, d=d)
    case.build(dev, chunk=23)
    for i in range(len(lens)):
        if lens[i]:
            _check_records(case, i)
    q = rng.standard_normal((len(lens), hq, d)).astype(np.float32) * 2
    gate = rng.standard_normal((len(lens), hq, d)).astype(np.float32)
    out = rt.tq_attn_decode(dev, to_dev(q), case.pool, case.pt_d, to_dev(np.array(lens, np.int32)),
                            gqa_mode=gqa_mode, gate=to_dev(gate)).cpu().numpy()
    assert np.all(out[3] == 0.0)
    for i in range(len(lens)):
        if lens[i]:
            err = row_rel_err(out[i], case.oracle_out(i, q[i], gqa_mode, gate[i]))
            assert err <= 2e-5, f"seq {i} (L={lens[i]}): rel err {err}"


def test_weights_below_1e7_are_skipped():
    """One-hot values (token t's value is e_t) make the output the weight vector with the
    skipped weights zeroed.  A large query spreads the softmax so that several weights lie
    between 1e-10 and 5e-8 (float64 from the oracle's own dot): those come out exactly 0,
    as in the reference, and every other weight matches the oracle."""
    dev = device()
    rng = np.random.default_rng(0x7D01)
    d, n = 64, 48
    case = TqCase(rng, [n], 1, d=d)
    case.v = [np.zeros((n, 1, d), np.float32)]
    for t in range(n):
        case.v[0][t, 0, t] = 1.0
    case.build(dev)
    q = (rng.standard_normal((1, 1, d)) * 14).astype(np.float32)
    out = rt.tq_attn_decode(dev, to_dev(q), case.pool, case.pt_d,
                            to_dev(np.array([n], np.int32))).cpu().numpy()[0, 0]
    packed, norms, _ = case.oracle_cache(0)
    s = np.array([norms[t, 0] * o.tq_dot(q[0, 0], packed[t, 0], case.R[0], case.G[0], 3, d)
                  for t in range(n)], np.float64) / math.sqrt(d)
    w = np.exp(s - s.max())
    w /= w.sum()
    small = np.flatnonzero((w > 1e-10) & (w < 5e-8))
    assert small.size >= 3, f"only {small.size} weights in (1e-10, 5e-8): {np.sort(w)[:8]}"
    assert np.all(out[small] == 0.0)
    ref = case.oracle_out(0, q[0])[0]
    assert np.all(ref[small] == 0.0)
    big = w >= 1e-6
    assert np.allclose(out[:n][big], ref[:n][big], rtol=2e-5, atol=0)
    assert np.all(out[n:] == 0.0)


def test_any_width_pages_outside_the_pool_hold_no_tokens():
    """A page id outside [0, n_pages) in a sequence's table holds no tokens (as in the
    decode of the other pools): its keys leave the softmax, the rest match the oracle over
    the keys that remain."""
    dev = device()
    rng = np.random.default_rng(0x7D02)
    d, hq, hkv = 48, 4, 2
    case = TqCase(rng, [80], hkv, d=d)
    case.build(dev)
    pt = case.pt.copy()
    pt[0, 2] = case.n_pages + 5  # tokens 32 .. 47
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    out = rt.tq_attn_decode(dev, to_dev(q), case.pool, to_dev(pt),
                            to_dev(np.array([80], np.int32))).cpu().numpy()[0]
    packed, norms, vals = case.oracle_cache(0)
    keep = np.r_[0:32, 48:80]
    for h in range(hq):
        kvh = h % hkv
        ref = o.tq_cache_attend(q[0, h], packed[keep], norms[keep], vals[keep], case.R[kvh],
                                case.G[kvh], kvh)
        assert row_rel_err(out[h], ref) <= 2e-5, h


@pytest.mark.parametrize("d", [0, 257])
def test_width_outside_range_raises(d):
    dev = device()
    with pytest.raises(rt.Unsupported):
        rt.TqPool(dev, 4, 2, head_dim=d)

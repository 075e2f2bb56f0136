"""Decode attention on the GPU vs the CPU oracle (src/model/mod.rs:1035-1196).

Tolerances: max-abs <= 2e-3 for the f32 cache;
<= 1e-2 relative (per head row, ||d||_2/||ref||_2) for the f16 cache; exact
argmax of synthetic logits (ties within the error bound are reported, not
failed).
"""
import math

import numpy as np
import pytest
import torch

from tests import ref64
from tests.gpu_util import PagedCase, argmax_agreement, device, row_rel_err, to_dev

pytestmark = pytest.mark.gpu


def _check_f16(case, out, gate=None, tol=1e-2):
    for i in range(len(case.lens)):
        ref = case.oracle_out(i, kv_round=np.float16, gate=None if gate is None else gate[i])
        err = row_rel_err(out[i], ref)
        assert err <= tol, f"seq {i} (L={case.lens[i]}): rel err {err}"
    refs = np.stack([case.oracle_out(i, kv_round=np.float16,
                                     gate=None if gate is None else gate[i])
                     for i in range(len(case.lens))])
    n, mism, ties = argmax_agreement(out, refs)
    assert mism == 0, f"argmax mismatch on {mism}/{n} rows ({ties} ties)"


def test_c1_llama2_mha_f32_cache():
    """Config 1: 32/32 heads, D 128, 512 cached + the query token, theta 1e4, f32 KV."""
    dev = device()
    rng = np.random.default_rng(0x5EED0000)
    case = PagedCase(rng, [513], 32, 32, 128, theta=1e4)
    case.gpu_build(dev, torch.float32)
    out = case.gpu_decode(dev)
    ref = case.oracle_out(0)
    err = np.abs(out[0] - ref).max()
    assert err <= 2e-3, f"max-abs {err}"
    n, mism, ties = argmax_agreement(out, ref[None])
    assert mism == 0


@pytest.mark.parametrize("seed", [1, 2])
def test_c2_qwen3_gqa_f16_paged_ragged(seed):
    """Config 2 at reduced batch: 32/8 heads (modulo GQA), D 128, theta 1e6, f16 pages."""
    dev = device()
    rng = np.random.default_rng(0x5EED0001 + seed)
    lens = rng.integers(1, 3000, size=6)
    lens[0] = 1
    lens[1] = 16 * 37  # exact page multiple
    case = PagedCase(rng, lens, 32, 8, 128, theta=1e6)
    case.gpu_build(dev, torch.float16)
    out = case.gpu_decode(dev)
    _check_f16(case, out)


def test_c2_full_lengths_sampled():
    """Config 2 lengths up to 32768 (4 sequences incl. the 32k maximum)."""
    dev = device()
    rng = np.random.default_rng(0x5EED0001)
    lens = [32768, 1024, int(rng.integers(1024, 32768)), 16383]
    case = PagedCase(rng, lens, 32, 8, 128, theta=1e6)
    case.gpu_build(dev, torch.float16)
    out = case.gpu_decode(dev)
    _check_f16(case, out)


def test_decode_repeatable_bitwise():
    """Two launches give identical bits (split merge order and counters reset)."""
    dev = device()
    rng = np.random.default_rng(7)
    case = PagedCase(rng, [5000, 77, 4096], 32, 8, 128)
    case.gpu_build(dev, torch.float16)
    a = case.gpu_decode(dev)
    b = case.gpu_decode(dev)
    np.testing.assert_array_equal(a, b)


def test_decode_single_key_is_v_and_empty_is_zero():
    dev = device()
    rng = np.random.default_rng(8)
    case = PagedCase(rng, [1, 0, 2], 8, 8, 64, theta=1e4)
    case.gpu_build(dev, torch.float32)
    out = case.gpu_decode(dev)
    np.testing.assert_allclose(out[0], case.v[0][0][np.arange(8) % 8], rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(out[1], 0)
    ref = case.oracle_out(2)
    assert np.abs(out[2] - ref).max() <= 2e-3


@pytest.mark.parametrize("hq,hkv,d", [(16, 2, 256), (8, 1, 128), (4, 4, 64), (16, 1, 128)])
def test_decode_shapes_f16(hq, hkv, d):
    dev = device()
    rng = np.random.default_rng(hq * 1000 + hkv * 10 + d)
    case = PagedCase(rng, [1500, 33, 4097], hq, hkv, d)
    case.gpu_build(dev, torch.float16)
    out = case.gpu_decode(dev)
    _check_f16(case, out)


def test_decode_f32_cache_long():
    dev = device()
    rng = np.random.default_rng(11)
    case = PagedCase(rng, [9000, 640], 32, 8, 128, theta=1e6)
    case.gpu_build(dev, torch.float32)
    out = case.gpu_decode(dev)
    for i in range(2):
        assert np.abs(out[i] - case.oracle_out(i)).max() <= 2e-3


def test_c4_gated_qknorm_imrope_decode():
    """Config 4 at reduced batch/length: 16/2 heads, D 256, Q/K RMSNorm, IMRoPE over
    the first 64 dims (theta 1e7, sections [11,11,10,0]), sigmoid gate."""
    dev = device()
    rng = np.random.default_rng(0x5EED0003)
    d = 256
    qn = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, d).astype(np.float32)
    case = PagedCase(rng, [6000, 65], 16, 2, d, theta=1e7, rope_dim=64,
                     sections=[11, 11, 10, 0], q_norm_w=qn, k_norm_w=kn)
    gate = rng.standard_normal((2, 16, d)).astype(np.float32)
    case.gpu_build(dev, torch.float16)
    out = case.gpu_decode(dev, gate=gate)
    _check_f16(case, out, gate=gate)


def test_decode_grouped_mode_f64():
    """PI_GQA_GROUPED (not the reference mapping) against float64 brute force."""
    dev = device()
    rng = np.random.default_rng(12)
    case = PagedCase(rng, [700, 1200], 32, 8, 128)
    case.gpu_build(dev, torch.float16)
    out = case.gpu_decode(dev, gqa_mode=1)
    for i in range(2):
        kc, vc = case.oracle_caches(i, kv_round=np.float16)
        ref = ref64.attention(case.oracle_q(i), kc, vc, lambda h: h // 4)
        assert row_rel_err(out[i], ref) <= 1e-2


def test_attention_head_host_dropin():
    """ops::attention_head (src/ops.rs:213-247) with host slices, KAT input of ops.rs:340-357."""
    from powerinfer_x64_amd import runtime as rt
    from oracle import oracle as orc
    dev = device()
    rng = np.random.default_rng(13)
    d, t = 128, 300
    q = rng.standard_normal(d).astype(np.float32)
    k = rng.standard_normal((t, d)).astype(np.float32)
    v = rng.standard_normal((t, d)).astype(np.float32)
    out = rt.attention_head(dev, q, k, v, t, d)
    assert np.abs(out - orc.attention_head(q, k, v, t, d)).max() <= 2e-3
    # KAT of src/ops.rs:340-357 padded to head_dim 64 (zeros do not change scores)
    q4 = np.zeros(64, np.float32)
    q4[0] = 1
    k3 = np.zeros((3, 64), np.float32)
    v3 = np.zeros((3, 64), np.float32)
    for i in range(3):
        k3[i, i] = 1
        v3[i, i] = 10 * (i + 1)
    out = rt.attention_head(dev, q4 * math.sqrt(64 / 4), k3, v3, 3, 64)
    np.testing.assert_allclose(out[:4], [4.51863, 5.48137, 8.22206, 0], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("grid", [None, "1", "7", "1000"])
def test_decode_balanced_schedule_edges(grid, monkeypatch):
    """Ragged batch with empty sequences in between, under several persistent-grid
    sizes (PI_DECODE_GRID): runs split a segment across many workgroups."""
    if grid is not None:
        monkeypatch.setenv("PI_DECODE_GRID", grid)
    dev = device()
    rng = np.random.default_rng(31)
    lens = [0, 5, 0, 0, 3000, 1, 0, 257, 4096, 16, 17]
    case = PagedCase(rng, lens, 8, 2, 128, theta=1e6)
    case.gpu_build(dev, torch.float16)
    out = case.gpu_decode(dev)
    for i, x in enumerate(lens):
        if x == 0:
            np.testing.assert_array_equal(out[i], 0)
        else:
            ref = case.oracle_out(i, kv_round=np.float16)
            assert row_rel_err(out[i], ref) <= 1e-2, (grid, i, x)


def test_decode_large_batch_scan():
    """More sequences than threads in a workgroup (multi-chunk prefix scan)."""
    dev = device()
    rng = np.random.default_rng(32)
    lens = rng.integers(0, 200, size=300)
    case = PagedCase(rng, lens, 4, 1, 64, theta=1e4)
    case.gpu_build(dev, torch.float16)
    out = case.gpu_decode(dev)
    for i in list(range(0, 300, 13)) + [299]:
        if lens[i] == 0:
            np.testing.assert_array_equal(out[i], 0)
        else:
            assert row_rel_err(out[i], case.oracle_out(i, kv_round=np.float16)) <= 1e-2


@pytest.mark.parametrize("pool_dtype,d,hq,hkv,length", [
    (torch.float32, 128, 8, 2, 1024),   # 4 heads a segment (cols * D = 512), 64 pages
    (torch.float32, 64, 4, 1, 1000),
    (torch.float16, 64, 16, 2, 17),     # 8 heads a segment at D 64
    (torch.float16, 128, 4, 4, 1),
    (torch.float16, 128, 32, 8, 700),
    (torch.float32, 128, 32, 32, 0),    # no tokens: zeros (written by the merge)
])
def test_one_sequence_short_contexts(pool_dtype, d, hq, hkv, length):
    """One sequence of at most 64 pages (a decode token stream): the split schedule spreads a
    few pages per workgroup and the merge folds them; every output row against the oracle
    (f32: max-abs 2e-3; f16: 1e-2 rel); the output starts as NaN."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(0x5EED0900 + d + hq + length)
    case = PagedCase(rng, [length], hq, hkv, d, theta=1e6)
    case.gpu_build(dev, pool_dtype)
    q = case.gpu_q(dev)
    out = torch.full_like(q, float("nan"))
    rt.attn_decode(dev, q, case.pool, case.pt, to_dev(np.array([length], np.int32)), out=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    if pool_dtype == torch.float32:
        ref = case.oracle_out(0)
        err = np.abs(got[0] - ref).max()
        assert err <= 2e-3, f"max-abs {err}"
    else:
        _check_f16(case, got)

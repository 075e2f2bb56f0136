"""Causal prefill attention on the GPU vs the CPU oracle.

The reference's prefill runs the decode attention once per prompt token with
append-then-attend (src/model/mod.rs:668,1140-1190), so row i of the oracle
is or_attn_decode over keys 0..i.  Inputs follow config 3: q/k/v drawn in f32,
RoPE (theta 1e6, adjacent pairs) applied in f32 by the oracle on the host,
then rounded to bf16 -- the kernel's input; the oracle reads the same bf16
values upcast.  Tolerance: <= 1e-2 relative per row (bf16 class), exact
argmax of synthetic logits.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests import ref64
from tests.gpu_util import argmax_agreement, device, row_rel_err

pytestmark = pytest.mark.gpu


def _inputs(rng, s, hq, hkv, d, theta=1e6, dtype=torch.bfloat16):
    q = rng.standard_normal((s, hq, d)).astype(np.float32)
    k = rng.standard_normal((s, hkv, d)).astype(np.float32)
    v = rng.standard_normal((s, hkv, d)).astype(np.float32)
    qr, kr = orc.attn_prepare(q, k, hq, hkv, d, rope_base=theta, pos0=0)
    tq = torch.from_numpy(qr).to(dtype)
    tk = torch.from_numpy(kr).to(dtype)
    tv = torch.from_numpy(v).to(dtype)
    return tq, tk, tv


def _oracle_rows(tq, tk, tv, rows):
    qf, kf, vf = (t.float().numpy() for t in (tq, tk, tv))
    return np.stack([orc.attn_decode(qf[i], kf[:i + 1], vf[:i + 1]) for i in rows])


def _run(tq, tk, tv, causal=True, gqa_mode=0):
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    out = rt.attn_prefill(dev, tq[None].cuda(), tk[None].cuda(), tv[None].cuda(), causal=causal,
                          gqa_mode=gqa_mode)
    torch.cuda.synchronize()
    return out[0].cpu().numpy()


@pytest.mark.parametrize("s", [1, 31, 64, 200, 513])
def test_prefill_small_all_rows(s):
    rng = np.random.default_rng(100 + s)
    tq, tk, tv = _inputs(rng, s, 32, 8, 128)
    out = _run(tq, tk, tv)
    ref = _oracle_rows(tq, tk, tv, range(s))
    assert row_rel_err(out, ref) <= 1e-2
    n, mism, ties = argmax_agreement(out, ref)
    assert mism == 0


def test_c3_qwen3_prefill_4096_sampled_rows():
    """Config 3: S 4096, 32/8 heads, D 128, bf16, causal; rows sampled across the prompt."""
    rng = np.random.default_rng(0x5EED0002)
    tq, tk, tv = _inputs(rng, 4096, 32, 8, 128)
    out = _run(tq, tk, tv)
    rows = [0, 1, 2, 31, 32, 63, 64, 65, 127, 128, 1000, 2047, 2048, 3071, 4094, 4095]
    rows += list(np.random.default_rng(5).integers(0, 4096, 16))
    ref = _oracle_rows(tq, tk, tv, rows)
    assert row_rel_err(out[rows], ref) <= 1e-2
    n, mism, ties = argmax_agreement(out[rows], ref)
    assert mism == 0
    assert np.isfinite(out).all()


@pytest.mark.parametrize("hq,hkv", [(8, 4), (4, 4), (12, 4), (16, 2)])
def test_prefill_gqa_groupings(hq, hkv):
    """Groups of 2, 1, 3 (128-row workgroups) and 8 (packed 4-head workgroups)."""
    rng = np.random.default_rng(hq * 7 + hkv)
    tq, tk, tv = _inputs(rng, 300, hq, hkv, 128)
    out = _run(tq, tk, tv)
    ref = _oracle_rows(tq, tk, tv, range(300))
    assert row_rel_err(out, ref) <= 1e-2


def test_prefill_f16_inputs():
    rng = np.random.default_rng(21)
    tq, tk, tv = _inputs(rng, 257, 32, 8, 128, dtype=torch.float16)
    out = _run(tq, tk, tv)
    ref = _oracle_rows(tq, tk, tv, range(257))
    assert row_rel_err(out, ref) <= 1e-2


def test_prefill_noncausal_and_grouped_vs_f64():
    """Options outside the reference (no mask; grouped GQA) against float64 brute force."""
    rng = np.random.default_rng(22)
    tq, tk, tv = _inputs(rng, 160, 16, 4, 128)
    qf, kf, vf = (t.float().numpy() for t in (tq, tk, tv))
    out = _run(tq, tk, tv, causal=False, gqa_mode=1)
    ref = np.stack([ref64.attention(qf[i], kf, vf, lambda h: h // 4) for i in range(160)])
    assert row_rel_err(out, ref) <= 1e-2


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_batch_of_two(causal):
    """Two sequences in one launch (the batch offsets of q, k, v and out): each
    against its own oracle rows, S = 200 (a partial last tile)."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(31 + causal)
    seqs = [_inputs(rng, 200, 32, 8, 128) for _ in range(2)]
    q = torch.stack([s[0] for s in seqs]).cuda()
    k = torch.stack([s[1] for s in seqs]).cuda()
    v = torch.stack([s[2] for s in seqs]).cuda()
    out = rt.attn_prefill(dev, q, k, v, causal=causal)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for bi, (tq, tk, tv) in enumerate(seqs):
        if causal:
            ref = _oracle_rows(tq, tk, tv, range(200))
        else:
            qf, kf, vf = (t.float().numpy() for t in (tq, tk, tv))
            ref = np.stack([ref64.attention(qf[i], kf, vf, lambda h: h % 8) for i in range(200)])
        assert row_rel_err(out[bi], ref) <= 1e-2, bi


@pytest.mark.parametrize("s,hq,hkv,dtype,causal,gqa_mode", [
    (1, 8, 2, torch.bfloat16, True, 0), (200, 32, 8, torch.bfloat16, True, 0),
    (513, 16, 4, torch.float16, True, 1), (300, 12, 4, torch.bfloat16, False, 0),
    (1000, 8, 8, torch.float16, True, 0), (129, 6, 2, torch.bfloat16, True, 0)])
def test_prefill_head_dim_64(s, hq, hkv, dtype, causal, gqa_mode):
    """head_dim 64 on its own kernel (8 dims of a V row's two 32-dim groups swizzled by row
    parity): every row against the oracle's per-row decode (causal) or float64 brute force."""
    rng = np.random.default_rng(6400 + s + hq)
    tq, tk, tv = _inputs(rng, s, hq, hkv, 64, dtype=dtype)
    out = _run(tq, tk, tv, causal=causal, gqa_mode=gqa_mode)
    group = hq // hkv
    kv_of = (lambda h: h // group) if gqa_mode else (lambda h: h % hkv)
    if causal and gqa_mode == 0:
        ref = _oracle_rows(tq, tk, tv, range(s))
    else:
        qf, kf, vf = (t.float().numpy() for t in (tq, tk, tv))
        ref = np.stack([ref64.attention(qf[i], kf[:i + 1] if causal else kf,
                                        vf[:i + 1] if causal else vf, kv_of) for i in range(s)])
    assert row_rel_err(out, ref) <= 1e-2
    n, mism, ties = argmax_agreement(out, ref)
    assert mism == 0


@pytest.mark.parametrize("paired,ksplit", [("1", None), (None, "3")])
def test_prefill_head_dim_64_forced_schedules(monkeypatch, paired, ksplit):
    """D 64 under the paired schedule and a three-way key split with its merge."""
    if paired:
        monkeypatch.setenv("PI_PREFILL_PAIRED", paired)
    if ksplit:
        monkeypatch.setenv("PI_PREFILL_PAIRED", "0")
        monkeypatch.setenv("PI_PREFILL_KSPLIT", ksplit)
    rng = np.random.default_rng(6464)
    tq, tk, tv = _inputs(rng, 300, 16, 4, 64)
    out = _run(tq, tk, tv)
    assert row_rel_err(out, _oracle_rows(tq, tk, tv, range(300))) <= 1e-2


@pytest.mark.parametrize("d,s,dtype,causal", [
    (48, 300, torch.bfloat16, True), (80, 200, torch.float16, True),
    (96, 129, torch.bfloat16, False), (192, 300, torch.bfloat16, True),
    (33, 70, torch.float16, True), (200, 150, torch.float16, False)])
def test_prefill_padded_head_dims(d, s, dtype, causal):
    """Head widths with no kernel of their own (run zero-padded to 64 / 128 / 256 dims), two
    sequences in one launch with 8 / 2 heads: every row against the oracle's per-row
    decode (causal) or float64 brute force (no mask); scale 1/sqrt(d)."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(7 * d + s)
    seqs = [_inputs(rng, s, 8, 2, d, dtype=dtype) for _ in range(2)]
    q, k, v = (torch.stack([t[i] for t in seqs]).cuda() for i in range(3))
    out = rt.attn_prefill(dev, q, k, v, causal=causal)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    assert out.shape == (2, s, 8, d)
    for bi, (tq, tk, tv) in enumerate(seqs):
        if causal:
            ref = _oracle_rows(tq, tk, tv, range(s))
        else:
            qf, kf, vf = (t.float().numpy() for t in (tq, tk, tv))
            ref = np.stack([ref64.attention(qf[i], kf, vf, lambda h: h % 2) for i in range(s)])
        assert row_rel_err(out[bi], ref) <= 1e-2, bi


@pytest.mark.parametrize("s,dtype", [(1, torch.bfloat16), (70, torch.bfloat16),
                                     (300, torch.float16), (700, torch.bfloat16)])
def test_prefill_head_dim_256(s, dtype):
    """head_dim 256 (config 4's 16 q / 2 kv heads, the Qwen3.5 full-attention layers):
    every row against the oracle's per-row decode."""
    rng = np.random.default_rng(200 + s)
    tq, tk, tv = _inputs(rng, s, 16, 2, 256, dtype=dtype)
    out = _run(tq, tk, tv)
    ref = _oracle_rows(tq, tk, tv, range(s))
    assert row_rel_err(out, ref) <= 1e-2
    n, mism, ties = argmax_agreement(out, ref)
    assert mism == 0


@pytest.mark.parametrize("s,hq,hkv,dtype", [(70, 16, 2, torch.bfloat16), (300, 16, 2, torch.float16),
                                             (180, 4, 2, torch.bfloat16), (129, 2, 2, torch.float16)])
def test_prefill_head_dim_256_one_wave_per_simd_kernel(monkeypatch, s, hq, hkv, dtype):
    """The alternative D 256 kernel (PI_PREFILL_FA256=0: one wavefront per SIMD, two unit
    buffers): every row against the oracle's per-row decode, 1e-2 relative per row."""
    monkeypatch.setenv("PI_PREFILL_FA256", "0")
    rng = np.random.default_rng(260 + s + hq)
    tq, tk, tv = _inputs(rng, s, hq, hkv, 256, dtype=dtype)
    out = _run(tq, tk, tv)
    ref = _oracle_rows(tq, tk, tv, range(s))
    assert row_rel_err(out, ref) <= 1e-2
    n, mism, ties = argmax_agreement(out, ref)
    assert mism == 0


def test_prefill_head_dim_256_4096_sampled_rows():
    """The config-4 layer shape at S 4096 (16/2 heads, D 256): the launch pairs a heavy and a
    light query block per workgroup; rows sampled across the prompt, every block edge."""
    rng = np.random.default_rng(0x5EED0007)
    tq, tk, tv = _inputs(rng, 4096, 16, 2, 256, theta=1e7)
    out = _run(tq, tk, tv)
    rows = [0, 1, 15, 16, 17, 31, 32, 63, 64, 127, 128, 2047, 2048, 2049, 4064, 4094, 4095]
    rows += list(np.random.default_rng(6).integers(0, 4096, 15))
    ref = _oracle_rows(tq, tk, tv, rows)
    assert row_rel_err(out[rows], ref) <= 1e-2
    n, mism, ties = argmax_agreement(out[rows], ref)
    assert mism == 0
    assert np.isfinite(out).all()


@pytest.mark.parametrize("hq,hkv", [(4, 2), (3, 3), (5, 2)])
def test_prefill_head_dim_256_groupings(hq, hkv):
    """D 256 with two query heads per KV head (2-head workgroups), one (1-head workgroups) and
    a modulo map whose head count is not a multiple of the KV heads."""
    rng = np.random.default_rng(hq * 11 + hkv)
    tq, tk, tv = _inputs(rng, 180, hq, hkv, 256)
    out = _run(tq, tk, tv)
    ref = _oracle_rows(tq, tk, tv, range(180))
    assert row_rel_err(out, ref) <= 1e-2


def test_prefill_head_dim_256_noncausal_grouped_vs_f64():
    rng = np.random.default_rng(23)
    tq, tk, tv = _inputs(rng, 150, 8, 2, 256)
    qf, kf, vf = (t.float().numpy() for t in (tq, tk, tv))
    out = _run(tq, tk, tv, causal=False, gqa_mode=1)
    ref = np.stack([ref64.attention(qf[i], kf, vf, lambda h: h // 4) for i in range(150)])
    assert row_rel_err(out, ref) <= 1e-2


@pytest.mark.parametrize("paired,ksplit,s,hq,hkv", [("1", None, 300, 32, 8), ("1", None, 129, 4, 2),
                                                    ("0", "1", 700, 32, 8), ("0", "2", 300, 8, 2),
                                                    ("0", "3", 129, 4, 4), ("0", "4", 520, 32, 8)])
def test_prefill_forced_schedules(monkeypatch, paired, ksplit, s, hq, hkv):
    """PI_PREFILL_PAIRED / PI_PREFILL_KSPLIT (read per call) force the paired query-block
    schedule, or a given key split, on shapes the launch would schedule otherwise: every row
    against the oracle's per-row decode, 1e-2 relative per row, argmax exact."""
    monkeypatch.setenv("PI_PREFILL_PAIRED", paired)
    if ksplit is not None:
        monkeypatch.setenv("PI_PREFILL_KSPLIT", ksplit)
    rng = np.random.default_rng(380 + s + hq)
    tq, tk, tv = _inputs(rng, s, hq, hkv, 128)
    out = _run(tq, tk, tv)
    ref = _oracle_rows(tq, tk, tv, range(s))
    assert row_rel_err(out, ref) <= 1e-2
    n, mism, ties = argmax_agreement(out, ref)
    assert mism == 0


@pytest.mark.parametrize("s,hq,hkv,d", [(513, 32, 8, 128), (300, 16, 2, 256)])
def test_prefill_running_max_moves_in_late_tiles(s, hq, hkv, d):
    """Keys whose scale grows along the prompt, plus a few spike keys: the scores of later
    tiles exceed a row's running max by up to dozens of log2 units, tile after tile, so the
    kernels' rare path (max, rescale of O and the row sum, exps redone against the new max)
    runs in the middle of rows, not only on their first tile.  Every row against the oracle."""
    rng = np.random.default_rng(0x1A70 + d)
    q = rng.standard_normal((s, hq, d)).astype(np.float32)
    k = rng.standard_normal((s, hkv, d)).astype(np.float32)
    v = rng.standard_normal((s, hkv, d)).astype(np.float32)
    k *= (1.0 + np.arange(s, dtype=np.float32) / 32.0)[:, None, None]
    for t in (97, 200, 260):  # spike keys: aligned with their row's query
        if t < s:
            k[t, 0] = 6.0 * q[t, 0]
    qr, kr = orc.attn_prepare(q, k, hq, hkv, d, rope_base=1e6, pos0=0)
    tq, tk, tv = (torch.from_numpy(x).to(torch.bfloat16) for x in (qr, kr, v))
    out = _run(tq, tk, tv)
    ref = _oracle_rows(tq, tk, tv, range(s))
    assert np.isfinite(out).all()
    assert row_rel_err(out, ref) <= 1e-2

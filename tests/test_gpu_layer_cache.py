"""The device-resident LayerCache with forward's attention step (pi_attn_layer_*), fed host
slices the way InferenceContext::forward holds them (src/model/mod.rs:668-1219), against the
oracle's per-token restatement (or_attn_layer_tokens) of the same calls.

A sequence is driven through a prompt, single decode tokens and a continued multi-token chunk
(the paths of the forward: causal prefill of a prompt, one decode row per token, and a
continued chunk -- the flash prefill over the sequence's pages for an f16 cache, decode rows
over the cached history for an f32 one).  Tolerances as for the other attention tests: max-abs <= 2e-3 with an f32 cache,
per-row relative <= 1e-2 with an f16 cache; q and k come back normalised and rotated as in the
reference (<= 1e-5).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import device, row_rel_err

pytestmark = pytest.mark.gpu


def _drive(layer, chunks, oracle_kw, check, rng, hq, hkv, d, gate=False):
    kc = vc = None
    prev = 0
    for n in chunks:
        q = rng.standard_normal((n, hq, d)).astype(np.float32)
        k = rng.standard_normal((n, hkv, d)).astype(np.float32)
        v = rng.standard_normal((n, hkv, d)).astype(np.float32)
        g = rng.standard_normal((n, hq, d)).astype(np.float32) if gate else None
        ref, kc, vc = orc.attn_layer_tokens(q, k, v, gate=g, key_cache=kc, value_cache=vc,
                                            prev_seq_len=prev, **oracle_kw)
        qr, kr = orc.attn_prepare(q, k, hq, hkv, d, pos0=prev,
                                  **{x: oracle_kw[x] for x in oracle_kw if x != "gate"})
        qg, kg = q.copy(), k.copy()
        out = layer.forward(qg, kg, v, gate=g)
        check(out, ref, f"chunk of {n} at position {prev}")
        assert np.abs(qg - qr).max() <= 1e-5 and np.abs(kg - kr).max() <= 1e-5
        prev += n
        assert layer.seq_len == prev


def _rel(tol):
    def check(out, ref, what):
        for i in range(out.shape[0]):
            err = row_rel_err(out[i], ref[i])
            assert err <= tol, f"{what}: token {i} rel err {err}"
    return check


def _abs(tol):
    def check(out, ref, what):
        err = float(np.abs(out - ref).max())
        assert err <= tol, f"{what}: max-abs {err}"
    return check


def test_layer_qwen3_gqa_f16_prompt_decode_continuation():
    """32/8 heads, D 128, NORM RoPE theta 1e6, f16 cache: a 300-token prompt (causal
    prefill), three decode tokens, then a 70-token chunk over the cached history."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    layer = rt.AttnLayer(dev, 512, 32, 8, 128, torch.float16, rope_base=1e6)
    _drive(layer, [300, 1, 1, 1, 70], dict(rope_base=1e6), _rel(1e-2),
           np.random.default_rng(0x1A1), 32, 8, 128)


def test_layer_qwen35_gated_d256_norm_imrope():
    """16/2 heads, D 256, per-head Q/K RMSNorm, IMRoPE (64 rotated dims, sections
    [11, 11, 10, 0], base 1e7), sigmoid gate, f16 cache."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    rng = np.random.default_rng(0x1A2)
    qn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    sec = [11, 11, 10, 0]
    freqs = orc.compute_imrope_freqs(1e7, 64, sec)
    layer = rt.AttnLayer(dev, 256, 16, 2, 256, torch.float16, q_norm_w=qn, k_norm_w=kn,
                         rope_dim=64, rope_base=1e7, sections=sec)
    kw = dict(q_norm_w=qn, k_norm_w=kn, rope_dim=64, rope_base=1e7, freqs=freqs)
    _drive(layer, [100, 1, 1, 20], kw, _rel(1e-2), rng, 16, 2, 256, gate=True)


@pytest.mark.parametrize("d,dtype", [(192, torch.float16), (96, torch.float32)])
def test_layer_padded_width_norm_imrope(d, dtype):
    """A key head width with no kernel of its own (run padded to 256 / 128) under the Qwen3.5
    layer's options: per-head Q/K RMSNorm over d, IMRoPE on the first 64 dims (sections
    [11, 11, 10, 0], base 1e7) and the sigmoid gate."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    rng = np.random.default_rng(0x1A2 + d)
    qn = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, d).astype(np.float32)
    sec = [11, 11, 10, 0]
    freqs = orc.compute_imrope_freqs(1e7, 64, sec)
    layer = rt.AttnLayer(dev, 256, 16, 2, d, dtype, q_norm_w=qn, k_norm_w=kn,
                         rope_dim=64, rope_base=1e7, sections=sec)
    kw = dict(q_norm_w=qn, k_norm_w=kn, rope_dim=64, rope_base=1e7, freqs=freqs)
    chk = _rel(1e-2) if dtype == torch.float16 else _abs(2e-3)
    _drive(layer, [100, 1, 1, 20], kw, chk, rng, 16, 2, d, gate=True)


def test_layer_llama2_mha_f32_cache():
    """32/32 heads, D 128, theta 1e4, f32 cache: max-abs <= 2e-3."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    layer = rt.AttnLayer(dev, 128, 32, 32, 128, torch.float32, rope_base=1e4)
    _drive(layer, [64, 1, 1, 5], dict(rope_base=1e4), _abs(2e-3),
           np.random.default_rng(0x1A3), 32, 32, 128)


def test_layer_continued_chunk_over_256_rows():
    """A 300-token chunk continuing a 200-token prompt (f16 cache, 32/8 heads): more rows
    than one decode launch of the layer step takes (256), so the second launch reuses the
    per-row context lengths after the first."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    layer = rt.AttnLayer(dev, 600, 32, 8, 128, torch.float16, rope_base=1e6)
    _drive(layer, [200, 300, 1], dict(rope_base=1e6), _rel(1e-2),
           np.random.default_rng(0x1A5), 32, 8, 128)


def test_layer_f32_cache_prompt_over_256_rows():
    """A 300-token prompt with an f32 cache (32/32 heads, D 128, theta 1e4), then a
    continued 260-token chunk: max-abs <= 2e-3."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    layer = rt.AttnLayer(dev, 600, 32, 32, 128, torch.float32, rope_base=1e4)
    _drive(layer, [300, 260], dict(rope_base=1e4), _abs(2e-3),
           np.random.default_rng(0x1A6), 32, 32, 128)


def test_layer_f32_cache_gated_prompt_and_chunk():
    """The sigmoid gate on an f32 cache's prefill (applied in the f32-cache kernel's epilogue):
    a 150-token prompt, one decode token, then a 40-token chunk (8/2 heads, D 128)."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    layer = rt.AttnLayer(dev, 256, 8, 2, 128, torch.float32, rope_base=1e4)
    _drive(layer, [150, 1, 40], dict(rope_base=1e4), _abs(2e-3),
           np.random.default_rng(0x1A7), 8, 2, 128, gate=True)


@pytest.mark.parametrize("hq,hkv,d,chunks", [(16, 2, 256, [1100, 64]), (32, 8, 128, [700, 48])])
def test_layer_f16_cache_gated_prompt_and_key_split(hq, hkv, d, chunks):
    """The gate of an f16 cache's flash prefill in both places it is applied: a long prompt
    whose launch fills the chip (the gate in the prefill epilogue) and a short chunk over it
    (a small launch whose key splits are merged, the merge applying the gate)."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    layer = rt.AttnLayer(dev, sum(chunks) + 16, hq, hkv, d, torch.float16, rope_base=1e6)
    _drive(layer, chunks, dict(rope_base=1e6), _rel(1e-2),
           np.random.default_rng(0x1A8 + d), hq, hkv, d, gate=True)


def test_layer_c4_prompt_1024_split_pieces():
    """The C4 layer's fresh 1024-token prompt (16/2 heads, D 256, gated, f16 cache) under the
    default schedule: on a 256-CU chip its 128 query blocks of 1-16 key tiles run whole up to 6
    tiles and in two or three pieces beyond, so the merge combines rows of two and of three
    pieces and skips the rows the epilogue wrote."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    layer = rt.AttnLayer(dev, 1024 + 16, 16, 2, 256, torch.float16, rope_base=1e6)
    _drive(layer, [1024], dict(rope_base=1e6), _rel(1e-2), np.random.default_rng(0x1B9), 16, 2, 256,
           gate=True)


@pytest.mark.parametrize("paired,ksplit", [("1", None), (None, "2"), (None, "3"), (None, "4")])
@pytest.mark.parametrize("hq,hkv,d", [(16, 2, 256), (32, 8, 128), (8, 2, 64)])
def test_layer_f16_cache_gated_forced_schedules(monkeypatch, paired, ksplit, hq, hkv, d):
    """A gated prompt and a gated continued chunk of an f16 cache under each forced schedule: the
    paired blocks, and 2-4 key splits, where blocks longer than a split piece merge their splits
    (the merge applies the gate) and the shorter ones run whole (the epilogue applies it)."""
    if paired:
        monkeypatch.setenv("PI_PREFILL_PAIRED", paired)
    else:
        monkeypatch.setenv("PI_PREFILL_PAIRED", "0")
        monkeypatch.setenv("PI_PREFILL_KSPLIT", ksplit)
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    chunks = [300, 130]
    layer = rt.AttnLayer(dev, sum(chunks) + 16, hq, hkv, d, torch.float16, rope_base=1e6)
    _drive(layer, chunks, dict(rope_base=1e6), _rel(1e-2),
           np.random.default_rng(0x1B0 + d + (int(ksplit) if ksplit else 7)), hq, hkv, d, gate=True)


def test_layer_rejects_short_norm_weights():
    """Norm weights must hold head_dim values: a shorter array is refused before anything
    reads it."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    with pytest.raises(rt.InvalidArg):
        rt.AttnLayer(dev, 64, 16, 2, 256, torch.float16, q_norm_w=np.ones(128, np.float32),
                     k_norm_w=np.ones(256, np.float32))
    with pytest.raises(rt.InvalidArg):
        rt.AttnLayer(dev, 64, 16, 2, 256, torch.float16, k_norm_w=np.ones(255, np.float32))


def test_layer_reset_and_full_cache():
    """reset() restarts the sequence (the same prompt gives the same output); a forward that
    would overflow the cache fails with OutOfMemory and leaves the sequence as it was."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    rng = np.random.default_rng(0x1A4)
    layer = rt.AttnLayer(dev, 48, 4, 2, 128, torch.float16, rope_base=1e6)
    q = rng.standard_normal((40, 4, 128)).astype(np.float32)
    k = rng.standard_normal((40, 2, 128)).astype(np.float32)
    v = rng.standard_normal((40, 2, 128)).astype(np.float32)
    a = layer.forward(q.copy(), k.copy(), v)
    with pytest.raises(rt.OutOfMemory):
        layer.forward(q[:9].copy(), k[:9].copy(), v[:9])
    assert layer.seq_len == 40
    layer.reset()
    assert layer.seq_len == 0
    b = layer.forward(q.copy(), k.copy(), v)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("dtype,d", [(torch.float16, 128), (torch.float16, 64), (torch.float32, 128)])
def test_layer_forward_dev_misaligned_rows(dtype, d):
    """q, the gate and out at 4-byte offsets (views into larger buffers) give the bits of the
    same calls on 16-byte-aligned tensors, over a prompt, decode tokens and a chunk: the
    layer stages such rows itself, so nothing fails after the prologue has already
    rotated q and k and appended to the cache."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    hq, hkv = 4, 2
    rng = np.random.default_rng(0x1AA + d)
    a = rt.AttnLayer(dev, 256, hq, hkv, d, dtype, rope_base=1e6)
    b = rt.AttnLayer(dev, 256, hq, hkv, d, dtype, rope_base=1e6)

    def shifted(x):  # the same values one float past a 16-byte boundary
        buf = torch.empty(x.numel() + 4, dtype=x.dtype, device=x.device)
        view = buf[1:1 + x.numel()].view(x.shape)
        view.copy_(x)
        return view

    for n in (40, 1, 1, 20):
        q = torch.from_numpy(rng.standard_normal((n, hq, d)).astype(np.float32)).cuda()
        k = torch.from_numpy(rng.standard_normal((n, hkv, d)).astype(np.float32)).cuda()
        v = torch.from_numpy(rng.standard_normal((n, hkv, d)).astype(np.float32)).cuda()
        g = torch.from_numpy(rng.standard_normal((n, hq, d)).astype(np.float32)).cuda()
        qa, ka = q.clone(), k.clone()
        want = a.forward_dev(qa, ka, v, gate=g)
        qb, kb, gb = shifted(q), k.clone(), shifted(g)
        ob = shifted(torch.zeros((n, hq, d), dtype=torch.float32, device=q.device))
        assert qb.data_ptr() % 16 == 4 and gb.data_ptr() % 16 == 4 and ob.data_ptr() % 16 == 4
        got = b.forward_dev(qb, kb, v, gate=gb, out=ob)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), n
        assert torch.equal(qb.view(torch.int32), qa.view(torch.int32)), n
        assert torch.equal(kb.view(torch.int32), ka.view(torch.int32)), n
        assert a.seq_len == b.seq_len

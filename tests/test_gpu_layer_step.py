"""The fused prologue (pi_attn_prologue: per-head Q/K RMSNorm + RoPE + paged
append, src/model/mod.rs:1035-1146) and whole full-attention layer steps built
from it and pi_attn_decode, against the oracle's per-token layer
(or_attn_layer_tokens = src/model/mod.rs:1035-1196)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import device, row_rel_err, to_dev

pytestmark = pytest.mark.gpu


def _pool(rt, dev, n_seq, max_tokens, hkv, d, dtype, rng):
    pages = (max_tokens + 15) // 16
    perm = rng.permutation(n_seq * pages).astype(np.int32)
    pt = perm.reshape(n_seq, pages)
    return rt.KvPool(dev, n_seq * pages, hkv, d, dtype=dtype), to_dev(pt)


@pytest.mark.parametrize("shape", ["c2", "c4", "c2_prompt", "c4_prompt", "c4_f32"])
def test_prologue_matches_oracle(shape):
    """Three sequences, 5 tokens each at different offsets; *_prompt: one 1100-token
    prompt (a launch of >= 1024 tokens shares one cos / sin table per token), with NORM
    RoPE (c2) or Q/K RMSNorm and IMRoPE at D 256 (c4); the c2 shapes and c4_f32 append to an
    f32 pool, the other c4 shapes to an f16 one."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(50)
    if shape.startswith("c2"):
        hq, hkv, d, base, rd, sec, norm = 32, 8, 128, 1e6, 128, None, False
    else:
        hq, hkv, d, base, rd, sec, norm = 16, 2, 256, 1e7, 64, [11, 11, 10, 0], True
    n_seq, n_tok = 3, 5
    starts = np.array([0, 17, 40000], np.int32)
    if shape.endswith("_prompt"):
        n_seq, n_tok = 1, 1100
        starts = np.array([7], np.int32)
    q = rng.standard_normal((n_seq, n_tok, hq, d)).astype(np.float32)
    k = rng.standard_normal((n_seq, n_tok, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n_seq, n_tok, hkv, d)).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, d).astype(np.float32) if norm else None
    kn = rng.uniform(0.5, 1.5, d).astype(np.float32) if norm else None
    freqs = orc.compute_imrope_freqs(base, rd, sec) if sec else None
    pool_dtype = torch.float16 if shape in ("c4", "c4_prompt") else torch.float32
    pool, pt = _pool(rt, dev, n_seq, int(starts.max()) + n_tok, hkv, d, pool_dtype, rng)
    tq, tk = to_dev(q), to_dev(k)
    rt.attn_prologue(dev, tq, tk, to_dev(v), pool, pt, to_dev(starts),
                     None if qn is None else to_dev(qn), None if kn is None else to_dev(kn),
                     1e-6, rd, base, sec)
    torch.cuda.synchronize()
    for s in range(n_seq):
        rq, rk = orc.attn_prepare(q[s], k[s], hq, hkv, d, q_norm_w=qn, k_norm_w=kn, eps=1e-6,
                                  rope_dim=rd, rope_base=base, freqs=freqs, pos0=int(starts[s]))
        tol = 2e-5 * max(1.0, starts[s] / 1000)
        np.testing.assert_allclose(tq[s].cpu().numpy(), rq, rtol=0, atol=tol)
        np.testing.assert_allclose(tk[s].cpu().numpy(), rk, rtol=0, atol=tol)
        kc, vc = pool.read(pt, s, int(starts[s]), n_tok)
        torch.cuda.synchronize()
        if pool_dtype == torch.float32:
            np.testing.assert_allclose(kc.cpu().numpy(), rk, rtol=0, atol=tol)
            assert np.array_equal(vc.cpu().numpy(), v[s])
        else:  # f16 pool: RNE-rounded copies
            np.testing.assert_allclose(kc.cpu().numpy(), rk.astype(np.float16).astype(np.float32),
                                       rtol=2e-3, atol=tol)
            assert np.array_equal(vc.cpu().numpy(), v[s].astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("shape", ["c2", "c4", "c4_prompt", "c4_f32"])
def test_prologue_lds_staged_kernel(monkeypatch, shape):
    """PI_PROLOGUE_VEC=0 (read per call): the LDS-staged prologue kernel on the same
    shapes and checks as the register-resident one."""
    monkeypatch.setenv("PI_PROLOGUE_VEC", "0")
    test_prologue_matches_oracle(shape)

@pytest.mark.parametrize("case", ["c1_f32", "c4_f16"])
def test_layer_prefill_then_decode_steps(case):
    """A 48-token prompt through the prologue, then 6 decode steps (prologue
    n_tok=1 + pi_attn_decode); every decode output against the reference's
    per-token layer.  c1_f32: Llama-2 MHA shape (32/32 heads, D 128, NORM RoPE
    1e4), f32 pool, max-abs 2e-3.  c4_f16: Qwen3.5 gated shape (16/2 heads,
    D 256, q/k norm, IMRoPE 64 of 256, 1e7, sigmoid gate), f16 pool, 1e-2 rel."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(51)
    if case == "c1_f32":
        hq, hkv, d, base, rd, sec, pool_dtype, gated, norm = 32, 32, 128, 1e4, 128, None, torch.float32, False, False
    else:
        hq, hkv, d, base, rd, sec, pool_dtype, gated, norm = 16, 2, 256, 1e7, 64, [11, 11, 10, 0], torch.float16, True, True
    n_prompt, n_steps = 48, 6
    total = n_prompt + n_steps
    q = rng.standard_normal((total, hq, d)).astype(np.float32)
    k = rng.standard_normal((total, hkv, d)).astype(np.float32)
    v = rng.standard_normal((total, hkv, d)).astype(np.float32)
    gate = rng.standard_normal((total, hq, d)).astype(np.float32) if gated else None
    qn = rng.uniform(0.5, 1.5, d).astype(np.float32) if norm else None
    kn = rng.uniform(0.5, 1.5, d).astype(np.float32) if norm else None
    freqs = orc.compute_imrope_freqs(base, rd, sec) if sec else None
    ref, _, _ = orc.attn_layer_tokens(q, k, v, gate=gate, q_norm_w=qn, k_norm_w=kn, eps=1e-6,
                                      rope_dim=rd, rope_base=base, freqs=freqs)
    pool, pt = _pool(rt, dev, 1, total, hkv, d, pool_dtype, rng)
    tqn = None if qn is None else to_dev(qn)
    tkn = None if kn is None else to_dev(kn)
    rt.attn_prologue(dev, to_dev(q[None, :n_prompt]), to_dev(k[None, :n_prompt]),
                     to_dev(v[None, :n_prompt]), pool, pt,
                     torch.zeros(1, dtype=torch.int32, device="cuda"), tqn, tkn, 1e-6, rd, base, sec)
    for i in range(n_prompt, total):
        tq = to_dev(q[None, i:i + 1])
        rt.attn_prologue(dev, tq, to_dev(k[None, i:i + 1]), to_dev(v[None, i:i + 1]), pool, pt,
                         to_dev(np.array([i], np.int32)), tqn, tkn, 1e-6, rd, base, sec)
        out = rt.attn_decode(dev, tq[0], pool, pt, to_dev(np.array([i + 1], np.int32)),
                             gate=None if gate is None else to_dev(gate[i:i + 1]))
        torch.cuda.synchronize()
        o = out.cpu().numpy()[0]
        if pool_dtype == torch.float32:
            assert np.abs(o - ref[i]).max() <= 2e-3
        else:
            assert row_rel_err(o, ref[i]) <= 1e-2

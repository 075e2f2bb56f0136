"""The steps either side of the gated-DeltaNet recurrence on the GPU vs the
oracle: depthwise causal conv1d + SiLU with its rolling state
(src/model/mod.rs:750-776) and RMSNormGated x SiLU(z) (:918-932), then a whole
Qwen3.5 GDN layer body from the QKV projection output to the gated output."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import device, to_dev

pytestmark = pytest.mark.gpu


def _conv_oracle(x, hist, w):
    """Token by token through or_conv1d_silu; x [T, C], hist [d_conv-1, C]."""
    outs = []
    h = hist.copy()
    for t in range(x.shape[0]):
        o, h = orc.conv1d_silu(x[t], h, w, w.shape[1])
        outs.append(o)
    return np.stack(outs), h


@pytest.mark.parametrize("n_tok", [1, 2, 3, 4, 65, 4096])
def test_conv1d_matches_oracle(n_tok):
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(40 + n_tok)
    c, d_conv = 8192, 4  # Qwen3.5: conv_dim = 2*16*128 + 32*128
    x = rng.standard_normal((n_tok, c)).astype(np.float32)
    hist = rng.standard_normal((d_conv - 1, c)).astype(np.float32)
    w = (rng.standard_normal((c, d_conv)) * 0.5).astype(np.float32)
    ref, ref_hist = _conv_oracle(x, hist, w)
    st = to_dev(hist[None])
    out = rt.gdn_conv1d(dev, to_dev(x[None]), st, to_dev(w))
    torch.cuda.synchronize()
    np.testing.assert_allclose(out[0].cpu().numpy(), ref, rtol=1e-5, atol=1e-6)
    assert np.array_equal(st[0].cpu().numpy(), ref_hist)  # the state is a copy of raw inputs


@pytest.mark.parametrize("c,d_conv,n_tok", [(1022, 4, 70), (512, 3, 33), (512, 3, 1)])
def test_conv1d_general_shapes(c, d_conv, n_tok):
    """Channel counts not divisible by 4 and d_conv != 4 (the general kernel)."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(47 + c + n_tok)
    x = rng.standard_normal((n_tok, c)).astype(np.float32)
    hist = rng.standard_normal((d_conv - 1, c)).astype(np.float32)
    w = (rng.standard_normal((c, d_conv)) * 0.5).astype(np.float32)
    ref, ref_hist = _conv_oracle(x, hist, w)
    st = to_dev(hist[None])
    out = rt.gdn_conv1d(dev, to_dev(x[None]), st, to_dev(w))
    torch.cuda.synchronize()
    np.testing.assert_allclose(out[0].cpu().numpy(), ref, rtol=1e-5, atol=1e-6)
    assert np.array_equal(st[0].cpu().numpy(), ref_hist)


def test_conv1d_batched_decode_from_zero_state():
    """Three sequences, one token each, from the reference's zero initial window
    (src/model/mod.rs:752-756), then a second token."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(45)
    c, d_conv = 1024, 4
    w = rng.standard_normal((c, d_conv)).astype(np.float32)
    st = torch.zeros((3, d_conv - 1, c), device="cuda")
    hists = [np.zeros((d_conv - 1, c), np.float32) for _ in range(3)]
    for step in range(2):
        x = rng.standard_normal((3, 1, c)).astype(np.float32)
        out = rt.gdn_conv1d(dev, to_dev(x), st, to_dev(w))
        torch.cuda.synchronize()
        for s in range(3):
            ref, hists[s] = _conv_oracle(x[s], hists[s], w)
            np.testing.assert_allclose(out[s].cpu().numpy(), ref, rtol=1e-5, atol=1e-6)
            assert np.array_equal(st[s].cpu().numpy(), hists[s])


def test_rmsnorm_gated_matches_oracle():
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(46)
    o = rng.standard_normal((17, 32, 128)).astype(np.float32)
    z = rng.standard_normal((17, 32, 128)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    ref = orc.rmsnorm_gated(o, z, w, 1e-6)
    to = to_dev(o)
    rt.gdn_rmsnorm_gated(dev, to, to_dev(z), to_dev(w), 1e-6)
    torch.cuda.synchronize()
    np.testing.assert_allclose(to.cpu().numpy(), ref, rtol=2e-5, atol=2e-6)


def test_gdn_layer_body_prefill_then_decode():
    """conv1d -> split q/k/v -> gates -> recurrence -> RMSNormGated for a 200-token
    prompt and 3 decode tokens, all on the GPU, against the oracle's per-token
    chain of the same reference steps (src/model/mod.rs:750-932)."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(47)
    hk, hv, d, d_conv = 16, 32, 128, 4
    kd = hk * d
    c = 2 * kd + hv * d
    w_conv = (rng.standard_normal((c, d_conv)) * 0.5).astype(np.float32)
    ssm_a = -rng.uniform(0.5, 2.0, hv).astype(np.float32)
    dt_bias = rng.standard_normal(hv).astype(np.float32)
    w_norm = rng.uniform(0.5, 1.5, d).astype(np.float32)
    eps = 1e-6

    def oracle_tokens(qkv, br, ar, z, hist, state):
        outs = []
        for t in range(qkv.shape[0]):
            a, hist = orc.conv1d_silu(qkv[t], hist, w_conv, d_conv)
            q, k, v = a[:kd].reshape(1, hk, d), a[kd:2 * kd].reshape(1, hk, d), a[2 * kd:].reshape(1, hv, d)
            beta, g = orc.gdn_gates(br[t], ar[t], ssm_a, dt_bias)
            o, state = orc.gdn_tokens(q, k, v, beta[None], g[None], state)
            outs.append(orc.rmsnorm_gated(o, z[t][None], w_norm, eps)[0])
        return np.stack(outs), hist, state

    hist = np.zeros((d_conv - 1, c), np.float32)
    state = np.zeros((hv, d, d), np.float32)
    t_conv = torch.zeros((1, d_conv - 1, c), device="cuda")
    t_state = torch.zeros((hv, d, d), device="cuda")
    t_w = to_dev(w_conv)
    for n_tok in (200, 1, 1, 1):
        qkv = rng.standard_normal((n_tok, c)).astype(np.float32)
        br = rng.standard_normal((n_tok, hv)).astype(np.float32)
        ar = rng.standard_normal((n_tok, hv)).astype(np.float32)
        z = rng.standard_normal((n_tok, hv, d)).astype(np.float32)
        ref, hist, state = oracle_tokens(qkv, br, ar, z, hist, state)

        act = rt.gdn_conv1d(dev, to_dev(qkv[None]), t_conv, t_w)[0]
        q = act[:, :kd].reshape(n_tok, hk, d).contiguous()
        k = act[:, kd:2 * kd].reshape(n_tok, hk, d).contiguous()
        v = act[:, 2 * kd:].reshape(n_tok, hv, d).contiguous()
        beta, g = rt.gdn_gates(dev, to_dev(br), to_dev(ar), to_dev(ssm_a), to_dev(dt_bias))
        if n_tok > 1:
            o = rt.gdn_prefill(dev, q, k, v, beta, g, t_state)
        else:
            o = rt.gdn_decode(dev, q, k, v, beta, g, t_state[None])
        rt.gdn_rmsnorm_gated(dev, o, to_dev(z), to_dev(w_norm), eps)
        torch.cuda.synchronize()
        err = np.abs(o.cpu().numpy() - ref).max()
        assert err <= 2e-3, (n_tok, err)
        assert np.abs(t_state.cpu().numpy() - state).max() <= 2e-3

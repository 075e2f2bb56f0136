"""Gated-DeltaNet at head widths other than 128 and with the token-by-token prefill
(src/model/mod.rs:841-916 takes any k_hd / v_hd and any head counts, V head vh reading
K head vh % n_k_heads; here k_hd up to 1024), against the oracle's per-token recurrence: max-abs <= 2e-3 on
outputs and on the state, as for the 128-wide kernels.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import device, to_dev

pytestmark = pytest.mark.gpu

TOL = 2e-3
# k_hd above 256 runs with 2 state columns per wavefront (32 row groups), up to 1024
DIMS = [(64, 64), (96, 80), (256, 128), (128, 200), (32, 17), (200, 128), (257, 40), (512, 33),
        (1024, 16)]


def _inputs(rng, lead, hk, hv, dk, dv):
    q = rng.standard_normal(lead + (hk, dk)).astype(np.float32)
    k = rng.standard_normal(lead + (hk, dk)).astype(np.float32)
    v = rng.standard_normal(lead + (hv, dv)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal(lead + (hv,))))).astype(np.float32)
    g = (-np.log1p(np.exp(rng.standard_normal(lead + (hv,))))).astype(np.float32)
    return q, k, v, beta, g


@pytest.mark.parametrize("dk,dv", DIMS)
def test_gdn_decode_widths_batched(dk, dv):
    """Two steps of a batch of 3 sequences with non-zero states, 3 K heads / 5 V heads."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(dk * 1000 + dv)
    b, hk, hv = 3, 3, 5
    s0 = (0.3 * rng.standard_normal((b, hv, dk, dv))).astype(np.float32)
    state = to_dev(s0)
    steps = [_inputs(rng, (b,), hk, hv, dk, dv) for _ in range(2)]
    outs = [rt.gdn_decode(dev, *(to_dev(x) for x in st), state).cpu().numpy() for st in steps]
    st = state.cpu().numpy()
    for i in range(b):
        q, k, v, beta, g = (np.stack([s[j][i] for s in steps]) for j in range(5))
        ro, rs = orc.gdn_tokens(q, k, v, beta, g, state=s0[i])
        got = np.stack([o[i] for o in outs])
        assert np.abs(got - ro).max() <= TOL, f"seq {i}: out {np.abs(got - ro).max()}"
        assert np.abs(st[i] - rs).max() <= TOL, f"seq {i}: state {np.abs(st[i] - rs).max()}"


@pytest.mark.parametrize("dk,dv", DIMS)
def test_gdn_prefill_widths(dk, dv):
    """150 tokens of one sequence from a non-zero state (2 K heads, 6 V heads)."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(7 + dk + dv)
    t, hk, hv = 150, 2, 6
    q, k, v, beta, g = _inputs(rng, (t,), hk, hv, dk, dv)
    s0 = (0.3 * rng.standard_normal((hv, dk, dv))).astype(np.float32)
    ro, rs = orc.gdn_tokens(q, k, v, beta, g, state=s0)
    state = to_dev(s0)
    out = rt.gdn_prefill(dev, *(to_dev(x) for x in (q, k, v, beta, g)), state).cpu().numpy()
    assert np.abs(out - ro).max() <= TOL
    assert np.abs(state.cpu().numpy() - rs).max() <= TOL


def test_gdn_prefill_token_by_token_at_128():
    """chunk = 1 at the config-5 widths (16 / 32 heads of 128) over 300 tokens: the per-token
    kernel against the oracle, and against the chunked form on the same inputs."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(0x6D1)
    t, hk, hv = 300, 16, 32
    x = _inputs(rng, (t,), hk, hv, 128, 128)
    ro, rs = orc.gdn_tokens(*x)
    outs = {}
    for chunk in (1, 64):
        state = torch.zeros((hv, 128, 128), device="cuda")
        outs[chunk] = rt.gdn_prefill(dev, *(to_dev(a) for a in x), state, chunk=chunk).cpu().numpy()
        assert np.abs(outs[chunk] - ro).max() <= TOL, chunk
        assert np.abs(state.cpu().numpy() - rs).max() <= TOL, chunk
    assert np.abs(outs[1] - outs[64]).max() <= TOL


def test_gdn_layer_other_widths():
    """The layer step (conv1d, gates, recurrence, RMSNormGated) at k_hd 64, v_hd 96: a prompt,
    two decode tokens and a continued chunk against the oracle's per-token layer."""
    from powerinfer_x64_amd import runtime as rt
    from tests.test_gpu_gdn_layer import _OracleLayer, _inputs as layer_inputs, _weights
    dev = device()
    rng = np.random.default_rng(0x64_96)
    hk, hv, dk, dv = 2, 4, 64, 96
    w = _weights(rng, hk, hv, dk, dv, 4)
    layer = rt.GdnLayer(dev, hk, hv, dk, dv, *w, eps=1e-6)
    ref = _OracleLayer(hk, hv, dk, dv, *w, 1e-6)
    for n in (70, 1, 1, 25):
        x = layer_inputs(rng, n, hk, hv, dk, dv)
        want, tol = ref.forward(*x)
        got = layer.forward(*x)
        assert (np.abs(got - want) <= tol).all(), (n, float((np.abs(got - want) / tol).max()))
    layer.close()


def test_gdn_layer_wide_key_heads():
    """The layer step at k_hd 384 (two state columns per wavefront of the per-token kernel),
    v_hd 64: a prompt, a decode token and a continued chunk against the oracle's layer."""
    from powerinfer_x64_amd import runtime as rt
    from tests.test_gpu_gdn_layer import _OracleLayer, _inputs as layer_inputs, _weights
    dev = device()
    rng = np.random.default_rng(0x384)
    hk, hv, dk, dv = 1, 2, 384, 64
    w = _weights(rng, hk, hv, dk, dv, 4)
    layer = rt.GdnLayer(dev, hk, hv, dk, dv, *w, eps=1e-6)
    ref = _OracleLayer(hk, hv, dk, dv, *w, 1e-6)
    for n in (40, 1, 9):
        x = layer_inputs(rng, n, hk, hv, dk, dv)
        want, tol = ref.forward(*x)
        got = layer.forward(*x)
        assert (np.abs(got - want) <= tol).all(), (n, float((np.abs(got - want) / tol).max()))
    layer.close()


def test_gdn_rejects_unsupported_widths_and_chunks():
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(3)
    x = _inputs(rng, (4,), 1, 1, 1025, 8)
    state = torch.zeros((1, 1025, 8), device="cuda")
    with pytest.raises(rt.Unsupported):
        rt.gdn_prefill(dev, *(to_dev(a) for a in x), state)
    x = _inputs(rng, (4,), 1, 1, 128, 128)
    state = torch.zeros((1, 128, 128), device="cuda")
    with pytest.raises(rt.Unsupported):
        rt.gdn_prefill(dev, *(to_dev(a) for a in x), state, chunk=32)

"""Gated-DeltaNet on the GPU vs the CPU oracle (src/model/mod.rs:796-916).

Tolerance (f32 inputs): max-abs <= 2e-3 on outputs and
on the recurrent state.  Inputs follow config 5: q/k ~ N(0,1) (normalised by
the op), v ~ N(0,1), beta = sigmoid(N(0,1)), g = -softplus(N(0,1)).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import device, to_dev

pytestmark = pytest.mark.gpu

HK, HV, DK, DV = 16, 32, 128, 128


def _inputs(rng, t, b=None):
    lead = (t,) if b is None else (t, b)
    q = rng.standard_normal(lead + (HK, DK)).astype(np.float32)
    k = rng.standard_normal(lead + (HK, DK)).astype(np.float32)
    v = rng.standard_normal(lead + (HV, DV)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal(lead + (HV,))))).astype(np.float32)
    g = (-np.log1p(np.exp(rng.standard_normal(lead + (HV,))))).astype(np.float32)
    return q, k, v, beta, g


def _rt():
    from powerinfer_x64_amd import runtime as rt
    return rt


def test_gdn_gates_match_oracle():
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(1)
    br = rng.standard_normal((5, HV)).astype(np.float32) * 4
    ar = rng.standard_normal((5, HV)).astype(np.float32) * 8
    sa = -np.exp(rng.standard_normal(HV)).astype(np.float32)
    db = rng.standard_normal(HV).astype(np.float32)
    beta, g = rt.gdn_gates(dev, to_dev(br), to_dev(ar), to_dev(sa), to_dev(db))
    for t in range(5):
        eb, eg = orc.gdn_gates(br[t], ar[t], sa, db)
        np.testing.assert_allclose(beta[t].cpu().numpy(), eb, rtol=2e-6, atol=1e-7)
        np.testing.assert_allclose(g[t].cpu().numpy(), eg, rtol=2e-6, atol=1e-7)


def test_gdn_decode_steps_match_oracle():
    """16 consecutive single-token steps from a zero state (ssm::create_ssm_state)."""
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(0x5EED0004)
    t = 16
    q, k, v, beta, g = _inputs(rng, t)
    ref_out, ref_state = orc.gdn_tokens(q, k, v, beta, g)
    state = torch.zeros((1, HV, DK, DV), device="cuda")
    outs = []
    for i in range(t):
        o = rt.gdn_decode(dev, to_dev(q[i][None]), to_dev(k[i][None]), to_dev(v[i][None]),
                          to_dev(beta[i][None]), to_dev(g[i][None]), state)
        outs.append(o[0].cpu().numpy())
    out = np.stack(outs)
    assert np.abs(out - ref_out).max() <= 2e-3
    assert np.abs(state[0].cpu().numpy() - ref_state).max() <= 2e-3


def test_gdn_decode_batched_nonzero_state():
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(5)
    b = 3
    q, k, v, beta, g = _inputs(rng, 1, b)
    s0 = (0.3 * rng.standard_normal((b, HV, DK, DV))).astype(np.float32)
    state = to_dev(s0)
    out = rt.gdn_decode(dev, to_dev(q[0]), to_dev(k[0]), to_dev(v[0]), to_dev(beta[0]),
                        to_dev(g[0]), state).cpu().numpy()
    st = state.cpu().numpy()
    for i in range(b):
        ro, rs = orc.gdn_tokens(q[:, i], k[:, i], v[:, i], beta[:, i], g[:, i], state=s0[i])
        assert np.abs(out[i] - ro[0]).max() <= 2e-3
        assert np.abs(st[i] - rs).max() <= 2e-3


def test_gdn_decode_zero_state_closed_form():
    """src/bin/layer_trace.rs:180-196: from a zero state o = beta * (q.k) * v."""
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(6)
    q, k, v, beta, g = _inputs(rng, 1)
    state = torch.zeros((1, HV, DK, DV), device="cuda")
    out = rt.gdn_decode(dev, to_dev(q), to_dev(k), to_dev(v), to_dev(beta), to_dev(g),
                        state).cpu().numpy()[0]
    for h in range(HV):
        qq = q[0, h % HK].astype(np.float64)
        kk = k[0, h % HK].astype(np.float64)
        qk = (qq / np.linalg.norm(qq) / np.sqrt(DK)) @ (kk / np.linalg.norm(kk))
        np.testing.assert_allclose(out[h], beta[0, h] * qk * v[0, h], atol=1e-5)


def _check(out, ref_out, state, ref_state, tol=2e-3):
    eo = float(np.abs(out - ref_out).max())
    es = float(np.abs(state - ref_state).max())
    print(f"max-abs error: out {eo:.3e}, state {es:.3e}")
    assert eo <= tol, f"out max-abs {eo}"
    assert es <= tol, f"state max-abs {es}"


@pytest.mark.parametrize("t", [1, 63, 64, 65, 200, 1024, 1130])
def test_gdn_prefill_matches_oracle(t):
    """Chunked (64-token) prefill == the reference's per-token recurrence.  t = 1130 gives
    18 chunks, more than one per prep workgroup on a 256-CU device (16 K heads), with the
    ragged tail on a workgroup's second chunk."""
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(1000 + t)
    q, k, v, beta, g = _inputs(rng, t)
    s0 = (0.2 * rng.standard_normal((HV, DK, DV))).astype(np.float32) if t % 2 else \
        np.zeros((HV, DK, DV), np.float32)
    ref_out, ref_state = orc.gdn_tokens(q, k, v, beta, g, state=s0)
    state = to_dev(s0)
    out = rt.gdn_prefill(dev, to_dev(q), to_dev(k), to_dev(v), to_dev(beta), to_dev(g), state)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), ref_out, state.cpu().numpy(), ref_state)


@pytest.mark.parametrize("hk,hv,t", [(32, 32, 1250), (4, 12, 300)])
def test_gdn_prefill_other_head_counts(hk, hv, t):
    """Other K/V head tilings (vh % hk): 32 K heads with one V head each (the prep's second
    V-head half is idle, and on a 256-CU device each prep workgroup walks 3 chunks with the
    ragged tail on the last), and 4 K heads with 3 V heads each (two V-head passes)."""
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(5000 + hk + t)
    q = rng.standard_normal((t, hk, DK)).astype(np.float32)
    k = rng.standard_normal((t, hk, DK)).astype(np.float32)
    v = rng.standard_normal((t, hv, DV)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((t, hv))))).astype(np.float32)
    g = (-np.log1p(np.exp(rng.standard_normal((t, hv))))).astype(np.float32)
    s0 = (0.2 * rng.standard_normal((hv, DK, DV))).astype(np.float32)
    ref_out, ref_state = orc.gdn_tokens(q, k, v, beta, g, state=s0)
    state = to_dev(s0)
    out = rt.gdn_prefill(dev, to_dev(q), to_dev(k), to_dev(v), to_dev(beta), to_dev(g), state)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), ref_out, state.cpu().numpy(), ref_state)


def test_gdn_prefill_strong_decay_and_zero_beta():
    """Edge gates: g -> -1e4 (state reset each token) and beta = 0 (pure decay)."""
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(77)
    t = 130
    q, k, v, beta, g = _inputs(rng, t)
    g[::3] = -1e4
    beta[1::5] = 0.0
    s0 = (0.2 * rng.standard_normal((HV, DK, DV))).astype(np.float32)
    ref_out, ref_state = orc.gdn_tokens(q, k, v, beta, g, state=s0)
    state = to_dev(s0)
    out = rt.gdn_prefill(dev, to_dev(q), to_dev(k), to_dev(v), to_dev(beta), to_dev(g), state)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), ref_out, state.cpu().numpy(), ref_state)


def test_c5_gdn_prefill_4096_then_256_decode():
    """Config 5: chunked prefill of 4096 tokens, then 256 recurrent decode steps,
    continuing the same state; outputs and final state vs the oracle."""
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(0x5EED0004)
    tp, td = 4096, 256
    q, k, v, beta, g = _inputs(rng, tp + td)
    ref_out, ref_state = orc.gdn_tokens(q, k, v, beta, g)
    state = torch.zeros((HV, DK, DV), device="cuda")
    out_p = rt.gdn_prefill(dev, to_dev(q[:tp]), to_dev(k[:tp]), to_dev(v[:tp]),
                           to_dev(beta[:tp]), to_dev(g[:tp]), state)
    st = state[None]
    outs = []
    for i in range(tp, tp + td):
        o = rt.gdn_decode(dev, to_dev(q[i][None]), to_dev(k[i][None]), to_dev(v[i][None]),
                          to_dev(beta[i][None]), to_dev(g[i][None]), st)
        outs.append(o[0])
    torch.cuda.synchronize()
    out = np.concatenate([out_p.cpu().numpy(), torch.stack(outs).cpu().numpy()])
    _check(out, ref_out, st[0].cpu().numpy(), ref_state)

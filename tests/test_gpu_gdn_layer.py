"""The device-resident gated-DeltaNet layer (pi_gdn_layer_*) against the oracle's
per-token chain of the reference's GDN step (src/model/mod.rs:750-932): conv1d +
SiLU with the rolling state, the q / k / v split, beta / g, the delta rule and
RMSNormGated, with both states carried across calls and cleared by reset
(src/model/mod.rs:1867-1869)."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import device

pytestmark = pytest.mark.gpu

# max-abs bound on the recurrence's output (the delta-rule tests hold it at 2e-3)
TOL = 2e-3


class _OracleLayer:
    """Token-by-token restatement of one GDN layer with its own conv and SSM state."""

    def __init__(self, hk, hv, dk, dv, w_conv, ssm_a, dt_bias, w_norm, eps):
        self.hk, self.hv, self.dk, self.dv = hk, hv, dk, dv
        self.w, self.a, self.dt, self.nw, self.eps = w_conv, ssm_a, dt_bias, w_norm, eps
        self.reset()

    def reset(self):
        self.hist = np.zeros((self.w.shape[1] - 1, self.w.shape[0]), np.float32)
        self.state = np.zeros((self.hv, self.dk, self.dv), np.float32)

    def forward(self, qkv, z, br, ar):
        """Returns the gated output [n, Hv, Dv] and its per-element tolerance: the
        recurrence's max-abs bound TOL carried through RMSNormGated to first order,
        y = o / rms(o) * w * SiLU(z), |dy_i| <= TOL * |w_i SiLU(z_i)| / rms * (1 + |o_i| / rms)."""
        kd = self.hk * self.dk
        outs, tols = [], []
        for t in range(qkv.shape[0]):
            a, self.hist = orc.conv1d_silu(qkv[t], self.hist, self.w, self.w.shape[1])
            q = a[:kd].reshape(1, self.hk, self.dk)
            k = a[kd:2 * kd].reshape(1, self.hk, self.dk)
            v = a[2 * kd:].reshape(1, self.hv, self.dv)
            beta, g = orc.gdn_gates(br[t], ar[t], self.a, self.dt)
            o, self.state = orc.gdn_tokens(q, k, v, beta[None], g[None], self.state)
            outs.append(orc.rmsnorm_gated(o, z[t][None], self.nw, self.eps)[0])
            o = o[0].astype(np.float64)
            rms = np.sqrt((o * o).mean(axis=-1, keepdims=True) + self.eps)
            zt = z[t].astype(np.float64)
            gain = np.abs(self.nw * zt / (1 + np.exp(-zt))) / rms
            tols.append(TOL * gain * (1 + np.abs(o) / rms))
        return np.stack(outs), np.stack(tols)


def _weights(rng, hk, hv, dk, dv, d_conv):
    c = 2 * hk * dk + hv * dv
    return ((rng.standard_normal((c, d_conv)) * 0.5).astype(np.float32),
            -rng.uniform(0.5, 2.0, hv).astype(np.float32),
            rng.standard_normal(hv).astype(np.float32),
            rng.uniform(0.5, 1.5, dv).astype(np.float32))


def _inputs(rng, n, hk, hv, dk, dv):
    c = 2 * hk * dk + hv * dv
    return (rng.standard_normal((n, c)).astype(np.float32),
            rng.standard_normal((n, hv, dv)).astype(np.float32),
            rng.standard_normal((n, hv)).astype(np.float32),
            rng.standard_normal((n, hv)).astype(np.float32))


@pytest.mark.parametrize("hk,hv,d", [(16, 32, 128), (2, 4, 128), (3, 6, 128), (4, 4, 128)])
def test_gdn_layer_prompt_decode_chunk_reset(hk, hv, d):
    """A 200-token prompt, 3 decode tokens, a 65-token continued chunk, then reset
    and a fresh 1-token start and 40-token prompt.  Each output element within the
    recurrence's 2e-3 bound carried through RMSNormGated (_OracleLayer.forward), and each
    (token, V head) row within 1e-2 relative."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(90 + hk)
    w = _weights(rng, hk, hv, d, d, 4)
    eps = 1e-6
    layer = rt.GdnLayer(dev, hk, hv, d, d, *w, eps=eps)
    ref = _OracleLayer(hk, hv, d, d, *w, eps)
    for n in (200, 1, 1, 1, 65, "reset", 1, 40):
        if n == "reset":
            layer.reset()
            ref.reset()
            continue
        qkv, z, br, ar = _inputs(rng, n, hk, hv, d, d)
        want, tol = ref.forward(qkv, z, br, ar)
        got = layer.forward(qkv, z, br, ar)
        err = np.abs(got - want)
        row = np.sqrt((err ** 2).sum(-1) / np.maximum((want ** 2).sum(-1), 1e-30))
        print(f"hk={hk} hv={hv} n={n} max_abs={err.max():.2e} "
              f"max err/tol={(err / tol).max():.3f} row_rel={row.max():.2e}", flush=True)
        assert (err <= tol).all(), (n, float((err / tol).max()))
        # and per (token, V head) row, relative L2 <= 1e-2 (the norm makes every row unit
        # scale, so rows of a near-zero recurrence output carry its absolute error as relative)
        assert row.max() <= 1e-2, (n, float(row.max()))
    layer.close()


def test_gdn_layer_two_layers_keep_their_own_state():
    """Two layer objects with different weights, interleaved token by token, match two
    independent oracle layers: no state is shared between layers."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(93)
    hk, hv, d = 2, 4, 128
    ws = [_weights(rng, hk, hv, d, d, 4) for _ in range(2)]
    layers = [rt.GdnLayer(dev, hk, hv, d, d, *w) for w in ws]
    refs = [_OracleLayer(hk, hv, d, d, *w, 1e-6) for w in ws]
    for n in (17, 1, 1, 9):
        for L, R in zip(layers, refs):
            x = _inputs(rng, n, hk, hv, d, d)
            want, tol = R.forward(*x)
            assert (np.abs(L.forward(*x) - want) <= tol).all(), n
    for L in layers:
        L.close()


def test_gdn_layer_rejects_bad_shapes():
    from powerinfer_x64_amd import runtime as rt
    from powerinfer_x64_amd.runtime import InvalidArg
    dev = device()
    rng = np.random.default_rng(95)
    hk, hv, d = 2, 4, 128
    w = _weights(rng, hk, hv, d, d, 4)
    with pytest.raises(InvalidArg):
        rt.GdnLayer(dev, hk, hv, d, d, w[0][:-1], *w[1:])
    layer = rt.GdnLayer(dev, hk, hv, d, d, *w)
    qkv, z, br, ar = _inputs(rng, 3, hk, hv, d, d)
    with pytest.raises(InvalidArg):
        layer.forward(qkv[:, :-1].copy(), z, br, ar)
    with pytest.raises(InvalidArg):
        layer.forward(qkv, z[:2].copy(), br, ar)
    assert layer.forward(qkv[:0].copy(), z[:0].copy(), br[:0].copy(), ar[:0].copy()).shape == (0, hv, d)
    layer.close()


def test_gdn_layer_forward_dev_equals_host_slices():
    """pi_gdn_layer_forward_dev on device tensors gives pi_gdn_layer_forward's bits over a
    prompt, an odd and an even run of one-token steps (the one-launch step alternates two
    conv-state buffers) and continued chunks, so the two seams share every kernel and state."""
    import torch
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(97)
    hk, hv, d = 2, 4, 128
    w = _weights(rng, hk, hv, d, d, 4)
    host, devl = rt.GdnLayer(dev, hk, hv, d, d, *w), rt.GdnLayer(dev, hk, hv, d, d, *w)
    to_dev = lambda a: torch.from_numpy(a).to("cuda")  # noqa: E731
    for n in (33, 1, 1, 1, 7, 1, 1, 12):
        x = _inputs(rng, n, hk, hv, d, d)
        want = host.forward(*x)
        got = devl.forward_dev(*(to_dev(a) for a in x)).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n
    host.close()
    devl.close()


def test_gdn_layer_reset_orders_after_side_stream_steps():
    """Steps enqueued on a non-blocking torch side stream, then pi_gdn_layer_reset with no
    synchronisation in between: the reset waits for those steps before it zeroes the conv
    state (both of the one-token step's alternating buffers) and the recurrent state, so the
    steps that follow give a fresh layer's bits."""
    import torch
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(99)
    hk, hv, d = 2, 4, 128
    w = _weights(rng, hk, hv, d, d, 4)
    used, fresh = rt.GdnLayer(dev, hk, hv, d, d, *w), rt.GdnLayer(dev, hk, hv, d, d, *w)
    side = torch.cuda.Stream()
    before = [_inputs(rng, n, hk, hv, d, d) for n in (300, 1, 1, 1)]
    after = [_inputs(rng, n, hk, hv, d, d) for n in (1, 1, 20, 1)]
    with torch.cuda.stream(side):
        for x in before:
            used.forward_dev(*(torch.from_numpy(a).to("cuda", non_blocking=False) for a in x))
        used.reset()
        got = [used.forward_dev(*(torch.from_numpy(a).to("cuda") for a in x)) for x in after]
    side.synchronize()
    for x, g in zip(after, got):
        want = fresh.forward(*x)
        assert np.array_equal(g.cpu().numpy().view(np.uint32), want.view(np.uint32))
    used.close()
    fresh.close()

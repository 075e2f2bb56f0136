"""Host-slice drop-ins of src/ops.rs and the gated-delta step (pi_ops_* /
pi_ssm_gated_delta_step) against the oracle on seeded inputs."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import device

pytestmark = pytest.mark.gpu


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def test_rms_norm_any_length():
    dev = device()
    rng = np.random.default_rng(31)
    for n in (4, 128, 256, 1000, 4096):
        x = rng.standard_normal(n).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        out = np.zeros(n, np.float32)
        dev.check(dev.lib.pi_ops_rms_norm(dev.h, _p(out), _p(x), _p(w), n, 1e-6))
        np.testing.assert_allclose(out, orc.rms_norm(x, w, 1e-6), rtol=2e-6, atol=2e-6)


def test_softmax_rows():
    dev = device()
    rng = np.random.default_rng(32)
    for n in (1, 3, 1000, 65537):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        ref = orc.softmax(x)
        x64 = np.exp(x.astype(np.float64) - x.max())
        x64 /= x64.sum()
        dev.check(dev.lib.pi_ops_softmax(dev.h, _p(x), n))
        # the reference sums n values sequentially in f32 (src/ops.rs:171-174):
        # its result carries up to ~n * 2^-24 relative error; the GPU's tree
        # sum stays within 1e-5 of the float64 softmax
        np.testing.assert_allclose(x, x64, rtol=1e-5, atol=1e-12)
        np.testing.assert_allclose(x, ref, rtol=max(1e-5, 2 * n * 2.0 ** -24), atol=1e-12)
        assert abs(float(x.astype(np.float64).sum()) - 1.0) < 1e-5


@pytest.mark.parametrize("pos", [0, 1, 513, 32767, 65535])
def test_apply_rope_and_with_freqs(pos):
    dev = device()
    rng = np.random.default_rng(33 + pos)
    for hd, rd, base in ((128, 128, 1e6), (4, 4, 1e4), (128, 64, 1e4), (6, 8, 1e4)):
        q = rng.standard_normal(hd).astype(np.float32)
        k = rng.standard_normal(hd).astype(np.float32)
        rq, rk = orc.apply_rope(q, k, pos, hd, rd, base)
        dev.check(dev.lib.pi_ops_apply_rope(dev.h, _p(q), _p(k), pos, hd, rd, base))
        np.testing.assert_allclose(q, rq, rtol=0, atol=2e-5 * max(1, pos / 1000))
        np.testing.assert_allclose(k, rk, rtol=0, atol=2e-5 * max(1, pos / 1000))
    f = orc.compute_imrope_freqs(1e7, 64, [11, 11, 10, 0])
    q = rng.standard_normal(256).astype(np.float32)
    k = rng.standard_normal(256).astype(np.float32)
    rq, rk = orc.apply_rope_with_freqs(q, k, pos, 256, f)
    dev.check(dev.lib.pi_ops_apply_rope_with_freqs(dev.h, _p(q), _p(k), pos, 256, _p(f), f.size))
    np.testing.assert_allclose(q, rq, rtol=0, atol=2e-5 * max(1, pos / 1000))
    np.testing.assert_allclose(k, rk, rtol=0, atol=2e-5 * max(1, pos / 1000))


def test_gated_delta_step_host_slices_match_oracle():
    """Eight consecutive steps from a random state, Qwen3.5 shape (16 K / 32 V heads)."""
    dev = device()
    rng = np.random.default_rng(34)
    hk, hv, d = 16, 32, 128
    state = (rng.standard_normal((hv, d, d)) * 0.1).astype(np.float32)
    ref_state = state.copy()
    for step in range(8):
        q = rng.standard_normal((hk, d)).astype(np.float32)
        k = rng.standard_normal((hk, d)).astype(np.float32)
        v = rng.standard_normal((hv, d)).astype(np.float32)
        beta = (1 / (1 + np.exp(-rng.standard_normal(hv)))).astype(np.float32)
        g = (-np.log1p(np.exp(rng.standard_normal(hv)))).astype(np.float32)
        out = np.zeros((hv, d), np.float32)
        dev.check(dev.lib.pi_ssm_gated_delta_step(dev.h, _p(out), _p(state), _p(q), _p(k), _p(v),
                                                  _p(beta), _p(g), hk, hv, d, d))
        ref_out, ref_state = orc.gdn_tokens(q[None], k[None], v[None], beta[None], g[None],
                                            ref_state)
        assert np.abs(out - ref_out[0]).max() <= 2e-3
        assert np.abs(state - ref_state).max() <= 2e-3

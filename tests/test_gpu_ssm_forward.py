"""ssm::ssm_forward (src/ssm/mod.rs:40-157, the Mamba-2-style scan the reference keeps beside
the gated-DeltaNet path) on the device against the oracle's restatement: the state to
max-abs 1e-5 relative to its scale, y to 1e-4 relative to max |y| (the device sums the
projections in another order), over each of the reference's slice-length branches and
over three consecutive tokens carrying the state."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import device

pytestmark = pytest.mark.gpu


def _args(rng, d_inner, d_state, d_conv, branches):
    conv = (rng.standard_normal(d_inner * d_conv) * 0.5).astype(np.float32)
    a = (rng.standard_normal(d_state * d_inner) * 0.5).astype(np.float32)
    bias = rng.standard_normal(d_inner).astype(np.float32)
    alpha = (rng.standard_normal(d_inner * d_inner) / np.sqrt(d_inner)).astype(np.float32)
    beta = (rng.standard_normal(d_state * d_inner) / np.sqrt(d_inner)).astype(np.float32)
    out_w = (rng.standard_normal(d_inner * d_inner) / np.sqrt(d_inner)).astype(np.float32)
    if branches in ("no_conv", "none"):
        conv = conv[:3]
    if branches in ("no_b", "none"):
        beta = beta[:d_inner - 1]
    if branches in ("no_out", "none"):
        out_w = out_w[:0]
    return conv, a, bias, alpha, beta, out_w


@pytest.mark.parametrize("d_inner,d_state,d_conv,branches", [
    (4, 2, 4, "all"), (64, 16, 4, "all"), (300, 16, 4, "no_conv"), (1024, 16, 4, "no_b"),
    (129, 8, 3, "no_out"), (96, 4, 4, "none")])
def test_ssm_forward_matches_oracle(d_inner, d_state, d_conv, branches):
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(d_inner * 10 + d_state)
    args = _args(rng, d_inner, d_state, d_conv, branches)
    state = np.zeros(d_state * d_inner, np.float32)
    ref_state = state.copy()
    for step in range(3):
        x = rng.standard_normal(d_inner).astype(np.float32)
        y = rt.ssm_forward(dev, x, *args, state, d_inner, d_state, d_conv)
        ry, ref_state = orc.ssm_forward(x, *args, ref_state, d_inner, d_state, d_conv)
        ys = max(float(np.abs(ry).max()), 1e-6)
        ss = max(float(np.abs(ref_state).max()), 1e-6)
        assert np.abs(state - ref_state).max() <= 1e-5 * ss, (step, "state")
        assert np.abs(y - ry).max() <= 1e-4 * ys, (step, "y")


def test_ssm_forward_reference_tests_on_device():
    """src/ssm/mod.rs:176-231 through the device path."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    state = np.zeros(8, np.float32)
    y = rt.ssm_forward(dev, [1, 2, 3, 4], [0.1] * 16, [-0.5] * 8, [0.0] * 4, [0.1] * 16,
                       [0.1] * 8, [0.1] * 16, state, 4, 2, 4)
    assert y.shape == (4,) and np.isfinite(y).all() and (state != 0).any()
    state = np.zeros(32, np.float32)
    args = ([0.2] * 32, [-1.0] * 32, [0.5] * 8, [0.1] * 64, [0.1] * 32, [0.05] * 64)
    y1 = rt.ssm_forward(dev, [1.0] * 8, *args, state, 8, 4, 4)
    y2 = rt.ssm_forward(dev, [2.0] * 8, *args, state, 8, 4, 4)
    assert not np.array_equal(y1, y2)


def test_ssm_forward_rejects_short_slices():
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    with pytest.raises(rt.InvalidArg):
        rt.ssm_forward(dev, [1.0] * 4, [], [0.0] * 7, [0.0] * 4, [0.0] * 16, [], [],
                       np.zeros(8, np.float32), 4, 2, 4)

"""Head widths beyond the common equal-width 128 case (src/model/mod.rs:976-982: query, key
and value heads may have different widths; ops::attention_head takes any head_dim).

- the f32 KV pool at head_dim 256 (decode against the oracle, max-abs 2e-3);
- ops::attention_head (src/ops.rs:213-247) with head_dim 129..256 (padded to a kernel width);
- the LayerCache attention step with q_head_dim > head_dim and v_head_dim below and above
  head_dim, and with key head widths that are no kernel width (33, 48, 80, 96, 160, 192,
  200: run zero-padded to the next of 64 / 128 / 256), through the host and the device-pointer entries, against or_attn_layer_tokens
  (which carries the three widths as the reference does): max-abs 2e-3 with an f32 cache,
  per-row relative 1e-2 with an f16 cache; q comes back normalised and rotated in its first
  head_dim dims and untouched past them.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import PagedCase, device, row_rel_err, to_dev

pytestmark = pytest.mark.gpu


def test_decode_f32_pool_d256_gated():
    """16/2 heads at D 256 over an f32 cache, IMRoPE, a gate, ragged lengths."""
    dev = device()
    rng = np.random.default_rng(0xD256)
    lens = [1500, 1, 257, 0]
    case = PagedCase(rng, lens, 16, 2, 256, theta=1e7, rope_dim=64, sections=[11, 11, 10, 0])
    case.gpu_build(dev, torch.float32)
    gate = rng.standard_normal((len(lens), 16, 256)).astype(np.float32)
    out = case.gpu_decode(dev, gate=gate)
    for i in range(len(lens)):
        ref = case.oracle_out(i, gate=gate[i])
        if lens[i] == 0:
            ref = np.zeros_like(ref)
        err = float(np.abs(out[i] - ref).max())
        assert err <= 2e-3, f"seq {i} (L={lens[i]}): max-abs {err}"


@pytest.mark.parametrize("d,t", [(129, 40), (200, 333), (256, 1000)])
def test_attention_head_wide(d, t):
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(d)
    q = rng.standard_normal(d).astype(np.float32)
    k = rng.standard_normal((t, d)).astype(np.float32)
    v = rng.standard_normal((t, d)).astype(np.float32)
    out = rt.attention_head(dev, q, k, v, t, d)
    assert np.abs(out - orc.attention_head(q, k, v, t, d)).max() <= 2e-3


WIDTHS = [
    # (q_head_dim, head_dim, v_head_dim, cache dtype, gate)
    (256, 128, 128, torch.float16, True),
    (128, 128, 64, torch.float32, False),
    (128, 128, 200, torch.float16, True),
    (320, 256, 96, torch.float16, True),
    (96, 64, 100, torch.float32, True),
]


def _inputs(rng, n, hq, hkv, dq, dk, dv, gated):
    q = rng.standard_normal((n, hq, dq)).astype(np.float32)
    k = rng.standard_normal((n, hkv, dk)).astype(np.float32)
    v = rng.standard_normal((n, hkv, dv)).astype(np.float32)
    g = rng.standard_normal((n, hq, dq)).astype(np.float32) if gated else None
    return q, k, v, g


@pytest.mark.parametrize("dq,dk,dv,dtype,gated", WIDTHS)
def test_layer_distinct_widths(dq, dk, dv, dtype, gated):
    """A 90-token prompt, two decode tokens and a 17-token continued chunk, 8/2 heads with
    Q/K RMSNorm and NORM RoPE."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(dq * 7 + dk * 3 + dv)
    hq, hkv, eps, base = 8, 2, 1e-6, 1e6
    qn = rng.uniform(0.5, 1.5, dk).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, dk).astype(np.float32)
    layer = rt.AttnLayer(dev, 256, hq, hkv, dk, dtype, q_norm_w=qn, k_norm_w=kn, eps=eps,
                         rope_base=base, q_head_dim=dq, v_head_dim=dv)
    kw = dict(q_norm_w=qn, k_norm_w=kn, eps=eps, rope_base=base)
    kc = vc = None
    prev = 0
    for n in (90, 1, 1, 17):
        q, k, v, g = _inputs(rng, n, hq, hkv, dq, dk, dv, gated)
        ref, kc, vc = orc.attn_layer_tokens(q, k, v, gate=g, key_cache=kc, value_cache=vc,
                                            prev_seq_len=prev, **kw)
        qr, kr = orc.attn_prepare(q, k, hq, hkv, dk, pos0=prev, q_head_dim=dq, **kw)
        qg, kg = q.copy(), k.copy()
        out = layer.forward(qg, kg, v, gate=g)
        assert out.shape == (n, hq, dk)
        if dtype == torch.float32:
            err = float(np.abs(out - ref).max())
            assert err <= 2e-3, f"chunk {n} at {prev}: max-abs {err}"
        else:
            for i in range(n):
                err = row_rel_err(out[i], ref[i])
                assert err <= 1e-2, f"chunk {n} at {prev}: token {i} rel err {err}"
        if dv < dk:  # output dims past the value width stay zero
            assert not out[:, :, dv:].any()
        assert np.abs(qg - qr).max() <= 1e-5 and np.abs(kg - kr).max() <= 1e-5
        np.testing.assert_array_equal(qg[:, :, dk:], q[:, :, dk:])
        prev += n
        assert layer.seq_len == prev


@pytest.mark.parametrize("dq,dk,dv,dtype,gated", [WIDTHS[0], WIDTHS[1], WIDTHS[3]])
def test_layer_distinct_widths_device_entry(dq, dk, dv, dtype, gated):
    """pi_attn_layer_forward_dev with distinct widths gives pi_attn_layer_forward's bits
    (outputs, and q / k written back) over a prompt, a decode token and a chunk."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(0xDE7 + dq + dv)
    hq, hkv = 8, 2
    qn = rng.uniform(0.5, 1.5, dk).astype(np.float32)
    mk = lambda: rt.AttnLayer(dev, 160, hq, hkv, dk, dtype, q_norm_w=qn, rope_base=1e4,  # noqa: E731
                              q_head_dim=dq, v_head_dim=dv)
    host, devl = mk(), mk()
    for n in (70, 1, 9):
        q, k, v, g = _inputs(rng, n, hq, hkv, dq, dk, dv, gated)
        qh, kh = q.copy(), k.copy()
        out_h = host.forward(qh, kh, v, gate=g)
        tq, tk = to_dev(q), to_dev(k)
        out_d = devl.forward_dev(tq, tk, to_dev(v), gate=None if g is None else to_dev(g))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out_d.cpu().numpy(), out_h)
        np.testing.assert_array_equal(tq.cpu().numpy(), qh)
        np.testing.assert_array_equal(tk.cpu().numpy(), kh)


PADDED = [
    # (q_head_dim, head_dim, v_head_dim, cache dtype, gate, rope_dim): key heads that are no
    # kernel width run zero-padded to the next of 64 / 128 / 256
    (80, 80, 80, torch.float16, True, None),
    (96, 96, 96, torch.float32, False, 32),
    (64, 48, 40, torch.float16, True, None),
    (160, 160, 160, torch.float16, False, 64),
    (192, 192, 192, torch.float32, True, None),
    (33, 33, 33, torch.float16, True, None),
    (256, 200, 224, torch.float16, True, None),
]


@pytest.mark.parametrize("dq,dk,dv,dtype,gated,rope_dim", PADDED)
def test_layer_padded_head_dim(dq, dk, dv, dtype, gated, rope_dim):
    """A 150-token prompt, two decode tokens and a 40-token continued chunk, 8/2 heads with
    Q/K RMSNorm over head_dim (not the padded width), NORM RoPE over rope_dim (an odd
    head_dim leaves its last dim unrotated) and scale 1/sqrt(head_dim)."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(dq * 11 + dk * 5 + dv)
    hq, hkv, eps, base = 8, 2, 1e-6, 1e6
    qn = rng.uniform(0.5, 1.5, dk).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, dk).astype(np.float32)
    layer = rt.AttnLayer(dev, 256, hq, hkv, dk, dtype, q_norm_w=qn, k_norm_w=kn, eps=eps,
                         rope_base=base, rope_dim=rope_dim, q_head_dim=dq, v_head_dim=dv)
    kw = dict(q_norm_w=qn, k_norm_w=kn, eps=eps, rope_base=base,
              rope_dim=dk if rope_dim is None else rope_dim)
    kc = vc = None
    prev = 0
    for n in (150, 1, 1, 40):
        q, k, v, g = _inputs(rng, n, hq, hkv, dq, dk, dv, gated)
        ref, kc, vc = orc.attn_layer_tokens(q, k, v, gate=g, key_cache=kc, value_cache=vc,
                                            prev_seq_len=prev, **kw)
        qr, kr = orc.attn_prepare(q, k, hq, hkv, dk, pos0=prev, q_head_dim=dq, **kw)
        qg, kg = q.copy(), k.copy()
        out = layer.forward(qg, kg, v, gate=g)
        assert out.shape == (n, hq, dk)
        if dtype == torch.float32:
            err = float(np.abs(out - ref).max())
            assert err <= 2e-3, f"chunk {n} at {prev}: max-abs {err}"
        else:
            for i in range(n):
                err = row_rel_err(out[i], ref[i])
                assert err <= 1e-2, f"chunk {n} at {prev}: token {i} rel err {err}"
        if dv < dk:
            assert not out[:, :, dv:].any()
        assert np.abs(qg - qr).max() <= 1e-5 and np.abs(kg - kr).max() <= 1e-5
        np.testing.assert_array_equal(qg[:, :, dk:], q[:, :, dk:])
        prev += n
        assert layer.seq_len == prev


@pytest.mark.parametrize("dq,dk,dv,dtype,gated,rope_dim", [PADDED[0], PADDED[2], PADDED[4]])
def test_layer_padded_head_dim_device_entry(dq, dk, dv, dtype, gated, rope_dim):
    """pi_attn_layer_forward_dev at a padded head_dim gives pi_attn_layer_forward's bits
    (outputs, and q / k written back) over a prompt, a decode token and a chunk."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(0xAD + dq + dk + dv)
    hq, hkv = 8, 2
    kn = rng.uniform(0.5, 1.5, dk).astype(np.float32)
    mk = lambda: rt.AttnLayer(dev, 160, hq, hkv, dk, dtype, k_norm_w=kn, rope_base=1e4,  # noqa: E731
                              rope_dim=rope_dim, q_head_dim=dq, v_head_dim=dv)
    host, devl = mk(), mk()
    for n in (70, 1, 9):
        q, k, v, g = _inputs(rng, n, hq, hkv, dq, dk, dv, gated)
        qh, kh = q.copy(), k.copy()
        out_h = host.forward(qh, kh, v, gate=g)
        tq, tk = to_dev(q), to_dev(k)
        out_d = devl.forward_dev(tq, tk, to_dev(v), gate=None if g is None else to_dev(g))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out_d.cpu().numpy(), out_h)
        np.testing.assert_array_equal(tq.cpu().numpy(), qh)
        np.testing.assert_array_equal(tk.cpu().numpy(), kh)


def test_layer_rejects_head_dim_past_256():
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    with pytest.raises(rt.Unsupported):
        rt.AttnLayer(dev, 16, 4, 2, 320, torch.float16)


def test_layer_rejects_narrow_query_heads():
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    with pytest.raises(rt.InvalidArg):
        rt.AttnLayer(dev, 16, 4, 2, 128, torch.float16, q_head_dim=64)

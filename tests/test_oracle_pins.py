"""Pins the CPU oracle before it is trusted as the GPU path's checker.

Each test checks one oracle function against (a) the known-answer vectors the
reference's own tests hold (tests/golden/kat.json), (b) closed forms and
invariants, or (c) float64 brute force from the textbook formula
(tests/ref64.py).  The "mistake" tests show that a plausible slip (grouped
instead of modulo GQA, NeoX instead of adjacent RoPE pairs, attend-then-append)
fails the corresponding pin.
"""
import json
import math
import os

import numpy as np
import pytest

from tests import ref64

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))


# ---- src/simd.rs ------------------------------------------------------------

def test_dot_product_kat(orc):
    for case in KAT["dot_product"]:
        assert orc.dot_product(case["a"], case["b"]) == case["expected"]


def test_sum_squares_and_scale_kat(orc):
    for case in KAT["sum_squares"]:
        assert orc.sum_squares(case["a"]) == case["expected"]
    for case in KAT["scale"]:
        np.testing.assert_array_equal(orc.scale(case["a"], case["s"]), case["expected"])


def test_dot_product_lane_order(orc):
    # The SSE reduction order is (l0+l1)+(l2+l3) over 4 lane partials, then the tail.
    # With values chosen so that f32 rounding depends on the order, only that order
    # reproduces the result computed here step by step in float32.
    a = np.array([1e8, 1, -1e8, 1, 3, 5, 7, 11, 0.5], dtype=np.float32)
    b = np.ones_like(a)
    f = np.float32
    lanes = [f(a[0]) + f(a[4]), f(a[1]) + f(a[5]), f(a[2]) + f(a[6]), f(a[3]) + f(a[7])]
    expect = f(f(lanes[0] + lanes[1]) + f(lanes[2] + lanes[3])) + f(a[8])
    assert orc.dot_product(a, b) == expect
    seq = f(0)
    for x in a:
        seq = f(seq + x)
    assert seq != expect  # a sequential sum would be a different (wrong) oracle


# ---- src/ops.rs -------------------------------------------------------------

def test_rms_norm_kat(orc):
    for case in KAT["rms_norm"]:
        np.testing.assert_allclose(orc.rms_norm(case["x"], case["w"], case["eps"]),
                                   case["expected"], rtol=1e-6)


def test_rms_norm_random_f64(orc):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(256).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    np.testing.assert_allclose(orc.rms_norm(x, w, 1e-6), ref64.rms_norm(x, w, 1e-6), rtol=2e-6,
                               atol=1e-7)


def test_softmax_kat_and_invariants(orc):
    for case in KAT["softmax"]:
        np.testing.assert_allclose(orc.softmax(case["x"]), case["expected"], rtol=1e-6)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(1000).astype(np.float32) * 5
    s = orc.softmax(x)
    assert abs(s.sum(dtype=np.float64) - 1) < 1e-5
    np.testing.assert_allclose(orc.softmax(x + np.float32(3.0)), s, rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(s, ref64.softmax(x), rtol=1e-5, atol=1e-9)
    assert orc.softmax(np.zeros(0, np.float32)).size == 0


def test_rope_pos0_identity_kat(orc):
    for case in KAT["rope_pos0"]:
        q, k = orc.apply_rope(case["q"], case["k"], 0, case["head_dim"], case["rope_dim"],
                              case["base"])
        np.testing.assert_array_equal(q, case["q"])
        np.testing.assert_array_equal(k, case["k"])


@pytest.mark.parametrize("pos", [1, 7, 513, 32767])
def test_rope_adjacent_pairs_f64(orc, pos):
    rng = np.random.default_rng(pos)
    q = rng.standard_normal(128).astype(np.float32)
    k = rng.standard_normal(128).astype(np.float32)
    rq, rk = orc.apply_rope(q, k, pos, 128, 128, 1e6)
    # f32 angle pos*freq has granularity ~pos*6e-8 rad; scale the tolerance with pos.
    tol = 1e-5 + 4 * pos * 6e-8
    np.testing.assert_allclose(rq, ref64.rope_adjacent(q, pos, 128, 1e6), atol=tol * 4)
    np.testing.assert_allclose(rk, ref64.rope_adjacent(k, pos, 128, 1e6), atol=tol * 4)
    # rotation preserves each pair's norm
    np.testing.assert_allclose(np.hypot(rq[0::2], rq[1::2]), np.hypot(q[0::2], q[1::2]),
                               rtol=1e-5)


def test_rope_mistake_neox_pairing_detected(orc):
    rng = np.random.default_rng(3)
    q = rng.standard_normal(128).astype(np.float32)
    rq, _ = orc.apply_rope(q, q, 9, 128, 128, 1e4)
    assert np.abs(rq - ref64.rope_neox(q, 9, 128, 1e4)).max() > 0.1


def test_rope_relative_position(orc):
    rng = np.random.default_rng(4)
    q = rng.standard_normal(64).astype(np.float32)
    k = rng.standard_normal(64).astype(np.float32)
    d = []
    for m, n in [(10, 3), (110, 103), (1010, 1003)]:
        qm, _ = orc.apply_rope(q, q, m, 64, 64, 1e4)
        _, kn = orc.apply_rope(k, k, n, 64, 64, 1e4)
        d.append(float(np.dot(qm.astype(np.float64), kn)))
    assert max(d) - min(d) < 1e-3


def test_rope_partial_dims_untouched(orc):
    rng = np.random.default_rng(5)
    q = rng.standard_normal(256).astype(np.float32)
    rq, _ = orc.apply_rope(q, q, 77, 256, 64, 1e4)
    np.testing.assert_array_equal(rq[64:], q[64:])


def test_imrope_freqs_closed_form(orc):
    f = orc.compute_imrope_freqs(1e7, 64, [11, 11, 10, 0])
    assert f.shape == (32,) and f[0] == 1.0
    expect = np.array([1e7 ** (-2.0 * i / 64) for i in range(32)])
    np.testing.assert_allclose(f, expect, rtol=2e-6)
    # all four tracks advance together, so sections do not change the values
    np.testing.assert_array_equal(orc.compute_imrope_freqs(1e7, 64, [1, 0, 5, 2]), f)


@pytest.mark.parametrize("pos", [0, 5, 65535])
def test_rope_with_freqs_neox_f64(orc, pos):
    rng = np.random.default_rng(6)
    q = rng.standard_normal(256).astype(np.float32)
    k = rng.standard_normal(256).astype(np.float32)
    f = orc.compute_imrope_freqs(1e7, 64, [11, 11, 10, 0])
    rq, rk = orc.apply_rope_with_freqs(q, k, pos, 256, f)
    tol = 1e-5 + 8 * pos * 6e-8
    np.testing.assert_allclose(rq, ref64.rope_neox(q, pos, 64, 1e7), atol=tol * 4)
    np.testing.assert_allclose(rk, ref64.rope_neox(k, pos, 64, 1e7), atol=tol * 4)
    np.testing.assert_array_equal(rq[64:], q[64:])


def test_attention_head_kat(orc):
    for case in KAT["attention_head"]:
        q = np.array(case["q"], np.float32)
        k = np.array(case["k"], np.float32)
        v = np.array(case["v"], np.float32)
        out = orc.attention_head(q, k.ravel(), v.ravel(), k.shape[0], q.size)
        np.testing.assert_allclose(out, case["expected"], rtol=2e-6, atol=2e-6)


def test_attention_closed_forms(orc):
    rng = np.random.default_rng(7)
    d = 128
    v = rng.standard_normal((5, d)).astype(np.float32)
    k = rng.standard_normal((5, d)).astype(np.float32)
    # one key -> out = its value
    np.testing.assert_allclose(orc.attention_head(rng.standard_normal(d), k[:1], v[:1], 1, d),
                               v[0], rtol=1e-6)
    # q = 0 -> mean of V
    np.testing.assert_allclose(orc.attention_head(np.zeros(d), k, v, 5, d), v.mean(0),
                               atol=1e-6)
    # a dominant key -> ~ its value
    kd = k.copy()
    kd[2] = 100 * np.ones(d)
    np.testing.assert_allclose(orc.attention_head(np.ones(d), kd, v, 5, d), v[2], atol=1e-5)
    # permuting keys with their values leaves the output unchanged
    q = rng.standard_normal(d)
    perm = rng.permutation(5)
    np.testing.assert_allclose(orc.attention_head(q, k[perm], v[perm], 5, d),
                               orc.attention_head(q, k, v, 5, d), rtol=1e-5, atol=1e-6)


# ---- src/model/mod.rs attention core ---------------------------------------

def test_attn_decode_modulo_gqa_f64(orc):
    rng = np.random.default_rng(8)
    hq, hkv, d, t = 8, 2, 64, 37
    q = rng.standard_normal((hq, d)).astype(np.float32)
    k = rng.standard_normal((t, hkv, d)).astype(np.float32)
    v = rng.standard_normal((t, hkv, d)).astype(np.float32)
    out = orc.attn_decode(q, k, v)
    np.testing.assert_allclose(out, ref64.attention(q, k, v, lambda h: h % hkv), atol=2e-6)
    grouped = ref64.attention(q, k, v, lambda h: h // (hq // hkv))
    assert np.abs(out - grouped).max() > 0.05  # a grouped mapping is a detectable mistake


def test_attn_decode_matches_attention_head(orc):
    rng = np.random.default_rng(9)
    t, d = 19, 128
    q = rng.standard_normal((1, d)).astype(np.float32)
    k = rng.standard_normal((t, 1, d)).astype(np.float32)
    v = rng.standard_normal((t, 1, d)).astype(np.float32)
    a = orc.attn_decode(q, k, v)[0]
    b = orc.attention_head(q[0], k[:, 0], v[:, 0], t, d)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


def test_gate_closed_form(orc):
    rng = np.random.default_rng(10)
    o = rng.standard_normal(300).astype(np.float32)
    g = rng.standard_normal(300).astype(np.float32)
    np.testing.assert_allclose(orc.apply_gate(o, g), o / (1 + np.exp(-g.astype(np.float64))),
                               rtol=1e-6, atol=1e-7)


def _layer_f64(q, k, v, prev_k, prev_v, pos0, rope, qn=None, kn=None, gate=None, eps=1e-6):
    """Causal attention of n new tokens over prev + new keys, float64, modulo GQA."""
    n, hq, d = q.shape
    hkv = k.shape[1]
    if qn is not None:
        q = ref64.rms_norm(q, qn, eps)
    if kn is not None:
        k = ref64.rms_norm(k, kn, eps)
    qr = np.stack([rope(q[i], pos0 + i) for i in range(n)])
    kr = np.stack([rope(k[i], pos0 + i) for i in range(n)])
    K = np.concatenate([prev_k, kr]) if prev_k is not None else kr
    V = np.concatenate([prev_v, v]) if prev_v is not None else np.asarray(v, np.float64)
    out = np.stack([ref64.attention(qr[i], K[:pos0 + i + 1], V[:pos0 + i + 1],
                                    lambda h: h % hkv) for i in range(n)])
    if gate is not None:
        out = out / (1 + np.exp(-np.asarray(gate, np.float64)))
    return out, kr


def test_attn_layer_prefill_causal_f64(orc):
    rng = np.random.default_rng(11)
    n, hq, hkv, d = 12, 4, 2, 32
    q = rng.standard_normal((n, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    out, kc, vc = orc.attn_layer_tokens(q, k, v, rope_base=1e4)
    exp, kr = _layer_f64(q, k, v, None, None, 0, lambda x, p: ref64.rope_adjacent(x, p, d, 1e4))
    np.testing.assert_allclose(out, exp, atol=2e-5)
    np.testing.assert_allclose(kc, kr, atol=2e-5)  # cache holds rotated K
    np.testing.assert_array_equal(vc, v)


def test_attn_layer_mistake_attend_then_append_detected(orc):
    rng = np.random.default_rng(12)
    n, hq, hkv, d = 6, 2, 2, 16
    q = rng.standard_normal((n, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    out, _, _ = orc.attn_layer_tokens(q, k, v, rope_base=1e4)
    rope = lambda x, p: ref64.rope_adjacent(x, p, d, 1e4)
    qr = np.stack([rope(q[i], i) for i in range(n)])
    kr = np.stack([rope(k[i], i) for i in range(n)])
    # attending only to strictly earlier keys (row 0 has none, skip it)
    wrong = np.stack([ref64.attention(qr[i], kr[:i], v[:i], lambda h: h % hkv)
                      for i in range(1, n)])
    assert np.abs(out[1:] - wrong).max() > 0.05


def test_attn_layer_qk_norm_imrope_gate_f64(orc):
    rng = np.random.default_rng(13)
    n, hq, hkv, d, prev = 3, 4, 2, 256, 5
    q = rng.standard_normal((n, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    gate = rng.standard_normal((n, hq, d)).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, d).astype(np.float32)
    pk = rng.standard_normal((prev, hkv, d)).astype(np.float32)
    pv = rng.standard_normal((prev, hkv, d)).astype(np.float32)
    freqs = orc.compute_imrope_freqs(1e7, 64, [11, 11, 10, 0])
    out, kc, _ = orc.attn_layer_tokens(q, k, v, gate=gate, q_norm_w=qn, k_norm_w=kn, eps=1e-6,
                                       rope_dim=64, rope_base=1e7, freqs=freqs,
                                       key_cache=pk, value_cache=pv, prev_seq_len=prev)
    exp, kr = _layer_f64(q, k, v, pk, pv, prev, lambda x, p: ref64.rope_neox(x, p, 64, 1e7),
                         qn=qn, kn=kn, gate=gate)
    np.testing.assert_allclose(out, exp, atol=5e-5)
    np.testing.assert_allclose(kc[prev:], kr, atol=5e-5)


@pytest.mark.parametrize("dq,dk,dv", [(48, 32, 32), (32, 32, 20), (40, 32, 44)])
def test_attn_layer_distinct_head_widths_f64(orc, dq, dk, dv):
    """Query, key and value heads of different widths (src/model/mod.rs:976-982, 1035-1196):
    the Q norm and RoPE touch the first dk dims of a query head and attention reads only
    those; output dims at or past dv stay zero and value dims past dk are not read; the gate
    is the flat prefix of hq * dk values of each token's hq * dq."""
    rng = np.random.default_rng(dq * 1000 + dv)
    n, hq, hkv, eps = 5, 4, 2, 1e-6
    q = rng.standard_normal((n, hq, dq)).astype(np.float32)
    k = rng.standard_normal((n, hkv, dk)).astype(np.float32)
    v = rng.standard_normal((n, hkv, dv)).astype(np.float32)
    gate = rng.standard_normal((n, hq, dq)).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, dk).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, dk).astype(np.float32)
    out, kc, vc = orc.attn_layer_tokens(q, k, v, gate=gate, q_norm_w=qn, k_norm_w=kn, eps=eps,
                                        rope_base=1e4)
    assert out.shape == (n, hq, dk) and vc.shape == (n, hkv, dv)
    qr = ref64.rms_norm(q[:, :, :dk], qn, eps)
    kr = ref64.rms_norm(k, kn, eps)
    qr = np.stack([ref64.rope_adjacent(qr[i], i, dk, 1e4) for i in range(n)])
    kr = np.stack([ref64.rope_adjacent(kr[i], i, dk, 1e4) for i in range(n)])
    m = min(dk, dv)
    exp = np.zeros((n, hq, dk))
    for i in range(n):
        exp[i, :, :m] = ref64.attention(qr[i], kr[:i + 1], v[:i + 1, :, :m], lambda h: h % hkv)
    g = gate.reshape(n, hq * dq)[:, :hq * dk].reshape(n, hq, dk).astype(np.float64)
    exp = exp / (1 + np.exp(-g))
    np.testing.assert_allclose(out, exp, atol=2e-5)
    assert not out[:, :, m:].any()
    np.testing.assert_allclose(kc, kr, atol=2e-5)
    # the Q dims past dk are neither normalised, rotated nor read
    qq, _ = orc.attn_prepare(q, None, hq, hkv, dk, q_norm_w=qn, eps=eps, rope_base=1e4,
                             q_head_dim=dq)
    np.testing.assert_allclose(qq[:, :, :dk], qr, atol=2e-5)
    np.testing.assert_array_equal(qq[:, :, dk:], q[:, :, dk:])
    q2 = q.copy()
    q2[:, :, dk:] = rng.standard_normal(q2[:, :, dk:].shape)
    out2, _, _ = orc.attn_layer_tokens(q2, k, v, gate=gate, q_norm_w=qn, k_norm_w=kn, eps=eps,
                                       rope_base=1e4)
    np.testing.assert_array_equal(out, out2)


# ---- src/model/mod.rs gated-DeltaNet ---------------------------------------

def test_gdn_gates_closed_form(orc):
    br = np.array([-3, 0, 2.5, 9], np.float32)
    ar = np.array([-1, 0.5, 9.5, 30], np.float32)
    sa = np.array([-0.5, -1, -2, -0.1], np.float32)
    db = np.array([0.2, 0.1, 0.6, 1.0], np.float32)
    beta, g = orc.gdn_gates(br, ar, sa, db)
    np.testing.assert_allclose(beta, 1 / (1 + np.exp(-br.astype(np.float64))), rtol=1e-6)
    x = (ar + db).astype(np.float64)
    sp = np.where(x > 10, x, np.log1p(np.exp(x)))
    np.testing.assert_allclose(g, sa * sp, rtol=1e-5)
    assert g[3] == sa[3] * np.float32(ar[3] + db[3])  # identity branch above 10


def test_gdn_zero_state_kat(orc):
    case = KAT["gdn_zero_state"][0]
    q = np.array(case["q"], np.float32)[None]
    k = np.array(case["k"], np.float32)[None]
    v = np.array(case["v"], np.float32)[None]
    beta = np.array(case["beta"], np.float32)[None]
    g = np.array(case["g"], np.float32)[None]
    out, _ = orc.gdn_tokens(q, k, v, beta, g)
    np.testing.assert_allclose(out[0], case["expected"], rtol=1e-5, atol=1e-6)


def _gdn_inputs(rng, t, hk, hv, dk, dv):
    q = rng.standard_normal((t, hk, dk)).astype(np.float32)
    k = rng.standard_normal((t, hk, dk)).astype(np.float32)
    v = rng.standard_normal((t, hv, dv)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((t, hv))))).astype(np.float32)
    g = (-np.log1p(np.exp(rng.standard_normal((t, hv))))).astype(np.float32)
    return q, k, v, beta, g


def test_gdn_beta_zero_is_pure_decay(orc):
    rng = np.random.default_rng(14)
    q, k, v, _, g = _gdn_inputs(rng, 1, 2, 4, 16, 8)
    s0 = rng.standard_normal((4, 16, 8)).astype(np.float32)
    out, s1 = orc.gdn_tokens(q, k, v, np.zeros((1, 4), np.float32), g, state=s0)
    np.testing.assert_allclose(s1, s0 * np.exp(g[0])[:, None, None], rtol=1e-6)
    qp, _ = ref64.gdn_prepare(q[0], k[0], 4)
    np.testing.assert_allclose(out[0], np.einsum("hkv,hk->hv", s1.astype(np.float64), qp),
                               atol=1e-5)


def test_gdn_strong_decay_resets(orc):
    rng = np.random.default_rng(15)
    q, k, v, beta, _ = _gdn_inputs(rng, 4, 2, 4, 16, 8)
    g = np.full((4, 4), -1e4, np.float32)
    out, _ = orc.gdn_tokens(q, k, v, beta, g)
    for t in range(4):
        qp, kp = ref64.gdn_prepare(q[t], k[t], 4)
        exp = beta[t][:, None] * (qp * kp).sum(-1)[:, None] * v[t]
        np.testing.assert_allclose(out[t], exp, rtol=1e-5, atol=1e-6)


def test_gdn_sequential_equals_chunked_wy_f64(orc):
    rng = np.random.default_rng(16)
    t, hk, hv, dk, dv = 48, 2, 4, 32, 16
    q, k, v, beta, g = _gdn_inputs(rng, t, hk, hv, dk, dv)
    s0 = (0.1 * rng.standard_normal((hv, dk, dv))).astype(np.float32)
    out, s_end = orc.gdn_tokens(q, k, v, beta, g, state=s0)
    qp, kp = ref64.gdn_prepare(q, k, hv)
    for h in range(hv):
        S = s0[h].astype(np.float64)
        for c0 in range(0, t, 16):
            sl = slice(c0, c0 + 16)
            O, S = ref64.gdn_chunk_wy(qp[sl, h], kp[sl, h], v[sl, h], beta[sl, h], g[sl, h], S)
            np.testing.assert_allclose(out[sl, h], O, atol=2e-5)
        np.testing.assert_allclose(s_end[h], S, atol=2e-5)


def test_gdn_mistake_readout_before_update_detected(orc):
    rng = np.random.default_rng(17)
    q, k, v, beta, g = _gdn_inputs(rng, 1, 1, 1, 8, 8)
    out, s1 = orc.gdn_tokens(q, k, v, beta, g)
    qp, _ = ref64.gdn_prepare(q[0], k[0], 1)
    # reading out from the state before the update gives zeros from a zero state
    assert np.abs(out[0]).max() > 1e-3
    np.testing.assert_allclose(out[0, 0], s1[0].T.astype(np.float64) @ qp[0], atol=1e-6)


# ---- src/ssm/mod.rs ssm_forward ------------------------------------------------

def test_ssm_forward_reference_tests(orc):
    """The reference's own tests (src/ssm/mod.rs:176-231): finite outputs, the state moves
    off zero, and a second input gives a different output from the carried state."""
    d_inner, d_state, d_conv = 4, 2, 4
    y, st = orc.ssm_forward([1, 2, 3, 4], [0.1] * 16, [-0.5] * 8, [0.0] * 4, [0.1] * 16,
                            [0.1] * 8, [0.1] * 16, np.zeros(8), d_inner, d_state, d_conv)
    assert y.shape == (4,) and np.isfinite(y).all() and (st != 0).any()
    d_inner, d_state = 8, 4
    args = ([0.2] * 32, [-1.0] * 32, [0.5] * 8, [0.1] * 64, [0.1] * 32, [0.05] * 64)
    y1, st = orc.ssm_forward([1.0] * 8, *args, np.zeros(32), d_inner, d_state, d_conv)
    y2, _ = orc.ssm_forward([2.0] * 8, *args, st, d_inner, d_state, d_conv)
    assert not np.array_equal(y1, y2)


@pytest.mark.parametrize("branches", ["all", "no_conv", "no_b", "no_out", "none"])
def test_ssm_forward_f64(orc, branches):
    """Random inputs through each slice-length branch against the float64 matrix form."""
    rng = np.random.default_rng(len(branches))
    d_inner, d_state, d_conv = 24, 5, 4
    x = rng.standard_normal(d_inner)
    conv = rng.standard_normal(d_inner * d_conv) * 0.5
    a = rng.standard_normal(d_state * d_inner) * 0.5
    bias = rng.standard_normal(d_inner)
    alpha = rng.standard_normal(d_inner * d_inner) * 0.3
    beta = rng.standard_normal(d_state * d_inner) * 0.3
    out_w = rng.standard_normal(d_inner * d_inner) * 0.3
    st0 = rng.standard_normal(d_state * d_inner)
    if branches in ("no_conv", "none"):
        conv = conv[:-1]
    if branches in ("no_b", "none"):
        beta = beta[:d_inner]
    if branches in ("no_out", "none"):
        out_w = out_w[:5]
    x, conv, a, bias, alpha, beta, out_w, st0 = (np.asarray(v, np.float32) for v in
                                                 (x, conv, a, bias, alpha, beta, out_w, st0))
    y, st = orc.ssm_forward(x, conv, a, bias, alpha, beta, out_w, st0, d_inner, d_state, d_conv)
    ey, est = ref64.ssm_forward(x, conv, a, bias, alpha, beta, out_w, st0, d_inner, d_state, d_conv)
    np.testing.assert_allclose(st, est, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(y, ey, rtol=1e-4, atol=1e-4 * np.abs(ey).max())


def test_ssm_forward_closed_form(orc):
    """alpha = 0, A = 0, no conv taps, no B, no output projection: dt = softplus(bias) (0 under
    -20, bias over 20), S' = exp(-dt) S + dt x^2, y = column sums."""
    d_inner, d_state = 4, 2
    x = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    bias = np.array([0.3, -25.0, 25.0, -1.0], np.float32)
    st0 = np.array([1, 2, 3, 4, -1, 0.5, 0.25, 2], np.float32)
    y, st = orc.ssm_forward(x, [], np.zeros(8), bias, np.zeros(16), [], [], st0, d_inner, d_state, 3)
    dt = np.array([np.log1p(np.exp(0.3)), 0.0, 25.0, np.log1p(np.exp(-1.0))])
    S = np.exp(-dt) * st0.reshape(2, 4).astype(np.float64) + dt * x.astype(np.float64) ** 2
    np.testing.assert_allclose(st, S.reshape(-1), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(y, S.sum(axis=0), rtol=1e-6, atol=1e-6)


def test_rmsnorm_gated_closed_form(orc):
    rng = np.random.default_rng(18)
    o = rng.standard_normal((4, 128)).astype(np.float32)
    z = rng.standard_normal((4, 128)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    exp = ref64.rms_norm(o, w, 1e-6) * z / (1 + np.exp(-z.astype(np.float64)))
    np.testing.assert_allclose(orc.rmsnorm_gated(o, z, w, 1e-6), exp, rtol=1e-5, atol=1e-6)


def test_conv1d_silu_direct_convolution(orc):
    rng = np.random.default_rng(19)
    cd, dc, steps = 16, 4, 6
    w = rng.standard_normal((cd, dc)).astype(np.float32)
    xs = rng.standard_normal((steps, cd)).astype(np.float32)
    hist = np.zeros((dc - 1, cd), np.float32)
    padded = np.concatenate([np.zeros((dc - 1, cd)), xs.astype(np.float64)])
    for t in range(steps):
        y, hist = orc.conv1d_silu(xs[t], hist, w, dc)
        val = (padded[t:t + dc].T * w).sum(1)  # causal window, oldest first
        np.testing.assert_allclose(y, val / (1 + np.exp(-val)), rtol=1e-5, atol=1e-6)

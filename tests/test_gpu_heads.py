"""Head counts beyond one MFMA pass and beyond multiples (src/model/mod.rs:1155: query head h
reads KV head h % n_kv_heads for any counts).

Decode splits a KV head's query heads into column blocks of up to 16 (and cols * D <= 2048);
with the modulo map and n_q_heads not a multiple of n_kv_heads, the last KV heads simply have
fewer query heads.  Each case is checked against the oracle (whose loop is the reference's
modulo map) to the f16-cache bound of 1e-2 per head row (max-abs 2e-3 for the f32 cache).
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import PagedCase, device, parallel_map, row_rel_err, to_dev

pytestmark = pytest.mark.gpu


def _decode_check(case, dev, gqa_mode=0, gate=None, f32=False):
    out = case.gpu_decode(dev, gqa_mode=gqa_mode, gate=gate)
    hq, hkv = case.hq, case.hkv
    refs = []
    for i in range(len(case.lens)):
        g = None if gate is None else gate[i]
        if gqa_mode == 0:
            refs.append(case.oracle_out(i, kv_round=None if f32 else np.float16, gate=g))
        else:  # grouped head h -> KV head h // group, as modulo head (h % group) * hkv + h // group
            group = hq // hkv
            perm = [(h % group) * hkv + h // group for h in range(hq)]
            kc, vc = case.oracle_caches(i, kv_round=None if f32 else np.float16)
            q = case.oracle_q(i)
            qq = np.empty_like(q)
            qq[perm] = q
            o = orc.attn_decode(qq, kc, vc)[perm]
            refs.append(o if g is None else orc.apply_gate(o, g))
    for i, ref in enumerate(refs):
        if f32:
            err = float(np.abs(out[i] - ref).max())
            assert err <= 2e-3, f"seq {i}: max-abs {err}"
        else:
            err = row_rel_err(out[i], ref)
            assert err <= 1e-2, f"seq {i} (L={case.lens[i]}): rel err {err}"
    return out


@pytest.mark.parametrize("hq,hkv", [(12, 5), (7, 3), (9, 8)])
def test_decode_heads_not_a_multiple(hq, hkv):
    """Modulo map with n_q_heads % n_kv_heads != 0 (the last KV heads carry fewer heads)."""
    dev = device()
    rng = np.random.default_rng(hq * 100 + hkv)
    case = PagedCase(rng, [700, 1, 3000, 33], hq, hkv, 128, theta=1e6)
    case.gpu_build(dev, torch.float16)
    _decode_check(case, dev)


@pytest.mark.parametrize("gqa_mode", [0, 1])
def test_decode_more_than_16_heads_per_kv_head(gqa_mode):
    """40 query heads over 2 KV heads (20 per KV head: two column blocks of 10)."""
    dev = device()
    rng = np.random.default_rng(40 + gqa_mode)
    case = PagedCase(rng, [2000, 17, 513], 40, 2, 128, theta=1e6)
    case.gpu_build(dev, torch.float16)
    _decode_check(case, dev, gqa_mode=gqa_mode)


def test_decode_d256_16_heads_per_kv_head_gated():
    """D 256 holds 8 heads per pass (8 x 256 = 2048 floats): 32 / 2 heads run two blocks."""
    dev = device()
    rng = np.random.default_rng(256)
    case = PagedCase(rng, [4097, 100], 32, 2, 256, theta=1e7, rope_dim=64,
                     sections=[11, 11, 10, 0])
    case.gpu_build(dev, torch.float16)
    gate = rng.standard_normal((2, 32, 256)).astype(np.float32)
    _decode_check(case, dev, gate=gate)


def test_decode_f32_pool_d64_32_heads_per_kv_head():
    """f32 cache, D 64, 64 / 2 heads (two blocks of 16): max-abs 2e-3."""
    dev = device()
    rng = np.random.default_rng(64)
    case = PagedCase(rng, [300, 1000], 64, 2, 64, theta=1e4)
    case.gpu_build(dev, torch.float32)
    _decode_check(case, dev, f32=True)


def test_decode_noalloc_with_column_blocks():
    """The no-alloc entry over several column blocks per KV head gives pi_attn_decode's bits."""
    dev = device()
    rng = np.random.default_rng(0x40A)
    case = PagedCase(rng, [1500, 40, 800], 36, 2, 128, theta=1e6)
    case.gpu_build(dev, torch.float16)
    q = case.gpu_q(dev)
    ctx = to_dev(np.array(case.lens, np.int32))
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    outs = []
    for entry in ("pi_attn_decode", "pi_attn_decode_noalloc"):
        o = torch.empty_like(q)
        dev.check(getattr(dev.lib, entry)(dev.h, P(q), case.pool.p, P(case.pt), case.pt.shape[1],
                                          P(ctx), 3, 36, 0, 1 / math.sqrt(128), None, P(o),
                                          dev.stream()))
        torch.cuda.synchronize()
        outs.append(o.cpu().numpy())
    np.testing.assert_array_equal(outs[0], outs[1])


def test_grouped_map_needs_a_multiple():
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(1)
    case = PagedCase(rng, [10], 12, 5, 128)
    case.gpu_build(dev, torch.float16)
    with pytest.raises(rt.InvalidArg):
        case.gpu_decode(dev, gqa_mode=1)


def test_prefill_heads_not_a_multiple():
    """Causal prefill with 10 query heads over 4 KV heads (modulo map)."""
    from tests.test_gpu_prefill import _inputs, _run
    rng = np.random.default_rng(104)
    tq, tk, tv = _inputs(rng, 200, 10, 4, 128)
    out = _run(tq, tk, tv)
    qf, kf, vf = (t.float().numpy() for t in (tq, tk, tv))
    ref = np.stack(parallel_map(lambda i: orc.attn_decode(qf[i], kf[:i + 1], vf[:i + 1]), range(200)))
    assert row_rel_err(out, ref) <= 1e-2


def test_turboquant_heads_not_a_multiple():
    """TurboQuant decode with 7 query heads over 3 KV heads (modulo map)."""
    from powerinfer_x64_amd import runtime as rt
    from tests.test_gpu_turboquant import TqCase
    dev = device()
    rng = np.random.default_rng(73)
    lens = [300, 1, 64]
    case = TqCase(rng, lens, 3)
    case.build(dev)
    q = rng.standard_normal((3, 7, 128)).astype(np.float32)
    out = rt.tq_attn_decode(dev, to_dev(q), case.pool, case.pt_d,
                            to_dev(np.array(lens, np.int32))).cpu().numpy()
    for i in range(3):
        assert row_rel_err(out[i], case.oracle_out(i, q[i])) <= 1e-2

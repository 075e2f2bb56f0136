"""pi_attn_decode_noalloc (the decode entry point that allocates nothing: its split-run
partials live in a fixed per-GPU scratch array) against pi_attn_decode on the same inputs,
both called through the C ABI.  The two run the same plan and kernels, so their outputs
must agree bit for bit; each is also held to the oracle's tolerance (f16 cache: 1e-2 per
head row, src/model/mod.rs:1148-1196).  Two no-alloc calls run back to back, the second on
a smaller input, so a stale partial left in the shared scratch by the first would show."""
import ctypes
import math

import numpy as np
import pytest
import torch

from tests.gpu_util import PagedCase, device, row_rel_err, to_dev

pytestmark = pytest.mark.gpu


def _decode(dev, entry, q, case, ctx, gate=None):
    out = torch.full_like(q, float("nan"))
    fn = getattr(dev.lib, entry)
    vp = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    rc = fn(dev.h, vp(q), case.pool.p, vp(case.pt), case.pt.shape[1], vp(ctx), q.shape[0],
            q.shape[1], 0, 1.0 / math.sqrt(case.d), vp(gate), vp(out), dev.stream())
    dev.check(rc)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _pair(dev, case, q, ctx, gate=None):
    a = _decode(dev, "pi_attn_decode", q, case, ctx, gate)
    b = _decode(dev, "pi_attn_decode_noalloc", q, case, ctx, gate)
    assert np.isfinite(b).all()
    np.testing.assert_array_equal(a, b)
    return b


def test_noalloc_matches_decode_two_calls_c2_shape():
    """Config-2 heads (32/8, D 128, f16 pages): a 12-sequence ragged batch, then the first 3
    sequences cut to shorter contexts."""
    dev = device()
    rng = np.random.default_rng(0x5EED0A11)
    lens = [int(x) for x in rng.integers(1, 9000, size=12)]
    lens[0] = 8191
    case = PagedCase(rng, lens, 32, 8, 128, theta=1e6)
    case.gpu_build(dev, torch.float16)
    q = case.gpu_q(dev)
    out = _pair(dev, case, q, to_dev(np.array(lens, np.int32)))
    for i in range(len(lens)):
        err = row_rel_err(out[i], case.oracle_out(i, kv_round=np.float16))
        assert err <= 1e-2, f"seq {i} (L={lens[i]}): rel err {err}"
    # second call: 3 sequences over prefixes of their caches
    short = [700, 1, 33]
    q3 = q[:3].contiguous()
    pt3 = case.pt[:3].contiguous()
    keep = case.pt
    case.pt = pt3
    try:
        out3 = _pair(dev, case, q3, to_dev(np.array(short, np.int32)))
    finally:
        case.pt = keep
    for i, n in enumerate(short):
        sub = PagedCase.__new__(PagedCase)
        sub.__dict__.update(case.__dict__)
        sub.lens = list(case.lens)
        sub.k = [case.k[i][:n]]
        sub.v = [case.v[i][:n]]
        # the query was rotated at position lens[i] - 1, so compare with that query
        kc, vc = sub.oracle_caches(0, kv_round=np.float16)
        from oracle import oracle as orc
        ref = orc.attn_decode(case.oracle_q(i), kc, vc)
        err = row_rel_err(out3[i], ref)
        assert err <= 1e-2, f"short seq {i} (L={n}): rel err {err}"


def test_noalloc_matches_decode_c4_shape_gate():
    """Config-4 heads (16/2, D 256, q/k RMSNorm, IMRoPE, sigmoid gate), 4 sequences, then 2."""
    dev = device()
    rng = np.random.default_rng(0x5EED0A12)
    lens = [20000, 4097, 1, 777]
    qn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    case = PagedCase(rng, lens, 16, 2, 256, theta=1e7, rope_dim=64, sections=[11, 11, 10, 0],
                     q_norm_w=qn, k_norm_w=kn)
    case.gpu_build(dev, torch.float16)
    q = case.gpu_q(dev)
    gate = rng.standard_normal((4, 16, 256)).astype(np.float32)
    g = to_dev(gate)
    out = _pair(dev, case, q, to_dev(np.array(lens, np.int32)), g)
    for i in range(4):
        ref = case.oracle_out(i, kv_round=np.float16, gate=gate[i])
        assert row_rel_err(out[i], ref) <= 1e-2
    out2 = _pair(dev, case, q, to_dev(np.array([16, 1, 1, 5], np.int32)), g)
    assert np.isfinite(out2).all()


def test_noalloc_rejects_launch_beyond_scratch():
    """4096 sequences x 8 KV heads at 2 q heads per KV head and D 256 need more partial
    slots than the fixed scratch holds: the call fails with PI_ERR_UNSUPPORTED before any
    launch (the tables are well formed, so nothing unsafe would run either way)."""
    dev = device()
    from powerinfer_x64_amd import runtime as rt
    pool = rt.KvPool(dev, 4, 8, 256, dtype=torch.float16)
    b = 4096
    q = torch.zeros((b, 16, 256), dtype=torch.float32, device="cuda")
    pt = torch.zeros((b, 1), dtype=torch.int32, device="cuda")
    ctx = torch.ones(b, dtype=torch.int32, device="cuda")
    out = torch.zeros_like(q)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = dev.lib.pi_attn_decode_noalloc(dev.h, vp(q), pool.p, vp(pt), 1, vp(ctx), b, 16, 0,
                                        0.0625, None, vp(out), dev.stream())
    assert rc == 5, rc  # PI_ERR_UNSUPPORTED
    assert b"scratch" in dev.lib.pi_last_error(dev.h)
    torch.cuda.synchronize()
    assert not out.any()

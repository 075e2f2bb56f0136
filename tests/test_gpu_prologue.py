"""Decode prologue kernels vs the oracle: RoPE (src/ops.rs:35-157), per-head
RMSNorm (src/ops.rs:13-27) and the paged KV append/read round trip
(src/model/mod.rs:1140-1146)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import device, to_dev

pytestmark = pytest.mark.gpu


def _rt():
    from powerinfer_x64_amd import runtime as rt
    return rt


@pytest.mark.parametrize("mode", ["norm", "imrope"])
def test_rope_matches_oracle(mode):
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(1 if mode == "norm" else 2)
    n, hq, hkv, d = 64, 8, 2, 256 if mode == "imrope" else 128
    pos = np.concatenate([np.arange(32), rng.integers(0, 65536, 32)]).astype(np.int32)
    q = rng.standard_normal((n, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    if mode == "norm":
        theta, rd, sec, freqs = 1e6, 128, None, None
    else:
        theta, rd, sec = 1e7, 64, [11, 11, 10, 0]
        freqs = orc.compute_imrope_freqs(theta, rd, sec)
    tq, tk = to_dev(q), to_dev(k)
    rt.rope(dev, tq, tk, to_dev(pos), rd, theta, sec)
    torch.cuda.synchronize()
    gq, gk = tq.cpu().numpy(), tk.cpu().numpy()
    for i in range(n):
        eq, ek = orc.attn_prepare(q[i][None], k[i][None], hq, hkv, d, rope_dim=rd,
                                  rope_base=theta, freqs=freqs, pos0=int(pos[i]))
        # same f32 angle; cos/sin may differ by an ulp between the GPU and glibc
        np.testing.assert_allclose(gq[i], eq[0], atol=2e-6, rtol=0)
        np.testing.assert_allclose(gk[i], ek[0], atol=2e-6, rtol=0)


def test_head_rmsnorm_matches_oracle():
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(3)
    x = rng.standard_normal((50, 16, 256)).astype(np.float32) * 3
    w = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    tx = to_dev(x)
    rt.head_rmsnorm(dev, tx, to_dev(w), 1e-6)
    torch.cuda.synchronize()
    g = tx.cpu().numpy().reshape(-1, 256)
    ref = np.stack([orc.rms_norm(r, w, 1e-6) for r in x.reshape(-1, 256)])
    np.testing.assert_allclose(g, ref, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("pool_dtype,src", [(torch.float32, torch.float32),
                                            (torch.float16, torch.float32),
                                            (torch.float16, torch.float16),
                                            (torch.float16, torch.bfloat16)])
def test_kv_append_read_roundtrip(pool_dtype, src):
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(4)
    hkv, d = 4, 128
    pool = rt.KvPool(dev, 40, hkv, d, dtype=pool_dtype)
    pt = to_dev(rng.permutation(40)[:36].reshape(2, 18).astype(np.int32))
    k = rng.standard_normal((2, 100, hkv, d)).astype(np.float32)
    v = rng.standard_normal((2, 100, hkv, d)).astype(np.float32)
    tk, tv = to_dev(k, src), to_dev(v, src)
    # prompt of 100 tokens, then 3 single-token appends (decode steps)
    pool.append(tk[:, :97].contiguous(), tv[:, :97].contiguous(), pt,
                to_dev(np.zeros(2, np.int32)))
    for t in range(97, 100):
        pool.append(tk[:, t:t + 1].contiguous(), tv[:, t:t + 1].contiguous(), pt,
                    to_dev(np.full(2, t, np.int32)))
    for s in range(2):
        ko, vo = pool.read(pt, s, 0, 100)
        torch.cuda.synchronize()
        ek = tk[s].to(pool_dtype).float().cpu().numpy()
        ev = tv[s].to(pool_dtype).float().cpu().numpy()
        np.testing.assert_array_equal(ko.cpu().numpy(), ek)
        np.testing.assert_array_equal(vo.cpu().numpy(), ev)


@pytest.mark.parametrize("pool_dtype,d", [(torch.float16, 256), (torch.float16, 64),
                                         (torch.float32, 128)])
def test_kv_append_page_edges(pool_dtype, d):
    """Appends that start and end inside pages, at different positions per sequence, with a
    negative start (the positions below 0 are dropped) and rows past the table: every slot the
    call owns holds its value, every other slot keeps what it held."""
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(7 + d)
    hkv, n_pages, mp = 2, 30, 6
    pool = rt.KvPool(dev, n_pages, hkv, d, dtype=pool_dtype)
    table = rng.permutation(n_pages)[:2 * mp].reshape(2, mp).astype(np.int32)
    pt = to_dev(table)
    cap = 16 * mp
    ek = np.zeros((2, cap, hkv, d), np.float32)
    ev = np.zeros((2, cap, hkv, d), np.float32)

    def append(starts, n):
        k = rng.standard_normal((2, n, hkv, d)).astype(np.float32)
        v = rng.standard_normal((2, n, hkv, d)).astype(np.float32)
        pool.append(to_dev(k), to_dev(v), pt, to_dev(np.array(starts, np.int32)))
        for s_ in range(2):
            for t in range(n):
                p = starts[s_] + t
                if 0 <= p < cap:
                    ek[s_, p] = k[s_, t]
                    ev[s_, p] = v[s_, t]

    append([0, 0], 50)      # a prompt ending inside page 3
    append([50, 37], 7)     # continues seq 0; overwrites slots 37.. of seq 1 inside a page
    append([-3, 57], 5)     # seq 0: positions 0 and 1 only
    append([60, 93], 9)     # seq 1 runs past its 96-slot table: positions >= 96 dropped
    for s_ in range(2):
        ko, vo = pool.read(pt, s_, 0, cap)
        torch.cuda.synchronize()
        want_k = torch.from_numpy(ek[s_]).to(pool_dtype).float().numpy()
        want_v = torch.from_numpy(ev[s_]).to(pool_dtype).float().numpy()
        written = np.zeros(cap, bool)
        if s_ == 0:
            written[:57] = True
            written[60:69] = True
        else:
            written[:50] = True
            written[57:62] = True
            written[93:96] = True
        np.testing.assert_array_equal(ko.cpu().numpy()[written], want_k[written])
        np.testing.assert_array_equal(vo.cpu().numpy()[written], want_v[written])


@pytest.mark.parametrize("pool_dtype,d,mode", [(torch.float16, 256, "imrope"),
                                              (torch.float16, 128, "norm"),
                                              (torch.float32, 64, "norm")])
def test_prologue_prompt_appends_by_page(pool_dtype, d, mode):
    """A launch of 2 x 1030 tokens, enough for the K / V side to run by page: sequence 0
    starts inside a page (7) and sequence 1 below 0 (-20: those positions are dropped), both
    run past a 60-page table (positions >= 960 dropped), and one page id of sequence 0 lies
    outside the pool. q and k come back normed and rotated at every position (against the
    oracle where the position is >= 0); every slot the launch owns holds its K / V, every
    other slot keeps what an earlier append put there."""
    rt = _rt()
    dev = device()
    rng = np.random.default_rng(0xB1 + d)
    n_seq, n, hq, hkv, mp, n_pages = 2, 1030, 4, 2, 60, 130
    starts = [7, -20]
    cap = 16 * mp
    table = rng.permutation(n_pages)[:2 * mp].reshape(2, mp).astype(np.int32)
    table[0, 10] = n_pages + 3  # positions 160 .. 175 of sequence 0 have no page
    pool = rt.KvPool(dev, n_pages, hkv, d, dtype=pool_dtype)
    pt = to_dev(table)
    # earlier contents of every slot
    k0 = rng.standard_normal((n_seq, cap, hkv, d)).astype(np.float32)
    v0 = rng.standard_normal((n_seq, cap, hkv, d)).astype(np.float32)
    pool.append(to_dev(k0), to_dev(v0), pt, to_dev(np.zeros(n_seq, np.int32)))
    q = rng.standard_normal((n_seq, n, hq, d)).astype(np.float32)
    k = rng.standard_normal((n_seq, n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n_seq, n, hkv, d)).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, d).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, d).astype(np.float32)
    if mode == "norm":
        kw = dict(rope_dim=d, rope_base=1e6)
        sec, freqs = None, None
    else:
        sec = [11, 11, 10, 0]
        kw = dict(rope_dim=64, rope_base=1e7)
        freqs = orc.compute_imrope_freqs(1e7, 64, sec)
    tq, tk = to_dev(q), to_dev(k)
    rt.attn_prologue(dev, tq, tk, to_dev(v), pool, pt, to_dev(np.array(starts, np.int32)),
                     q_norm_w=to_dev(qn), k_norm_w=to_dev(kn), eps=1e-6, sections=sec, **kw)
    torch.cuda.synchronize()
    gq, gk = tq.cpu().numpy(), tk.cpu().numpy()
    rk = np.zeros_like(k)
    for s_ in range(n_seq):
        t0 = max(0, -starts[s_])  # first token at a position >= 0
        eq, ek = orc.attn_prepare(q[s_, t0:], k[s_, t0:], hq, hkv, d, q_norm_w=qn, k_norm_w=kn,
                                  eps=1e-6, freqs=freqs, pos0=starts[s_] + t0, **kw)
        np.testing.assert_allclose(gq[s_, t0:], eq, atol=2e-5, rtol=0)
        np.testing.assert_allclose(gk[s_, t0:], ek, atol=2e-5, rtol=0)
        rk[s_, t0:] = gk[s_, t0:]
    for s_ in range(n_seq):
        want_k = k0[s_].copy()
        want_v = v0[s_].copy()
        for t in range(n):
            p = starts[s_] + t
            if 0 <= p < cap:
                want_k[p] = rk[s_, t]
                want_v[p] = v[s_, t]
        if s_ == 0:
            want_k[160:176] = 0.0  # read back through an id outside the pool: zeros
            want_v[160:176] = 0.0
        ko, vo = pool.read(pt, s_, 0, cap)
        torch.cuda.synchronize()
        rd = lambda a: torch.from_numpy(a).to(pool_dtype).float().numpy()  # noqa: E731
        np.testing.assert_array_equal(vo.cpu().numpy(), rd(want_v))
        # K: the stored value is the device's rotated k rounded to the pool's type
        np.testing.assert_array_equal(ko.cpu().numpy(), rd(want_k))


def test_pool_rejects_bad_shapes():
    rt = _rt()
    dev = device()
    with pytest.raises(rt.Unsupported):
        rt.KvPool(dev, 4, 2, 96)
    with pytest.raises(rt.Unsupported):
        rt.KvPool(dev, 4, 2, 128, page_tokens=32)
    pool = rt.KvPool(dev, 4, 3, 128)
    q = torch.zeros((1, 4, 128), device="cuda")
    with pytest.raises(rt.InvalidArg):  # 4 q heads over 3 kv heads: the grouped map needs a multiple
        rt.attn_decode(dev, q, pool, torch.zeros((1, 1), dtype=torch.int32, device="cuda"),
                       torch.ones(1, dtype=torch.int32, device="cuda"), gqa_mode=1)

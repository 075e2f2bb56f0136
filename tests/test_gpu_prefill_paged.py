"""Causal prefill of a chunk that continues a sequence, over its paged cache
(pi_attn_prefill_paged), against the oracle.

The reference runs every token of a forward call against prev_seq_len + pos + 1 keys
(src/model/mod.rs:668 token loop over :1140-1190), so row i of a chunk starting at position
P is or_attn_decode over keys 0 .. P + i.  Keys are drawn raw, normalised / rotated at their
positions and appended to a pool with permuted pages on the GPU; the oracle prepares the
same raw rows (or_attn_prepare) and reads them rounded to f16 as the pool stores them; the
chunk's queries are rotated at P .. and rounded to f16 (the kernel's input).  Tolerance:
1e-2 relative per (token, head) row (f16 class); argmax of synthetic logits exact.  With an
f32 pool nothing is rounded and the bound is max-abs 2e-3 (f32 class).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import argmax_agreement, device, parallel_map, row_rel_err, to_dev

pytestmark = pytest.mark.gpu


class Chunk:
    """One sequence: `prev` cached tokens plus a chunk of `n`, all appended to the pool."""

    def __init__(self, rng, prev, n, hq, hkv, d, theta=1e6, rope_dim=None, sections=None,
                 norm=False, extra_pages=5):
        self.prev, self.n, self.hq, self.hkv, self.d = prev, n, hq, hkv, d
        self.theta, self.sections = theta, sections
        self.rope_dim = rope_dim or d
        self.freqs = orc.compute_imrope_freqs(theta, self.rope_dim, sections) if sections else None
        total = prev + n
        self.max_pages = (total + 15) // 16 + 2
        self.n_pages = self.max_pages + extra_pages
        self.row = rng.permutation(self.n_pages)[:self.max_pages].astype(np.int32)
        self.k = rng.standard_normal((total, hkv, d), dtype=np.float32)
        self.v = rng.standard_normal((total, hkv, d), dtype=np.float32)
        self.q = rng.standard_normal((n, hq, d), dtype=np.float32)
        self.qn = rng.uniform(0.5, 1.5, d).astype(np.float32) if norm else None
        self.kn = rng.uniform(0.5, 1.5, d).astype(np.float32) if norm else None

    def prepared(self, f32=False):
        """Rotated q and K, and V, rounded to f16 (f16 pool) or not (f32 pool), as f32."""
        kw = dict(eps=1e-6, rope_dim=self.rope_dim, rope_base=self.theta, freqs=self.freqs)
        _, kr = orc.attn_prepare(None, self.k, self.hq, self.hkv, self.d, k_norm_w=self.kn,
                                 pos0=0, **kw)
        qr, _ = orc.attn_prepare(self.q, None, self.hq, self.hkv, self.d, q_norm_w=self.qn,
                                 pos0=self.prev, **kw)
        if f32:
            return qr, kr, self.v
        r = lambda a: a.astype(np.float16).astype(np.float32)  # noqa: E731
        return r(qr), r(kr), r(self.v)

    def oracle(self, rows, f32=False):
        q, k, v = self.prepared(f32)
        p = self.prev
        return np.stack(parallel_map(lambda i: orc.attn_decode(q[i], k[:p + i + 1], v[:p + i + 1]),
                                     list(rows)))

    def gpu(self, dev, gqa_mode=0, pool_dtype=torch.float16):
        from powerinfer_x64_amd import runtime as rt
        pool = rt.KvPool(dev, self.n_pages, self.hkv, self.d, dtype=pool_dtype)
        row = to_dev(self.row)
        q, k, v = to_dev(self.q), to_dev(self.k), to_dev(self.v)
        # the prologue's steps: norm, RoPE at the positions, append
        if self.kn is not None:
            rt.head_rmsnorm(dev, k, to_dev(self.kn), 1e-6)
            rt.head_rmsnorm(dev, q, to_dev(self.qn), 1e-6)
        total = self.prev + self.n
        rt.rope(dev, k, None, torch.arange(total, dtype=torch.int32, device="cuda"),
                self.rope_dim, self.theta, self.sections)
        rt.rope(dev, q, None, torch.arange(self.prev, total, dtype=torch.int32, device="cuda"),
                self.rope_dim, self.theta, self.sections)
        pool.append(k[None].contiguous(), v[None].contiguous(), row[None].contiguous(),
                    torch.zeros(1, dtype=torch.int32, device="cuda"))
        qin = q.half().contiguous() if pool_dtype == torch.float16 else q
        out = rt.attn_prefill_paged(dev, qin, pool, row, self.prev, gqa_mode=gqa_mode)
        torch.cuda.synchronize()
        self.pool, self.row_dev, self.q16 = pool, row, q.half().contiguous()
        return out.cpu().numpy()


def _check(out, ref, what):
    err = row_rel_err(out, ref)
    n, mism, ties = argmax_agreement(out, ref)
    print(f"\n{what}: worst row rel err {err:.3e}, argmax mismatches {mism}/{n} ({ties} ties)")
    assert err <= 1e-2, f"{what}: rel err {err}"
    assert mism == 0, f"{what}: {mism} argmax mismatches"


def _check_f32(out, ref, what):
    err = float(np.abs(out - ref).max())
    n, mism, ties = argmax_agreement(out, ref)
    print(f"\n{what}: max-abs {err:.3e}, argmax mismatches {mism}/{n} ({ties} ties)")
    assert err <= 2e-3, f"{what}: max-abs {err}"
    assert mism == 0, f"{what}: {mism} argmax mismatches"


@pytest.mark.parametrize("prev,n,hq,hkv,d", [(0, 300, 32, 32, 128), (700, 150, 32, 8, 128),
                                             (33, 129, 10, 4, 64), (1000, 65, 16, 2, 256),
                                             (4095, 1, 8, 8, 128), (17, 2, 4, 1, 64)])
def test_paged_prefill_f32_pool(prev, n, hq, hkv, d):
    """An f32 pool: a fresh prompt (prev 0, config-1 heads), continued chunks at tile and
    non-tile offsets, modulo heads that are not a multiple, D 64 / 128 / 256."""
    dev = device()
    c = Chunk(np.random.default_rng(prev * 7 + n + d), prev, n, hq, hkv, d)
    out = c.gpu(dev, pool_dtype=torch.float32)
    _check_f32(out, c.oracle(range(n), f32=True), f"f32 prev {prev} + {n} D {d}")


def test_paged_prefill_f32_grouped_d256_norm():
    """f32 pool, 16/2 heads, D 256, q/k norm and IMRoPE, grouped head map."""
    dev = device()
    c = Chunk(np.random.default_rng(0xF32), 300, 100, 16, 2, 256, theta=1e7, rope_dim=64,
              sections=[11, 11, 10, 0], norm=True)
    out = c.gpu(dev, gqa_mode=1, pool_dtype=torch.float32)
    q, k, v = c.prepared(f32=True)
    perm = [(h % 8) * 2 + h // 8 for h in range(16)]

    def row(i):
        qq = np.empty_like(q[i])
        qq[perm] = q[i]
        return orc.attn_decode(qq, k[:c.prev + i + 1], v[:c.prev + i + 1])[perm]
    _check_f32(out, np.stack(parallel_map(row, range(c.n))), "f32 D 256 grouped")


def test_paged_prefill_f32_1024_over_8k_history():
    """A 1024-token chunk over an 8192-token history with an f32 pool (config-1 heads at
    config-2's GQA): sampled rows across the chunk."""
    dev = device()
    c = Chunk(np.random.default_rng(0xF8192), 8192, 1024, 32, 8, 128)
    out = c.gpu(dev, pool_dtype=torch.float32)
    rows = [0, 1, 31, 32, 63, 64, 1000, 1023] + list(np.random.default_rng(4).integers(0, 1024, 16))
    _check_f32(out[rows], c.oracle(rows, f32=True), "f32 1024 over 8192")


@pytest.mark.parametrize("prev,n", [(700, 300), (64, 64), (1000, 2), (4095, 1), (33, 129)])
def test_paged_prefill_c2_shape(prev, n):
    """32/8 heads, D 128, NORM RoPE 1e6: offsets that are and are not tile multiples (a
    wavefront's rows can then straddle two masked tiles)."""
    dev = device()
    c = Chunk(np.random.default_rng(prev * 31 + n), prev, n, 32, 8, 128)
    out = c.gpu(dev)
    _check(out, c.oracle(range(n)), f"prev {prev} + {n}")


@pytest.mark.parametrize("gqa_mode", [0, 1])
def test_paged_prefill_c4_shape_d256(gqa_mode):
    """16/2 heads, D 256, q/k RMSNorm, IMRoPE (64 dims, [11, 11, 10, 0], 1e7); both head maps."""
    dev = device()
    c = Chunk(np.random.default_rng(77 + gqa_mode), 1000, 129, 16, 2, 256, theta=1e7,
              rope_dim=64, sections=[11, 11, 10, 0], norm=True)
    out = c.gpu(dev, gqa_mode)
    if gqa_mode == 0:
        _check(out, c.oracle(range(c.n)), "D 256 prev 1000 + 129")
    else:  # grouped map: q head h reads KV head h // 8; the oracle's map is modulo
        q, k, v = c.prepared()
        hq, hkv = c.hq, c.hkv
        perm = [(h % 8) * hkv + h // 8 for h in range(hq)]  # grouped head h as modulo head

        def row(i):
            qq = np.empty_like(q[i])
            qq[perm] = q[i]
            o = orc.attn_decode(qq, k[:c.prev + i + 1], v[:c.prev + i + 1])
            return o[perm]
        _check(out, np.stack(parallel_map(row, range(c.n))), "D 256 grouped")


def test_paged_prefill_start_zero_equals_contiguous_prefill():
    """start_pos 0: the same f16 rows as pi_attn_prefill's.  The paged kernel takes a key step's
    16 keys in another slot order inside its MFMAs, so the two agree to f32 rounding."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    c = Chunk(np.random.default_rng(5), 0, 333, 32, 8, 128)
    out = c.gpu(dev)
    k16 = torch.from_numpy(c.k).cuda()
    rt.rope(dev, k16, None, torch.arange(333, dtype=torch.int32, device="cuda"), 128, 1e6, None)
    ref = rt.attn_prefill(dev, c.q16[None], k16.half()[None].contiguous(),
                          torch.from_numpy(c.v).cuda().half()[None].contiguous())
    torch.cuda.synchronize()
    ref = ref[0].cpu().numpy()
    assert row_rel_err(out, ref) <= 1e-5


def test_paged_prefill_1024_over_8k_history():
    """A 1024-token chunk over an 8192-token history (config-2 heads): rows across the chunk,
    including its first and last, against the oracle."""
    dev = device()
    c = Chunk(np.random.default_rng(0x8192), 8192, 1024, 32, 8, 128)
    out = c.gpu(dev)
    rows = [0, 1, 63, 64, 511, 1000, 1022, 1023] + list(np.random.default_rng(3).integers(0, 1024, 24))
    _check(out[rows], c.oracle(rows), "1024 over 8192")


def test_paged_prefill_rejects_bad_shapes():
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    pool = rt.KvPool(dev, 8, 2, 128, dtype=torch.float16)
    row = torch.arange(8, dtype=torch.int32, device="cuda")
    q = torch.zeros((10, 4, 128), dtype=torch.float16, device="cuda")
    with pytest.raises(rt.InvalidArg):  # 120 + 10 keys > 8 pages of 16
        rt.attn_prefill_paged(dev, q, pool, row, 120)
    pool32 = rt.KvPool(dev, 8, 2, 128, dtype=torch.float32)
    with pytest.raises(rt.InvalidArg):  # an f32 pool takes f32 queries
        rt.attn_prefill_paged(dev, q, pool32, row, 0)
    pool64 = rt.KvPool(dev, 8, 2, 64, dtype=torch.float16)
    with pytest.raises(rt.InvalidArg):  # q rows must match the pool's head_dim
        rt.attn_prefill_paged(dev, q, pool64, row, 0)


@pytest.mark.parametrize("prev,n,hq,hkv", [(0, 200, 8, 8), (300, 129, 16, 4), (1000, 1, 4, 2),
                                           (17, 64, 12, 4)])
def test_paged_prefill_f16_head_dim_64(prev, n, hq, hkv):
    """An f16 pool at head dim 64 (the flash prefill straight from the pages): a fresh prompt,
    continued chunks at tile and non-tile offsets, a single row, modulo heads."""
    dev = device()
    c = Chunk(np.random.default_rng(prev * 13 + n + 64), prev, n, hq, hkv, 64)
    out = c.gpu(dev)
    _check(out, c.oracle(range(n)), f"D 64 prev {prev} + {n}")


@pytest.mark.parametrize("prev,n,hq,hkv", [(0, 300, 16, 2), (17, 64, 16, 2), (1000, 1, 8, 2),
                                           (50, 129, 12, 4)])
def test_paged_prefill_f16_head_dim_256(prev, n, hq, hkv):
    """An f16 pool at head dim 256 (the two-wavefront-per-SIMD flash prefill straight from the
    pages): a fresh prompt, chunks at non-tile offsets, a single row, modulo heads."""
    dev = device()
    c = Chunk(np.random.default_rng(prev * 7 + n + 256), prev, n, hq, hkv, 256)
    out = c.gpu(dev)
    _check(out, c.oracle(range(n)), f"D 256 prev {prev} + {n}")


@pytest.mark.parametrize("d", [64, 128, 256])
def test_paged_prefill_page_ids_outside_the_pool_hold_no_tokens(d):
    """Page-table entries outside [0, n_pages) hold no tokens, as for the decode: their keys
    are masked (a row whose every key is masked gets zeros).  Two pages of the history, one
    inside a tile and one at a tile's start, are made invalid; the oracle drops their keys."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    c = Chunk(np.random.default_rng(0xBAD + d), 200, 100, 8, 2, d)
    c.gpu(dev)  # pool filled through the real row
    bad = [2, 4]  # pages 2 (keys 32..47) and 4 (keys 64..79)
    row = c.row.copy()
    row[2], row[4] = -1, c.n_pages + 3
    out = rt.attn_prefill_paged(dev, c.q16, c.pool, to_dev(row), c.prev)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    q, k, v = c.prepared()
    keep = np.ones(c.prev + c.n, bool)
    for pg in bad:
        keep[16 * pg:16 * pg + 16] = False

    def ref_row(i):
        m = keep[:c.prev + i + 1]
        return orc.attn_decode(q[i], k[:c.prev + i + 1][m], v[:c.prev + i + 1][m])
    _check(out, np.stack(parallel_map(ref_row, range(c.n))), "pages outside the pool")


@pytest.mark.parametrize("paired,ksplit", [("1", None), (None, "2"), (None, "3"), (None, "4")])
@pytest.mark.parametrize("prev,n,hq,hkv,d", [(700, 150, 32, 8, 128), (1000, 129, 16, 2, 256),
                                             (300, 129, 16, 4, 64)])
def test_paged_prefill_forced_schedules(monkeypatch, paired, ksplit, prev, n, hq, hkv, d):
    """The paired schedule and key splits 2-4 forced on continued chunks (start_pos > 0, so the
    last two tiles of a wavefront take the mask), for the paged kernel at D 64 / 128 and the
    gathered D 256 one, against the oracle."""
    if paired:
        monkeypatch.setenv("PI_PREFILL_PAIRED", paired)
    else:
        monkeypatch.setenv("PI_PREFILL_PAIRED", "0")
        monkeypatch.setenv("PI_PREFILL_KSPLIT", ksplit)
    dev = device()
    c = Chunk(np.random.default_rng(prev + n + d + (int(ksplit) if ksplit else 9)), prev, n, hq, hkv, d,
              theta=1e6)
    out = c.gpu(dev)
    _check(out, c.oracle(range(n)), f"forced paired={paired} ksplit={ksplit} D {d}")


def test_layer_forward_dev_equals_host_slices():
    """The device-pointer layer step gives the same bits as the host-slice one over a prompt,
    a continued chunk (the paged prefill) and decode tokens (config-4 layer shape)."""
    from powerinfer_x64_amd import runtime as rt
    dev = device()
    rng = np.random.default_rng(0x7D)
    qn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    kw = dict(q_norm_w=qn, k_norm_w=kn, rope_dim=64, rope_base=1e7, sections=[11, 11, 10, 0])
    a = rt.AttnLayer(dev, 1024, 16, 2, 256, torch.float16, **kw)
    b = rt.AttnLayer(dev, 1024, 16, 2, 256, torch.float16, **kw)
    for n in (300, 150, 1, 1, 77):
        q = rng.standard_normal((n, 16, 256)).astype(np.float32)
        k = rng.standard_normal((n, 2, 256)).astype(np.float32)
        v = rng.standard_normal((n, 2, 256)).astype(np.float32)
        g = rng.standard_normal((n, 16, 256)).astype(np.float32)
        oh = a.forward(q.copy(), k.copy(), v, gate=g)
        tq, tk = to_dev(q), to_dev(k)
        od = b.forward_dev(tq, tk, to_dev(v), gate=to_dev(g))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(oh, od.cpu().numpy())
    assert a.seq_len == b.seq_len == 529

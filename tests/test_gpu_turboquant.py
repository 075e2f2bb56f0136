"""TurboQuant compressed KV cache on the GPU vs the CPU oracle
(src/turboquant/mod.rs:408-566 and the compressed branch of the decode
attention, src/model/mod.rs:1161-1166).

Append: the stored key records (head_dim/2 bytes: 64 at D 128, 128 at D 256),
norms and f16 values must equal the restated quantize_vector / append byte for
byte.  Decode: per head row
||out - ref||_2 / ||ref||_2 <= 1e-2 (the north star's bound for an f16 KV
cache); the GPU dot uses f16 centroids (relative rounding <= 1.9e-4) and
keeps the weights below 1e-7 that the reference's value sum skips.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as o
from powerinfer_x64_amd import runtime as rt
from tests.gpu_util import device, parallel_map, row_rel_err, to_dev

pytestmark = pytest.mark.gpu
D = 128


def _matrices(n_kv, d=D):
    Rs, Gs = zip(*[o.tq_matrices(d, 0xCAFEBABE + h) for h in range(n_kv)])
    return np.stack(Rs), np.stack(Gs)


class TqCase:
    """Sequences of lengths `lens` appended in chunks into a permuted page table."""

    def __init__(self, rng, lens, hkv, extra_pages=2, key_scale=None, d=D):
        self.lens = [int(x) for x in lens]
        self.hkv, self.d = hkv, d
        b = len(self.lens)
        self.max_pages = max(1, max((x + 15) // 16 for x in self.lens))
        n_used = sum((x + 15) // 16 for x in self.lens)
        self.n_pages = n_used + extra_pages
        perm = rng.permutation(self.n_pages).astype(np.int32)
        self.pt = np.zeros((b, self.max_pages), np.int32)
        c = 0
        for i, L in enumerate(self.lens):
            np_i = (L + 15) // 16
            self.pt[i, :np_i] = perm[c:c + np_i]
            c += np_i
        self.k = [rng.standard_normal((L, hkv, d)).astype(np.float32) for L in self.lens]
        if key_scale is not None:
            self.k = [x * key_scale(rng, x.shape) for x in self.k]
            self.k = [x.astype(np.float32) for x in self.k]
        self.v = [rng.standard_normal((L, hkv, d)).astype(np.float32) for L in self.lens]
        self.R, self.G = _matrices(hkv, d)

    def build(self, dev, chunk=None):
        self.pool = rt.TqPool(dev, self.n_pages, self.hkv, head_dim=self.d)
        self.pt_d = to_dev(self.pt)
        for i, L in enumerate(self.lens):
            step = chunk or max(L, 1)
            for s0 in range(0, L, step):
                n = min(step, L - s0)
                pt_i = to_dev(self.pt[i:i + 1])
                self.pool.append(to_dev(self.k[i][None, s0:s0 + n]),
                                 to_dev(self.v[i][None, s0:s0 + n]), pt_i,
                                 to_dev(np.array([s0], np.int32)))
        torch.cuda.synchronize()

    def oracle_cache(self, i):
        L = self.lens[i]
        # the oracle's record stride is compressed_bytes() (:111-117), ceil(3d/8) + ceil(d/8)
        packed = np.zeros((L, self.hkv, o.tq_compressed_bytes(3, self.d, self.d)), np.uint8)
        norms = np.zeros((L, self.hkv), np.float32)
        for t in range(L):
            packed[t], norms[t] = o.tq_cache_append_keys(self.k[i][t], self.R, self.G)
        return packed, norms, self.v[i].astype(np.float16)

    def oracle_out(self, i, q, gqa_mode=0, gate=None):
        packed, norms, vals = self.oracle_cache(i)
        hq = q.shape[0]
        group = hq // self.hkv
        out = np.zeros((hq, self.d), np.float32)
        for h in range(hq):
            kvh = h % self.hkv if gqa_mode == 0 else h // group
            if self.lens[i]:
                out[h] = o.tq_cache_attend(q[h], packed, norms, vals, self.R[kvh], self.G[kvh], kvh)
        if gate is not None:
            out = out * (1.0 / (1.0 + np.exp(-gate.astype(np.float64)))).astype(np.float32)
        return out


def _check_records(case, i):
    keys, norms, vals = case.pool.read(case.pt_d, i, 0, case.lens[i])
    keys, norms, vals = keys.cpu().numpy(), norms.cpu().numpy(), vals.cpu().numpy()
    packed, norms_ref, vals_ref = case.oracle_cache(i)
    # the stored record is pack_compressed's bit stream, ceil(4d/8) bytes (:591-617); for
    # a d where compressed_bytes() is one longer the oracle's last byte is padding
    kb = keys.shape[2]
    assert kb == (4 * case.d + 7) // 8 and not packed[:, :, kb:].any()
    packed = packed[:, :, :kb]
    bad = np.argwhere((keys != packed).any(axis=2))
    assert bad.size == 0, f"seq {i}: {len(bad)} key records differ, first (token, head) {bad[0]}"
    assert np.array_equal(norms.view(np.uint32), norms_ref.view(np.uint32)), f"seq {i}: norms"
    assert np.array_equal(vals.view(np.uint16), vals_ref.view(np.uint16)), f"seq {i}: values"


def test_append_records_bit_exact():
    dev = device()
    rng = np.random.default_rng(0x70C0)
    case = TqCase(rng, [1, 16, 37, 300], 4)
    case.build(dev)
    for i in range(len(case.lens)):
        _check_records(case, i)


def test_append_in_chunks_and_edge_keys():
    """Chunked appends (start_pos), a zero key (norm 0 -> all codes of the zero vector),
    and keys spanning 1e-3 .. 1e3 in magnitude."""
    dev = device()
    rng = np.random.default_rng(0x70C1)

    def scale(r, shape):
        s = 10.0 ** r.uniform(-3, 3, size=shape[:2] + (1,))
        return s
    case = TqCase(rng, [53, 129], 2, key_scale=scale)
    case.k[0][5, 1, :] = 0.0
    case.build(dev, chunk=7)
    for i in range(len(case.lens)):
        _check_records(case, i)


@pytest.mark.parametrize("hq,hkv", [(8, 2), (12, 2), (3, 3), (32, 2), (42, 2)])
@pytest.mark.parametrize("gqa_mode", [0, 1])
def test_decode_matches_oracle_ragged(gqa_mode, hq, hkv):
    """Groups of 4, 6, 1 and 16 (the one-pass query precompute's head bounds 4, 8 and 16) and
    21 (above its bound: the two-pass precompute, full chunks of 4 heads and a partial one)."""
    dev = device()
    rng = np.random.default_rng(0x70C2 + gqa_mode + 16 * hq)
    lens = [1, 16, 200, 1000, 37]
    case = TqCase(rng, lens, hkv)
    case.build(dev)
    q = rng.standard_normal((len(lens), hq, D)).astype(np.float32) * 2
    out = rt.tq_attn_decode(dev, to_dev(q), case.pool, case.pt_d,
                            to_dev(np.array(lens, np.int32)), gqa_mode=gqa_mode)
    out = out.cpu().numpy()
    for i in range(len(lens)):
        ref = case.oracle_out(i, q[i], gqa_mode)
        err = row_rel_err(out[i], ref)
        assert err <= 1e-2, f"seq {i} (L={lens[i]}): rel err {err}"


def test_decode_gate_empty_context_and_long_sequence():
    dev = device()
    rng = np.random.default_rng(0x70C3)
    lens = [0, 4096, 5]
    hq, hkv = 4, 1
    case = TqCase(rng, lens, hkv)
    case.build(dev)
    q = rng.standard_normal((len(lens), hq, D)).astype(np.float32)
    gate = rng.standard_normal((len(lens), hq, D)).astype(np.float32)
    out = rt.tq_attn_decode(dev, to_dev(q), case.pool, case.pt_d,
                            to_dev(np.array(lens, np.int32)), gate=to_dev(gate)).cpu().numpy()
    assert np.all(out[0] == 0.0)
    for i in (1, 2):
        ref = case.oracle_out(i, q[i], gate=gate[i])
        err = row_rel_err(out[i], ref)
        assert err <= 1e-2, f"seq {i} (L={lens[i]}): rel err {err}"


def test_bad_arguments_raise():
    dev = device()
    for d in (257, 512):
        with pytest.raises(rt.Unsupported):
            rt.TqPool(dev, 4, 2, head_dim=d)
    pool = rt.TqPool(dev, 4, 2)
    q = torch.zeros((1, 3, D), dtype=torch.float32, device="cuda")
    with pytest.raises(rt.InvalidArg):  # 3 q heads over 2 kv heads: only the modulo map
        rt.tq_attn_decode(dev, q, pool, to_dev(np.zeros((1, 4), np.int32)),
                          to_dev(np.array([1], np.int32)), gqa_mode=1)


def test_append_records_bit_exact_d256():
    """head_dim 256 (config 4's attention layers): 128-byte records, chunked appends,
    magnitudes 1e-3 .. 1e3 and a zero key."""
    dev = device()
    rng = np.random.default_rng(0x70C4)

    def scale(r, shape):
        return 10.0 ** r.uniform(-3, 3, size=shape[:2] + (1,))
    case = TqCase(rng, [1, 16, 37, 130], 2, key_scale=scale, d=256)
    case.k[2][3, 0, :] = 0.0
    case.build(dev, chunk=11)
    for i in range(len(case.lens)):
        _check_records(case, i)


@pytest.mark.parametrize("gqa_mode", [0, 1])
def test_decode_c4_shape_d256_gate(gqa_mode):
    """Config-4 heads over a TurboQuant cache: 16 q / 2 kv heads, D 256, sigmoid gate, ragged
    contexts up to 4097 (the score scale is 1/sqrt(256))."""
    dev = device()
    rng = np.random.default_rng(0x70C5 + gqa_mode)
    lens = [4097, 1, 700, 64]
    hq, hkv = 16, 2
    case = TqCase(rng, lens, hkv, d=256)
    case.build(dev)
    q = rng.standard_normal((len(lens), hq, 256)).astype(np.float32) * 2
    gate = rng.standard_normal((len(lens), hq, 256)).astype(np.float32)
    out = rt.tq_attn_decode(dev, to_dev(q), case.pool, case.pt_d, to_dev(np.array(lens, np.int32)),
                            gqa_mode=gqa_mode, gate=to_dev(gate)).cpu().numpy()
    refs = parallel_map(lambda i: case.oracle_out(i, q[i], gqa_mode, gate[i]), range(len(lens)))
    for i in range(len(lens)):
        err = row_rel_err(out[i], refs[i])
        print(f"\nD 256 seq {i} (L={lens[i]}): rel err {err:.3e}")
        assert err <= 1e-2, f"seq {i} (L={lens[i]}): rel err {err}"

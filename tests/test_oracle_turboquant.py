"""Pins the TurboQuant restatement in oracle/ (src/turboquant/mod.rs).

Known answers: SplitMix64's published test vector, hand-derived bit packing,
the reference's own unit tests (src/turboquant/mod.rs:752-951: centroid
order/symmetry, orthogonality, reconstruction MSE, QJL dot accuracy, packing
round trips, compressed sizes, cache compression ratio).  Properties: the
QJL estimator is unbiased, the precomputed-query path equals the direct one,
and a float64 numpy evaluation of the cache attention from the unpacked
fields agrees with the f32 restatement.  The codebooks equal float64 Lloyd-Max
iteration for N(0,1), and every code and QJL sign of the quantizer equals a
float64 evaluation of its steps.  Planted slips (a sign slip in the QJL
correction, a dropped sqrt(d) scale) are caught.
"""
import numpy as np
import pytest

from oracle import oracle as o


def test_splitmix64_published_vector():
    # the reference generator's test vector for seed 1234567
    assert o.splitmix64(1234567, 5) == [6457827717110365317, 3203168211198807973,
                                        9817491932198370423, 4593380528125082431,
                                        16408922859458223821]


def _box_muller_f64(seed, n, trig=np.cos):
    """The reference's Gaussian (src/turboquant/mod.rs:733-746) recomputed in float64 numpy
    from SplitMix64 outputs (pinned above by the published vector): u = (x >> 11) / 2^53,
    g = sqrt(-2 ln max(u1, 1e-10)) * cos(2 pi u2), rounded to f32."""
    xs = np.array(o.splitmix64(seed, 2 * n), dtype=np.uint64)
    u = (xs >> np.uint64(11)).astype(np.float64) / 2.0 ** 53
    r = np.sqrt(-2.0 * np.log(np.maximum(u[0::2], 1e-10)))
    return (r * trig(2.0 * np.pi * u[1::2])).astype(np.float32)


def _ulps(a, b):
    ia, ib = (np.asarray(x, np.float32).view(np.int32).astype(np.int64) for x in (a, b))
    return np.abs(ia - ib)


@pytest.mark.parametrize("seed", [0xCAFEBABE, 0xCAFEBABE ^ 0xDEADBEEF, 1])
def test_box_muller_gaussians_match_float64_restatement(seed):
    """The oracle's f32 Gaussians equal an independent float64 evaluation of r cos(theta) to
    1 f32 ulp (the two libm's may round the f64 log / cos differently in the last bit); a
    sin-for-cos slip, the swapped uniforms or a dropped factor 2 in the radius does not."""
    n = 4096
    got = o.splitmix64_gaussians(seed, n)
    assert _ulps(got, _box_muller_f64(seed, n)).max() <= 1
    assert _ulps(got, _box_muller_f64(seed, n, np.sin)).max() > 1000
    xs = np.array(o.splitmix64(seed, 2 * n), dtype=np.uint64)
    u = (xs >> np.uint64(11)).astype(np.float64) / 2.0 ** 53
    swapped = (np.sqrt(-2.0 * np.log(np.maximum(u[1::2], 1e-10))) *
               np.cos(2.0 * np.pi * u[0::2])).astype(np.float32)
    assert _ulps(got, swapped).max() > 1000
    no_two = (np.sqrt(-np.log(np.maximum(u[0::2], 1e-10))) *
              np.cos(2.0 * np.pi * u[1::2])).astype(np.float32)
    assert _ulps(got, no_two).max() > 1000


@pytest.mark.parametrize("dim", [128, 256])
def test_product_matrices_from_float64_gaussians(dim):
    """The product's host generator (pi_tq_generate): the QJL matrix is the Gaussians of
    seed ^ 0xDEADBEEF row by row, and the rotation's first column is the first column of the
    seed's Gaussian matrix, normalised (Gram-Schmidt's first step), both from the float64
    restatement."""
    from powerinfer_x64_amd import runtime as rt
    seed = 0xCAFEBABE + 1
    R, G = rt.tq_generate(dim, seed)
    g = _box_muller_f64(seed ^ 0xDEADBEEF, dim * dim).reshape(dim, dim)
    assert _ulps(G, g).max() <= 1
    a = _box_muller_f64(seed, dim * dim).reshape(dim, dim).astype(np.float64)
    col = a[:, 0] / np.linalg.norm(a[:, 0])
    assert np.abs(R[:, 0] - col).max() < 1e-6


def test_box_muller_gaussians_are_standard_normal():
    x = o.splitmix64_gaussians(0xCAFEBABE, 200000).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    # kurtosis of a normal is 3
    assert abs(((x - x.mean()) ** 4).mean() / x.var() ** 2 - 3.0) < 0.05


def test_centroids_sorted_symmetric():
    # src/turboquant/mod.rs:752-769
    for bw in range(1, 5):
        c = o.tq_centroids(bw)
        assert c.size == 1 << bw
        assert np.all(np.diff(c) > 0)
        assert np.all(np.abs(c + c[::-1]) < 0.01)


@pytest.mark.parametrize("dim,seed", [(8, 42), (128, 0xCAFEBABE)])
def test_orthogonal_matrix(dim, seed):
    # src/turboquant/mod.rs:771-790 (dim 8, seed 42, 0.01) and the cache's dim
    q = o.tq_orthogonal(dim, seed).astype(np.float64)
    assert np.abs(q.T @ q - np.eye(dim)).max() < (0.01 if dim == 8 else 1e-4)


def test_bit_packing_known_bytes():
    # src/turboquant/mod.rs:896-916; bytes derived by hand, LSB first:
    # 2-bit codes 0,1,2,3 -> 0b11_10_01_00 = 0xE4; 1,0,3,2 -> 0b10_11_00_01 = 0xB1;
    # signs 1,0,1,1 -> 0b1101 = 0x0D
    idx = [0, 1, 2, 3, 1, 0, 3, 2]
    packed = o.tq_pack(idx, 2, [1, 0, 1, 1])
    assert list(packed) == [0xE4, 0xB1, 0x0D]
    i2, s2 = o.tq_unpack(packed, 8, 2, 4)
    assert list(i2) == idx and list(s2) == [1, 0, 1, 1]
    assert list(o.tq_pack(idx, 2)) == [0xE4, 0xB1]


def test_bit_packing_round_trip_3bit():
    rng = np.random.default_rng(1)
    idx = rng.integers(0, 8, 128).astype(np.uint8)
    sg = rng.integers(0, 2, 128).astype(np.uint8)
    packed = o.tq_pack(idx, 3, sg)
    assert packed.size == 64
    i2, s2 = o.tq_unpack(packed, 128, 3, 128)
    assert np.array_equal(i2, idx) and np.array_equal(s2, sg)
    # code i occupies bits 3i .. 3i+2
    bits = np.unpackbits(packed, bitorder="little")
    assert np.array_equal(bits[0:384:3] + 2 * bits[1:384:3] + 4 * bits[2:384:3], idx)
    assert np.array_equal(bits[384:], sg)


def test_odd_width_record_is_the_bit_stream():
    """At d = 33 pack_compressed (:591-617) emits ceil(4 d / 8) = 17 bytes: the 99 code bits,
    then the signs from bit 99 on (inside byte 12), while compressed_bytes() (:111-117) counts
    ceil(3 d / 8) + ceil(d / 8) = 18.  The oracle's quantizer writes the bit stream into an
    18-byte record whose last byte stays zero; the device records are the 17 stream bytes."""
    rng = np.random.default_rng(33)
    d = 33
    idx = rng.integers(0, 8, d).astype(np.uint8)
    sg = rng.integers(0, 2, d).astype(np.uint8)
    packed = o.tq_pack(idx, 3, sg)
    assert packed.size == 17 and o.tq_compressed_bytes(3, d, d) == 18
    bits = np.unpackbits(packed, bitorder="little")
    assert np.array_equal(bits[0:99:3] + 2 * bits[1:99:3] + 4 * bits[2:99:3], idx)
    assert np.array_equal(bits[99:132], sg) and not bits[132:].any()
    R, G = o.tq_matrices(d, 7)
    x = rng.standard_normal(d).astype(np.float32)
    x /= np.linalg.norm(x)
    q = o.tq_quantize(x, R, G, 3, d)
    assert q.size == 18 and q[17] == 0
    i2, s2 = o.tq_unpack(q[:17], d, 3, d)
    assert np.array_equal(o.tq_pack(i2, 3, s2), q[:17])


def test_compressed_sizes():
    # src/turboquant/mod.rs:918-951
    assert o.tq_compressed_bytes(3, 128, 128) == 64
    assert o.tq_compressed_bytes(4, 128, 128) == 80
    assert o.tq_compressed_bytes(3, 128, 0) == 48
    assert o.tq_compressed_bytes(4, 128, 0) == 64


@pytest.mark.parametrize("qjl", [16, 0])
def test_quantize_dequantize_mse(qjl):
    # src/turboquant/mod.rs:792-834
    dim = 16
    R, G = o.tq_matrices(dim, 123, qjl)
    x = np.sin(np.arange(dim, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    x = (x / np.sqrt((x * x).sum())).astype(np.float32)
    rec = o.tq_dequantize(o.tq_quantize(x, R, G, 3, qjl), R, 3)
    assert float(((x - rec) ** 2).mean()) < 0.2


def test_dot_accuracy_qjl():
    # src/turboquant/mod.rs:836-865: 50 random unit pairs, mean |err| < 0.15
    dim = 64
    R, G = o.tq_matrices(dim, 456)
    g = o.splitmix64_gaussians(789, 50 * 2 * dim).reshape(50, 2, dim)
    err = []
    for a, b in g:
        a = a / np.float32(np.sqrt((a * a).sum()))
        b = b / np.float32(np.sqrt((b * b).sum()))
        est = o.tq_dot(a, o.tq_quantize(b, R, G, 3, dim), R, G, 3, dim)
        err.append(abs(float(a @ b) - est))
    assert np.mean(err) < 0.15


def _estimator_errors(n, flip=False):
    dim = 64
    R, G = o.tq_matrices(dim, 7)
    rng = np.random.default_rng(3)
    errs = []
    for _ in range(n):
        a, b = rng.standard_normal((2, dim)).astype(np.float32)
        a /= np.linalg.norm(a)
        b /= np.linalg.norm(b)
        pk = o.tq_quantize(b, R, G, 3, dim)
        if flip:  # planted slip: every QJL sign inverted
            idx, sg = o.tq_unpack(pk, dim, 3, dim)
            pk = o.tq_pack(idx, 3, 1 - sg)
        errs.append(o.tq_dot(a, pk, R, G, 3, dim) - float(a @ b))
    return np.array(errs)


def test_qjl_estimator_unbiased_and_sign_slip_caught():
    e = _estimator_errors(400)
    assert abs(e.mean()) < 3 * e.std() / np.sqrt(e.size)
    bad = _estimator_errors(400, flip=True)
    assert np.abs(bad).mean() > 1.5 * np.abs(e).mean()


def test_precomputed_query_matches_direct_dot():
    dim = 128
    R, G = o.tq_matrices(dim, 0xCAFEBABE)
    rng = np.random.default_rng(5)
    qrot = np.zeros(dim, np.float32)
    qp = np.zeros(dim, np.float32)
    for _ in range(20):
        q = rng.standard_normal(dim).astype(np.float32)
        k = rng.standard_normal(dim).astype(np.float32)
        k /= np.linalg.norm(k)
        pk = o.tq_quantize(k, R, G, 3, dim)
        o.lib().or_tq_precompute_query(o._p(qrot), o._p(qp), o._p(q), o._p(o._f32(R)),
                                       o._p(o._f32(G)), dim, dim)
        a = float(o.lib().or_tq_dot_precomputed(o._p(qrot), o._p(qp),
                                                pk.ctypes.data_as(o._u8p), dim, 3, dim))
        b = o.tq_dot(q, pk, R, G, 3, dim)
        assert abs(a - b) <= 1e-5 * (1 + abs(b))


def _attend_f64(q, packed, norms, vals, R, G, kv_h):
    """float64 numpy evaluation of the cache attention from the unpacked fields."""
    T, n_kv, dim = vals.shape
    c = o.tq_centroids(3).astype(np.float64)
    R64, G64 = R.astype(np.float64), G.astype(np.float64)
    qr = R64 @ q.astype(np.float64)
    qp = (G64 @ qr) / np.sqrt(dim)
    qr /= np.sqrt(dim)
    rn = np.sqrt(0.043 / np.sqrt(dim))
    qs = np.sqrt(np.pi / (2 * dim))
    sc = np.zeros(T)
    for t in range(T):
        idx, sg = o.tq_unpack(packed[t, kv_h], dim, 3, dim)
        mse = qr @ c[idx]
        corr = rn * qs * (qp @ np.where(sg == 1, 1.0, -1.0))
        sc[t] = norms[t, kv_h] * (mse + corr) / np.sqrt(dim)
    w = np.exp(sc - sc.max())
    w /= w.sum()
    w[w < 1e-7] = 0.0
    return w @ vals[:, kv_h, :].astype(np.float64)


def test_cache_attention_matches_f64_evaluation():
    dim, n_kv, T = 128, 2, 40
    rng = np.random.default_rng(11)
    Rs, Gs = zip(*[o.tq_matrices(dim, 0xCAFEBABE + h) for h in range(n_kv)])
    R = np.stack(Rs)
    G = np.stack(Gs)
    keys = rng.standard_normal((T, n_kv, dim)).astype(np.float32)
    vals = rng.standard_normal((T, n_kv, dim)).astype(np.float16)
    packed = np.zeros((T, n_kv, 64), np.uint8)
    norms = np.zeros((T, n_kv), np.float32)
    for t in range(T):
        packed[t], norms[t] = o.tq_cache_append_keys(keys[t], R, G)
        assert np.allclose(norms[t], np.linalg.norm(keys[t].astype(np.float64), axis=1), rtol=1e-6)
    q = rng.standard_normal(dim).astype(np.float32) * 2
    for kv_h in range(n_kv):
        got = o.tq_cache_attend(q, packed, norms, vals, R[kv_h], G[kv_h], kv_h)
        ref = _attend_f64(q, packed, norms, vals, R[kv_h], G[kv_h], kv_h)
        assert np.abs(got - ref).max() < 1e-4


def test_cache_compression_ratio():
    # src/turboquant/mod.rs:867-894: 10 tokens, 2 heads, dim 16 -> ratio > 2
    T, n_kv, dim = 10, 2, 16
    mem = T * n_kv * (o.tq_compressed_bytes(3, dim, dim) + 4 + 2 * dim)
    assert T * n_kv * dim * 4 * 2 / mem > 2.0


def _lloyd_max_gaussian(levels, iters=3000):
    """Lloyd-Max quantizer of N(0,1) with `levels` levels in float64 (Max 1960): boundaries
    at the midpoints of adjacent centroids, each centroid the conditional mean of its cell,
    E[X | a < X < b] = (phi(a) - phi(b)) / (Phi(b) - Phi(a))."""
    from scipy.stats import norm
    c = np.linspace(-2.0, 2.0, levels)
    for _ in range(iters):
        b = np.concatenate(([-np.inf], (c[1:] + c[:-1]) / 2, [np.inf]))
        c = (norm.pdf(b[:-1]) - norm.pdf(b[1:])) / (norm.cdf(b[1:]) - norm.cdf(b[:-1]))
    return c


@pytest.mark.parametrize("bits", [1, 3, 4])
def test_centroids_are_the_gaussian_lloyd_max_levels(bits):
    """The 1-, 3- and 4-bit codebooks of src/turboquant/mod.rs:27-41 are Max's optimal
    quantizers of N(0,1), printed to 4 decimals: the oracle's tables equal float64 Lloyd
    iteration to that rounding.  (The reference's 2-bit table, +-0.4950 / +-1.4996, is not
    Max's +-0.4528 / +-1.5104; the oracle keeps the reference's values, and no path here
    quantizes at 2 bits.)"""
    got = o.tq_centroids(bits).astype(np.float64)
    assert np.abs(got - _lloyd_max_gaussian(1 << bits)).max() <= 6e-4


def test_two_bit_table_is_the_references_not_maxs():
    got = o.tq_centroids(2).astype(np.float64)
    assert np.allclose(got, [-1.4996, -0.4950, 0.4950, 1.4996], atol=1e-6)
    assert np.abs(got - _lloyd_max_gaussian(4)).max() > 0.04


def _quantize_f64(x, R, G, sqrt_d=True):
    """quantize_vector (src/turboquant/mod.rs:128-187) evaluated in float64: rotate, scale by
    sqrt(d) (sqrt_d=False plants the dropped-scale slip), nearest centroid with the first
    strict minimum winning, residual, QJL signs G.r >= 0.  Also returns, per coordinate and per
    sign, whether f32 rounding could flip the decision (within 1e-4 of a cell boundary, or a
    projection within 1e-3 of zero); those are left out of the comparison."""
    d = x.size
    c = o.tq_centroids(3).astype(np.float64)
    rot = R.astype(np.float64) @ x.astype(np.float64)
    if sqrt_d:
        rot *= np.sqrt(d)
    dist = np.abs(rot[:, None] - c[None, :])
    idx = np.argmin(dist, axis=1)  # the first of equal minima, as `dist < best_dist` keeps
    bounds = (c[1:] + c[:-1]) / 2
    amb_idx = np.abs(rot[:, None] - bounds[None, :]).min(axis=1) < 1e-4
    res = rot - c[idx]
    proj = G.astype(np.float64) @ res
    return idx.astype(np.uint8), (proj >= 0).astype(np.uint8), amb_idx, np.abs(proj) < 1e-3


@pytest.mark.parametrize("dim", [16, 128])
@pytest.mark.parametrize("seed", [0xCAFEBABE, 0xCAFEBABF, 7])
def test_quantizer_codes_match_float64_brute_force(dim, seed):
    """Every 3-bit code and QJL sign of or_tq_quantize equals the float64 evaluation of the
    reference's steps (away from the f32 rounding ties), and whole records are byte-identical
    to the float64 fields packed; the same check rejects a quantizer that drops the sqrt(d)
    scale before the nearest-centroid search, which a reconstruction-MSE bound accepts."""
    R, G = o.tq_matrices(dim, seed)
    rng = np.random.default_rng(seed & 0xFFFF)
    n_vec, n_amb, exact, slip_diff, slip_mse = 40, 0, 0, 0, []
    for _ in range(n_vec):
        x = rng.standard_normal(dim).astype(np.float32)
        x /= np.linalg.norm(x)
        pk = o.tq_quantize(x, R, G, 3, dim)
        idx_o, sg_o = o.tq_unpack(pk, dim, 3, dim)
        idx, sg, amb_i, amb_s = _quantize_f64(x, R, G)
        assert np.array_equal(idx_o[~amb_i], idx[~amb_i])
        assert np.array_equal(sg_o[~amb_s], sg[~amb_s])
        n_amb += int(amb_i.sum() + amb_s.sum())
        if not amb_i.any() and not amb_s.any():
            assert np.array_equal(pk, o.tq_pack(idx, 3, sg))
            exact += 1
        # planted slip: no sqrt(d) scale
        idx_b, _, _, _ = _quantize_f64(x, R, G, sqrt_d=False)
        slip_diff += int((idx_b != idx_o).sum())
        rec = o.tq_dequantize(o.tq_pack(idx_b, 3, np.zeros(dim, np.uint8)), R, 3)
        slip_mse.append(float(((rec - x) ** 2).mean()))
    assert n_amb <= 0.02 * n_vec * 2 * dim
    assert exact >= n_vec * 3 // 4
    assert slip_diff >= 0.3 * n_vec * dim
    if dim == 16:  # the slipped codes still pass the reconstruction bound of :792-834
        assert np.mean(slip_mse) < 0.2

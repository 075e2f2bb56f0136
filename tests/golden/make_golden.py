"""Writes tests/golden/kat.json: known-answer vectors for the attention path.

Inputs are the ones the reference's own tests use (cited per entry); expected
outputs are computed here in float64 from the closed form each test implies
(never from the oracle under test), so the fixture pins the oracle.

Run:  python tests/golden/make_golden.py
"""
import json
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def softmax64(x):
    x = np.asarray(x, dtype=np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()


def attn64(q, k, v):
    q, k, v = (np.asarray(a, dtype=np.float64) for a in (q, k, v))
    w = softmax64(k @ q / math.sqrt(q.size))
    return w @ v, w


def main():
    kat = {}
    # src/simd.rs:247-256 and :258-265
    kat["dot_product"] = [
        {"a": [1, 2, 3, 4, 5, 6, 7, 8], "b": [8, 7, 6, 5, 4, 3, 2, 1], "expected": 120.0},
        {"a": [1, 2, 3, 4, 5], "b": [5, 4, 3, 2, 1], "expected": 35.0},
    ]
    # src/simd.rs:297-303 and :305-311
    kat["sum_squares"] = [{"a": [1, 2, 3, 4], "expected": 30.0}]
    kat["scale"] = [{"a": [1, 2, 3, 4, 5], "s": 2.0, "expected": [2, 4, 6, 8, 10]}]
    # src/ops.rs:303-315: out = x / sqrt(mean(x^2) + eps)
    x = np.array([1, 2, 3, 4], dtype=np.float64)
    kat["rms_norm"] = [{"x": x.tolist(), "w": [1, 1, 1, 1], "eps": 1e-6,
                        "expected": (x / math.sqrt((x * x).mean() + 1e-6)).tolist()}]
    # src/ops.rs:317-327
    kat["softmax"] = [{"x": [1, 2, 3], "expected": softmax64([1, 2, 3]).tolist()}]
    # src/ops.rs:373-383 and tests/smoke.rs:46-53: position 0 is the identity
    kat["rope_pos0"] = [{"q": [1, 2, 3, 4], "k": [5, 6, 7, 8], "head_dim": 4, "rope_dim": 4,
                         "base": 10000.0}]
    # src/ops.rs:340-357 (the comment at :358-361 quoting 0.622 is wrong: 3 keys, not 2)
    q = [1, 0, 0, 0]
    k3 = [[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0]]
    v3 = [[10, 0, 0, 0], [0, 20, 0, 0], [0, 0, 30, 0]]
    o3, w3 = attn64(q, k3, v3)
    # tests/smoke.rs:56-61
    k2 = [[1, 0, 0, 0], [0, 1, 0, 0]]
    v2 = [[10, 0, 0, 0], [0, 20, 0, 0]]
    o2, w2 = attn64(q, k2, v2)
    # tests/soak.rs:126-143 (input pattern; expected by float64 brute force)
    hd, sl = 64, 32
    qs = np.sin(np.arange(hd, dtype=np.float32) * np.float32(0.1))
    ks = np.cos(np.arange(sl * hd, dtype=np.float32) * np.float32(0.01)).reshape(sl, hd)
    vs = np.sin(np.arange(sl * hd, dtype=np.float32) * np.float32(0.02)).reshape(sl, hd)
    os_, _ = attn64(qs, ks, vs)
    kat["attention_head"] = [
        {"src": "src/ops.rs:340-357", "q": q, "k": k3, "v": v3, "weights": w3.tolist(),
         "expected": o3.tolist()},
        {"src": "tests/smoke.rs:56-61", "q": q, "k": k2, "v": v2, "weights": w2.tolist(),
         "expected": o2.tolist()},
        {"src": "tests/soak.rs:126-143", "q": qs.astype(np.float64).tolist(),
         "k": ks.astype(np.float64).tolist(), "v": vs.astype(np.float64).tolist(),
         "expected": os_.tolist()},
    ]
    # src/bin/layer_trace.rs:180-196: from zero state o = beta * (q_hat . k_hat) * v,
    # q_hat = q/|q|/sqrt(Dk), k_hat = k/|k|.
    rng = np.random.default_rng(1234)
    hk, hv, dk, dv = 2, 4, 8, 8
    qr = rng.standard_normal((hk, dk)).astype(np.float32)
    kr = rng.standard_normal((hk, dk)).astype(np.float32)
    vv = rng.standard_normal((hv, dv)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal(hv)))).astype(np.float32)
    g = (-np.log1p(np.exp(rng.standard_normal(hv)))).astype(np.float32)
    exp = np.zeros((hv, dv))
    for h in range(hv):
        qq = qr[h % hk].astype(np.float64)
        kk = kr[h % hk].astype(np.float64)
        qq = qq / np.linalg.norm(qq) / math.sqrt(dk)
        kk = kk / np.linalg.norm(kk)
        exp[h] = beta[h] * (qq @ kk) * vv[h]
    kat["gdn_zero_state"] = [{"src": "src/bin/layer_trace.rs:180-196", "hk": hk, "hv": hv,
                              "dk": dk, "dv": dv, "q": qr.tolist(), "k": kr.tolist(),
                              "v": vv.tolist(), "beta": beta.tolist(), "g": g.tolist(),
                              "expected": exp.tolist()}]
    with open(os.path.join(HERE, "kat.json"), "w") as f:
        json.dump(kat, f, indent=1)


if __name__ == "__main__":
    main()

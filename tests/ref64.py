"""Float64 textbook formulas used to pin the oracle on tiny shapes.

These are independent of the oracle's loop structure: vectorised numpy in
float64 written from the mathematics (softmax attention, rotary embedding as a
2x2 rotation, the gated delta rule in its chunked WY matrix form).
"""
import math

import numpy as np


def softmax(x, axis=-1):
    x = np.asarray(x, dtype=np.float64)
    e = np.exp(x - x.max(axis=axis, keepdims=True))
    return e / e.sum(axis=axis, keepdims=True)


def attention(q, k, v, kv_of_head):
    """q [Hq,D], k/v [T,Hkv,D]; kv_of_head(h) -> kv head index."""
    q, k, v = (np.asarray(a, dtype=np.float64) for a in (q, k, v))
    out = np.zeros((q.shape[0], v.shape[2]))
    for h in range(q.shape[0]):
        kh = kv_of_head(h)
        w = softmax(k[:, kh, :] @ q[h] / math.sqrt(q.shape[1]))
        out[h] = w @ v[:, kh, :]
    return out


def rope_adjacent(x, pos, rope_dim, base):
    """Rotate pairs (2i, 2i+1) by pos * base^(-2i/rope_dim)."""
    x = np.array(x, dtype=np.float64, copy=True)
    for i in range(rope_dim // 2):
        th = pos * base ** (-2.0 * i / rope_dim)
        a, b = x[..., 2 * i].copy(), x[..., 2 * i + 1].copy()
        x[..., 2 * i] = a * math.cos(th) - b * math.sin(th)
        x[..., 2 * i + 1] = a * math.sin(th) + b * math.cos(th)
    return x


def rope_neox(x, pos, n_rot, base):
    """Rotate pairs (i, i + n_rot/2) by pos * base^(-2i/n_rot); dims >= n_rot untouched."""
    x = np.array(x, dtype=np.float64, copy=True)
    half = n_rot // 2
    for i in range(half):
        th = pos * base ** (-2.0 * i / n_rot)
        a, b = x[..., i].copy(), x[..., i + half].copy()
        x[..., i] = a * math.cos(th) - b * math.sin(th)
        x[..., i + half] = a * math.sin(th) + b * math.cos(th)
    return x


def rms_norm(x, w, eps):
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def gdn_prepare(q_raw, k_raw, n_v_heads):
    """Tile K heads to V heads (vh -> vh % Hk), L2-normalise, scale q by 1/sqrt(Dk)."""
    q_raw = np.asarray(q_raw, dtype=np.float64)
    k_raw = np.asarray(k_raw, dtype=np.float64)
    hk, dk = q_raw.shape[-2:]
    idx = np.arange(n_v_heads) % hk
    q = q_raw[..., idx, :]
    k = k_raw[..., idx, :]
    q = q / np.maximum(np.linalg.norm(q, axis=-1, keepdims=True), 1e-12) / math.sqrt(dk)
    k = k / np.maximum(np.linalg.norm(k, axis=-1, keepdims=True), 1e-12)
    return q, k


def gdn_chunk_wy(q, k, v, beta, g, S0):
    """One chunk of the gated delta rule in closed (WY) form, one head.

    q,k [C,Dk] (prepared), v [C,Dv], beta/g [C], S0 [Dk,Dv].  With gamma_i =
    exp(sum_{j<=i} g_j): (I + A) Delta = diag(beta) (V - diag(gamma) K S0),
    A_ij = beta_i (gamma_i/gamma_j) k_i.k_j for j < i;  O = diag(gamma) Q S0 +
    (M o Q K^T) Delta with M_ij = gamma_i/gamma_j for j <= i;  S_C = gamma_C S0 +
    K^T diag(gamma_C/gamma) Delta.
    """
    q, k, v, beta, g, S0 = (np.asarray(a, dtype=np.float64) for a in (q, k, v, beta, g, S0))
    c = q.shape[0]
    lg = np.cumsum(g)
    ratio = np.exp(lg[:, None] - lg[None, :])
    A = np.tril(beta[:, None] * ratio * (k @ k.T), -1)
    rhs = beta[:, None] * (v - np.exp(lg)[:, None] * (k @ S0))
    delta = np.linalg.solve(np.eye(c) + A, rhs)
    M = np.tril(ratio)
    O = np.exp(lg)[:, None] * (q @ S0) + (M * (q @ k.T)) @ delta
    S = np.exp(lg[-1]) * S0 + k.T @ (np.exp(lg[-1] - lg)[:, None] * delta)
    return O, S


def ssm_forward(x, conv1d, a, dt_bias, alpha, beta, out_w, state, d_inner, d_state, d_conv):
    """Mamba-2-style selective scan of one token in float64 matrix form: conv taps as a
    row-sum scale, dt = softplus(bias + alpha u) (0 below -20, identity above 20),
    S = exp(-dt * exp(A)) * S + dt B u, y = W^T-free projection of the column sums."""
    x = np.asarray(x, np.float64)
    w = np.asarray(conv1d, np.float64)
    u = x * w.reshape(d_inner, d_conv).sum(axis=1) if w.size == d_inner * d_conv else x.copy()
    z = np.asarray(dt_bias, np.float64) + np.asarray(alpha, np.float64).reshape(d_inner, d_inner) @ u
    dt = np.where(z > 20, z, np.where(z < -20, 0.0, np.log1p(np.exp(np.minimum(z, 20)))))
    b = np.asarray(beta, np.float64)
    bvals = (b.reshape(d_state, d_inner) @ u)[:, None] if (d_state and b.size == d_state * d_inner) \
        else u[None, :]
    S = np.asarray(state, np.float64).reshape(d_state, d_inner)
    A = np.asarray(a, np.float64).reshape(d_state, d_inner)
    S = np.exp(-dt[None, :] * np.exp(A)) * S + dt[None, :] * bvals * u[None, :]
    col = S.sum(axis=0)
    o = np.asarray(out_w, np.float64)
    y = o.reshape(d_inner, d_inner) @ col if o.size == d_inner * d_inner else col
    return y, S.reshape(-1)

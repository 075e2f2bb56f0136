/*
 * oracle.c -- CPU restatement of PowerInfer_x64's attention + gated-DeltaNet path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and timed CPU baseline); the
 * product never links or loads it.  Build: oracle/Makefile
 * (gcc -O3 -msse4.1 -ffp-contract=off).  Each function cites the reference
 * function it restates; see oracle.h for the contract of every entry.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* The reference's SSE horizontal sum (src/simd.rs:43-53):
 * movehdup + add gives [a+b, ., c+d, .]; movehl + add_ss gives (a+b)+(c+d). */
static float hsum4(const float l[4]) { return (l[0] + l[1]) + (l[2] + l[3]); }

float or_dot_product(const float* a, const float* b, size_t n) {
    /* src/simd.rs:14-40: four lane accumulators, sum += a*b (mul then add). */
    float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    size_t i = 0;
    for (; i + 4 <= n; i += 4) {
        for (int j = 0; j < 4; ++j) {
            float p = a[i + j] * b[i + j];
            lane[j] = lane[j] + p;
        }
    }
    float r = hsum4(lane);
    for (; i < n; ++i) r += a[i] * b[i];
    return r;
}

float or_sum_squares(const float* a, size_t n) {
    /* src/simd.rs:115-135 */
    float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    size_t i = 0;
    for (; i + 4 <= n; i += 4) {
        for (int j = 0; j < 4; ++j) {
            float p = a[i + j] * a[i + j];
            lane[j] = lane[j] + p;
        }
    }
    float r = hsum4(lane);
    for (; i < n; ++i) r += a[i] * a[i];
    return r;
}

void or_scale(float* out, const float* a, float s, size_t n) {
    /* src/simd.rs:139-156 */
    for (size_t i = 0; i < n; ++i) out[i] = a[i] * s;
}

void or_rms_norm(float* out, const float* x, const float* w, size_t n, float eps) {
    /* src/ops.rs:13-27: rms = sqrt(sum_sq/n + eps); out = (x * (1/rms)) * w. */
    float sum_sq = or_sum_squares(x, n);
    float rms = sqrtf(sum_sq / (float)n + eps);
    float inv_rms = 1.0f / rms;
    or_scale(out, x, inv_rms, n);
    for (size_t i = 0; i < n; ++i) out[i] *= w[i];
}

void or_apply_rope(float* q, float* k, size_t position, size_t head_dim, size_t rope_dim,
                   float base) {
    /* src/ops.rs:35-67: freq_i = 1/base^(2i/rope_dim) in f32; theta = pos * freq. */
    size_t half = rope_dim / 2;
    for (size_t i = 0; i < half; ++i) {
        float expo = 2.0f * (float)i / (float)rope_dim;
        float freq = 1.0f / powf(base, expo);
        float theta = (float)position * freq;
        float c = cosf(theta);
        float s = sinf(theta);
        if (2 * i + 1 < head_dim) {
            float q0 = q[2 * i], q1 = q[2 * i + 1];
            q[2 * i] = q0 * c - q1 * s;
            q[2 * i + 1] = q0 * s + q1 * c;
        }
        if (2 * i + 1 < head_dim) {
            float k0 = k[2 * i], k1 = k[2 * i + 1];
            k[2 * i] = k0 * c - k1 * s;
            k[2 * i + 1] = k0 * s + k1 * c;
        }
    }
}

void or_compute_imrope_freqs(float base, size_t n_rot, const int32_t sections[4], float* freqs) {
    /* src/ops.rs:78-122: theta_scale = base^(-2/n_rot); four tracks that all
     * start at 1 and advance by one f32 multiply per pair, so every track
     * holds theta_scale^k obtained by repeated multiplication. */
    float theta_scale = powf(base, -2.0f / (float)n_rot);
    size_t sect_dims = (size_t)(sections[0] + sections[1] + sections[2] + sections[3]);
    size_t n_pairs = n_rot / 2;
    float t_t = 1.0f, t_h = 1.0f, t_w = 1.0f, t_e = 1.0f;
    for (size_t pair = 0; pair < n_pairs; ++pair) {
        size_t sector = sect_dims > 0 ? pair % sect_dims : pair;
        float theta;
        if (sector % 3 == 0 && sector < 3 * (size_t)sections[0])
            theta = t_t;
        else if (sector % 3 == 1 && sector < 3 * (size_t)sections[1])
            theta = t_h;
        else if (sector % 3 == 2 && sector < 3 * (size_t)sections[2])
            theta = t_w;
        else
            theta = t_e;
        freqs[pair] = theta;
        t_t *= theta_scale;
        t_h *= theta_scale;
        t_w *= theta_scale;
        t_e *= theta_scale;
    }
}

void or_apply_rope_with_freqs(float* q, float* k, size_t position, size_t head_dim,
                              const float* freqs, size_t n_freqs) {
    /* src/ops.rs:130-157 */
    size_t half = n_freqs;
    for (size_t i = 0; i < n_freqs; ++i) {
        float theta = (float)position * freqs[i];
        float c = cosf(theta);
        float s = sinf(theta);
        if (i + half < head_dim) {
            float q0 = q[i], q1 = q[i + half];
            q[i] = q0 * c - q1 * s;
            q[i + half] = q0 * s + q1 * c;
        }
        if (i + half < head_dim) {
            float k0 = k[i], k1 = k[i + half];
            k[i] = k0 * c - k1 * s;
            k[i + half] = k0 * s + k1 * c;
        }
    }
}

void or_softmax(float* x, size_t n) {
    /* src/ops.rs:160-180: max fold, exp(x-max) with a sequential f32 sum, x *= 1/sum. */
    if (n == 0) return;
    float max_val = -INFINITY;
    for (size_t i = 0; i < n; ++i) max_val = fmaxf(max_val, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - max_val);
        sum += x[i];
    }
    float inv_sum = 1.0f / sum;
    for (size_t i = 0; i < n; ++i) x[i] *= inv_sum;
}

void or_attention_head(float* out, const float* q, const float* k_cache, const float* v_cache,
                       size_t seq_len, size_t head_dim) {
    /* src/ops.rs:213-247 -- scalar dot (not the SSE one), scores * scale, softmax, t-outer V sum. */
    float scale = 1.0f / sqrtf((float)head_dim);
    float* scores = (float*)malloc((seq_len ? seq_len : 1) * sizeof(float));
    for (size_t t = 0; t < seq_len; ++t) {
        float dot = 0.0f;
        for (size_t d = 0; d < head_dim; ++d) dot += q[d] * k_cache[t * head_dim + d];
        scores[t] = dot * scale;
    }
    or_softmax(scores, seq_len);
    for (size_t d = 0; d < head_dim; ++d) out[d] = 0.0f;
    for (size_t t = 0; t < seq_len; ++t)
        for (size_t d = 0; d < head_dim; ++d) out[d] += scores[t] * v_cache[t * head_dim + d];
    free(scores);
}

void or_attn_decode(float* out, const float* q, size_t q_head_dim, const float* key_cache,
                    const float* value_cache, size_t total_seq, size_t n_heads, size_t n_kv_heads,
                    size_t kv_head_dim, size_t v_head_dim) {
    /* src/model/mod.rs:1154-1190 (f32 cache path). */
    float scale = 1.0f / sqrtf((float)kv_head_dim);
    float* scores = (float*)malloc((total_seq ? total_seq : 1) * sizeof(float));
    size_t n = kv_head_dim < v_head_dim ? kv_head_dim : v_head_dim;
    for (size_t h = 0; h < n_heads; ++h) {
        size_t kv_h = h % n_kv_heads; /* modulo GQA, :1155 */
        const float* q_attn = q + h * q_head_dim;
        for (size_t t = 0; t < total_seq; ++t) {
            const float* ks = key_cache + t * n_kv_heads * kv_head_dim + kv_h * kv_head_dim;
            scores[t] = or_dot_product(q_attn, ks, kv_head_dim) * scale;
        }
        or_softmax(scores, total_seq);
        float* ho = out + h * kv_head_dim;
        for (size_t d = 0; d < kv_head_dim; ++d) ho[d] = 0.0f;
        for (size_t t = 0; t < total_seq; ++t) {
            float w = scores[t];
            const float* vs = value_cache + t * n_kv_heads * v_head_dim + kv_h * v_head_dim;
            for (size_t d = 0; d < n; ++d) ho[d] += w * vs[d];
        }
    }
    free(scores);
}

void or_apply_gate(float* out, const float* gate, size_t n) {
    /* src/model/mod.rs:1192-1196 */
    for (size_t i = 0; i < n; ++i) {
        float s = 1.0f / (1.0f + expf(-gate[i]));
        out[i] *= s;
    }
}

/* The Q/K norm + RoPE part of one token (src/model/mod.rs:1035-1138). */
static void prepare_token(float* qt, float* kt, size_t n_heads, size_t n_kv_heads,
                          size_t q_head_dim, size_t kv_head_dim, const float* q_norm_w,
                          const float* k_norm_w, float eps, size_t attn_rope_dim,
                          float rope_base, const float* freqs, size_t n_attn_freqs,
                          size_t abs_pos, float* tmp, float* dummy_k) {
    size_t norm_end = kv_head_dim < q_head_dim ? kv_head_dim : q_head_dim;
    /* Q/K RMSNorm (:1035-1070): first norm_end dims of each Q head, whole K head. */
    if (q_norm_w && qt)
        for (size_t h = 0; h < n_heads; ++h) {
            or_rms_norm(tmp, qt + h * q_head_dim, q_norm_w, norm_end, eps);
            memcpy(qt + h * q_head_dim, tmp, norm_end * sizeof(float));
        }
    if (k_norm_w && kt)
        for (size_t h = 0; h < n_kv_heads; ++h) {
            or_rms_norm(tmp, kt + h * kv_head_dim, k_norm_w, kv_head_dim, eps);
            memcpy(kt + h * kv_head_dim, tmp, kv_head_dim * sizeof(float));
        }
    /* RoPE driver (:1072-1138): every Q head; K head h only when h < n_kv_heads. */
    for (size_t h = 0; h < n_heads; ++h) {
        float* qh = qt ? qt + h * q_head_dim : NULL;
        float* kh = (kt && h < n_kv_heads) ? kt + (h % n_kv_heads) * kv_head_dim : NULL;
        if (!qh) {
            memset(tmp, 0, kv_head_dim * sizeof(float));
            qh = tmp;
        }
        if (!kh) memset(dummy_k, 0, kv_head_dim * sizeof(float));
        float* kk = kh ? kh : dummy_k;
        if (freqs)
            or_apply_rope_with_freqs(qh, kk, abs_pos, kv_head_dim, freqs, n_attn_freqs);
        else
            or_apply_rope(qh, kk, abs_pos, kv_head_dim, attn_rope_dim, rope_base);
    }
}

static size_t cap_rope(size_t rope_dim, size_t kv_head_dim) {
    return rope_dim < kv_head_dim ? rope_dim : kv_head_dim;
}

void or_attn_prepare(float* q, float* k, size_t n_tokens, size_t n_heads, size_t n_kv_heads,
                     size_t q_head_dim, size_t kv_head_dim, const float* q_norm_w,
                     const float* k_norm_w, float eps, size_t rope_dim, float rope_base,
                     const float* freqs, size_t n_freqs, size_t pos0) {
    size_t attn_rope_dim = cap_rope(rope_dim, kv_head_dim);
    size_t n_attn_freqs = freqs ? attn_rope_dim / 2 : 0;
    if (n_attn_freqs > n_freqs) n_attn_freqs = n_freqs;
    size_t mx = kv_head_dim > q_head_dim ? kv_head_dim : q_head_dim;
    float* tmp = (float*)malloc(mx * sizeof(float));
    float* dummy_k = (float*)calloc(kv_head_dim, sizeof(float));
    for (size_t pos = 0; pos < n_tokens; ++pos)
        prepare_token(q ? q + pos * n_heads * q_head_dim : NULL,
                      k ? k + pos * n_kv_heads * kv_head_dim : NULL, n_heads, n_kv_heads,
                      q_head_dim, kv_head_dim, q_norm_w, k_norm_w, eps, attn_rope_dim, rope_base,
                      freqs, n_attn_freqs, pos0 + pos, tmp, dummy_k);
    free(tmp);
    free(dummy_k);
}

void or_attn_layer_tokens(float* out, float* q, const float* gate, float* k, const float* v,
                          size_t n_tokens, size_t n_heads, size_t n_kv_heads, size_t q_head_dim,
                          size_t kv_head_dim, size_t v_head_dim, const float* q_norm_w,
                          const float* k_norm_w, float eps, size_t rope_dim, float rope_base,
                          const float* freqs, size_t n_freqs, float* key_cache,
                          float* value_cache, size_t prev_seq_len) {
    size_t attn_rope_dim = cap_rope(rope_dim, kv_head_dim);
    size_t n_attn_freqs = freqs ? attn_rope_dim / 2 : 0;
    if (n_attn_freqs > n_freqs) n_attn_freqs = n_freqs;
    size_t mx = kv_head_dim > q_head_dim ? kv_head_dim : q_head_dim;
    float* tmp = (float*)malloc(mx * sizeof(float));
    float* dummy_k = (float*)calloc(kv_head_dim, sizeof(float));
    for (size_t pos = 0; pos < n_tokens; ++pos) {
        float* qt = q + pos * n_heads * q_head_dim;
        float* kt = k + pos * n_kv_heads * kv_head_dim;
        const float* vt = v + pos * n_kv_heads * v_head_dim;
        size_t t_idx = prev_seq_len + pos;
        prepare_token(qt, kt, n_heads, n_kv_heads, q_head_dim, kv_head_dim, q_norm_w, k_norm_w,
                      eps, attn_rope_dim, rope_base, freqs, n_attn_freqs, t_idx, tmp, dummy_k);
        /* Append-then-attend (:1140-1148). */
        memcpy(key_cache + t_idx * n_kv_heads * kv_head_dim, kt,
               n_kv_heads * kv_head_dim * sizeof(float));
        memcpy(value_cache + t_idx * n_kv_heads * v_head_dim, vt,
               n_kv_heads * v_head_dim * sizeof(float));
        float* ot = out + pos * n_heads * kv_head_dim;
        or_attn_decode(ot, qt, q_head_dim, key_cache, value_cache, t_idx + 1, n_heads, n_kv_heads,
                       kv_head_dim, v_head_dim);
        if (gate) or_apply_gate(ot, gate + pos * n_heads * q_head_dim, n_heads * kv_head_dim);
    }
    free(tmp);
    free(dummy_k);
}

void or_gdn_gates(float* beta, float* g, const float* beta_raw, const float* a_raw,
                  const float* ssm_a, const float* dt_bias, size_t n_v_heads) {
    /* src/model/mod.rs:806-809 (beta) and :826-839 (g). */
    for (size_t h = 0; h < n_v_heads; ++h) beta[h] = 1.0f / (1.0f + expf(-beta_raw[h]));
    for (size_t h = 0; h < n_v_heads; ++h) {
        float sp_in = a_raw[h] + dt_bias[h];
        float sp = sp_in > 10.0f ? sp_in : logf(1.0f + expf(sp_in));
        g[h] = ssm_a[h] * sp;
    }
}

/* Iterator::sum::<f32>() over x*x: a sequential left fold. */
static float seq_sum_sq(const float* x, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += x[i] * x[i];
    return s;
}

void or_gdn_step(float* out, float* state, const float* q_raw, const float* k_raw, const float* v,
                 const float* beta, const float* g, size_t n_k_heads, size_t n_v_heads,
                 size_t k_hd, size_t v_hd) {
    float* qh = (float*)malloc(k_hd * sizeof(float));
    float* kh = (float*)malloc(k_hd * sizeof(float));
    float* kv_mem = (float*)malloc(v_hd * sizeof(float));
    float q_scale = 1.0f / sqrtf((float)k_hd); /* :859 */
    for (size_t vh = 0; vh < n_v_heads; ++vh) {
        /* Tiled repeat (:845-853): V head vh reads K head vh % n_k_heads. */
        size_t src = (vh % n_k_heads) * k_hd;
        memcpy(qh, q_raw + src, k_hd * sizeof(float));
        memcpy(kh, k_raw + src, k_hd * sizeof(float));
        /* L2 norm with max(norm, 1e-12), q additionally scaled (:860-875). */
        float nq = sqrtf(seq_sum_sq(qh, k_hd));
        if (nq < 1e-12f) nq = 1e-12f;
        for (size_t i = 0; i < k_hd; ++i) qh[i] = qh[i] / nq * q_scale;
        float nk = sqrtf(seq_sum_sq(kh, k_hd));
        if (nk < 1e-12f) nk = 1e-12f;
        for (size_t i = 0; i < k_hd; ++i) kh[i] /= nk;

        /* Delta rule (:883-916). */
        float decay = expf(g[vh]);
        float beta_h = beta[vh];
        const float* v_h = v + vh * v_hd;
        float* S = state + vh * k_hd * v_hd;
        for (size_t i = 0; i < k_hd * v_hd; ++i) S[i] *= decay;
        for (size_t vi = 0; vi < v_hd; ++vi) kv_mem[vi] = 0.0f;
        for (size_t ki = 0; ki < k_hd; ++ki) {
            float kval = kh[ki];
            const float* row = S + ki * v_hd;
            for (size_t vi = 0; vi < v_hd; ++vi) kv_mem[vi] += row[vi] * kval;
        }
        float* o = out + vh * v_hd;
        for (size_t vi = 0; vi < v_hd; ++vi) o[vi] = 0.0f;
        for (size_t ki = 0; ki < k_hd; ++ki) {
            float kval = kh[ki], qval = qh[ki];
            float* row = S + ki * v_hd;
            for (size_t vi = 0; vi < v_hd; ++vi) {
                float delta = (v_h[vi] - kv_mem[vi]) * beta_h;
                row[vi] += kval * delta;
                o[vi] += row[vi] * qval;
            }
        }
    }
    free(qh);
    free(kh);
    free(kv_mem);
}

void or_gdn_tokens(float* out, float* state, const float* q_raw, const float* k_raw,
                   const float* v, const float* beta, const float* g, size_t n_tokens,
                   size_t n_k_heads, size_t n_v_heads, size_t k_hd, size_t v_hd) {
    for (size_t t = 0; t < n_tokens; ++t)
        or_gdn_step(out + t * n_v_heads * v_hd, state, q_raw + t * n_k_heads * k_hd,
                    k_raw + t * n_k_heads * k_hd, v + t * n_v_heads * v_hd, beta + t * n_v_heads,
                    g + t * n_v_heads, n_k_heads, n_v_heads, k_hd, v_hd);
}

void or_rmsnorm_gated(float* o, const float* z, const float* w, size_t n_v_heads, size_t v_hd,
                      float eps) {
    /* src/model/mod.rs:918-932 */
    for (size_t vh = 0; vh < n_v_heads; ++vh) {
        float* oh = o + vh * v_hd;
        const float* zh = z + vh * v_hd;
        float var = seq_sum_sq(oh, v_hd) / (float)v_hd;
        float scale = 1.0f / sqrtf(var + eps);
        for (size_t i = 0; i < v_hd; ++i) {
            float normed = oh[i] * scale * w[i];
            float zv = zh[i];
            float silu_z = zv / (1.0f + expf(-zv));
            oh[i] = normed * silu_z;
        }
    }
}

void or_conv1d_silu(float* x, float* hist, const float* w, size_t conv_dim, size_t d_conv) {
    /* src/model/mod.rs:750-776: window = the d_conv-1 previous raw inputs plus
     * this one, oldest first; w[i*d_conv + k] multiplies window[k][i]. */
    size_t nh = d_conv - 1;
    for (size_t i = 0; i < conv_dim; ++i) {
        float raw = x[i];
        float val = 0.0f;
        for (size_t kk = 0; kk < d_conv; ++kk) {
            float cs = kk < nh ? hist[kk * conv_dim + i] : raw;
            val += w[i * d_conv + kk] * cs;
        }
        /* shift the raw input into the history */
        for (size_t kk = 0; kk + 1 < nh; ++kk) hist[kk * conv_dim + i] = hist[(kk + 1) * conv_dim + i];
        if (nh > 0) hist[(nh - 1) * conv_dim + i] = raw;
        x[i] = val / (1.0f + expf(-val));
    }
}

void or_ssm_forward(float* y, const float* x, const float* conv1d, size_t conv1d_len,
                    const float* ssm_a, const float* dt_bias, const float* alpha,
                    const float* beta, size_t beta_len, const float* out_w, size_t out_len,
                    float* state, size_t d_inner, size_t d_state, size_t d_conv) {
    float* conv_out = (float*)calloc(d_inner ? d_inner : 1, sizeof(float));
    float* dt = (float*)calloc(d_inner ? d_inner : 1, sizeof(float));
    float* b_vals = (float*)calloc(d_state ? d_state : 1, sizeof(float));
    /* Step 1 (:63-74): every tap multiplies the current input, or pass-through. */
    if (conv1d_len == d_inner * d_conv) {
        for (size_t i = 0; i < d_inner; ++i) {
            float sum = 0.0f;
            for (size_t k = 0; k < d_conv; ++k) sum += x[i] * conv1d[i * d_conv + k];
            conv_out[i] = sum;
        }
    } else {
        memcpy(conv_out, x, d_inner * sizeof(float));
    }
    /* dt (:85-99): softplus with cut-offs at +-20. */
    for (size_t i = 0; i < d_inner; ++i) {
        float sum = dt_bias[i];
        for (size_t j = 0; j < d_inner; ++j) sum += conv_out[j] * alpha[i * d_inner + j];
        dt[i] = sum > 20.0f ? sum : (sum < -20.0f ? 0.0f : logf(1.0f + expf(sum)));
    }
    /* B (:102-110) */
    int has_b = beta_len == d_state * d_inner && d_state > 0;
    if (has_b)
        for (size_t s = 0; s < d_state; ++s) {
            float sum = 0.0f;
            for (size_t j = 0; j < d_inner; ++j) sum += conv_out[j] * beta[s * d_inner + j];
            b_vals[s] = sum;
        }
    /* discretise and scan (:113-128) */
    for (size_t s = 0; s < d_state; ++s)
        for (size_t i = 0; i < d_inner; ++i) {
            size_t idx = s * d_inner + i;
            float b_val = has_b ? b_vals[s] : conv_out[i];
            float a_discrete = expf(-dt[i] * expf(ssm_a[idx]));
            float b_discrete = dt[i] * b_val;
            state[idx] = a_discrete * state[idx] + b_discrete * conv_out[i];
        }
    /* output (:131-155) */
    for (size_t i = 0; i < d_inner; ++i) y[i] = 0.0f;
    if (out_len == d_inner * d_inner) {
        for (size_t i = 0; i < d_inner; ++i) {
            float sum = 0.0f;
            for (size_t s = 0; s < d_state; ++s) sum += state[s * d_inner + i];
            for (size_t j = 0; j < d_inner; ++j) y[j] += sum * out_w[j * d_inner + i];
        }
    } else {
        for (size_t i = 0; i < d_inner; ++i) {
            float sum = 0.0f;
            for (size_t s = 0; s < d_state; ++s) sum += state[s * d_inner + i];
            y[i] = sum;
        }
    }
    free(conv_out);
    free(dt);
    free(b_vals);
}

/* ---- TurboQuant compressed KV (src/turboquant/mod.rs) ---------------------------------- */

/* Lloyd-Max centroids for N(0,1) by bit width 1..4 (src/turboquant/mod.rs:27-40). */
static const float tq_c1[2] = {-0.7979f, 0.7979f};
static const float tq_c2[4] = {-1.4996f, -0.4950f, 0.4950f, 1.4996f};
static const float tq_c3[8] = {-2.1520f, -1.3440f, -0.7560f, -0.2451f,
                               0.2451f,  0.7560f,  1.3440f,  2.1520f};
static const float tq_c4[16] = {-2.7330f, -2.0690f, -1.6180f, -1.2560f, -0.9424f, -0.6568f,
                                -0.3880f, -0.1284f, 0.1284f,  0.3880f,  0.6568f,  0.9424f,
                                1.2560f,  1.6180f,  2.0690f,  2.7330f};
static const float* tq_centroids(size_t bits) {
    return bits == 1 ? tq_c1 : bits == 2 ? tq_c2 : bits == 3 ? tq_c3 : tq_c4;
}
float or_tq_centroid(size_t bits, size_t j) { return tq_centroids(bits)[j]; }

/* expected_distortion (:372-379) */
static float tq_distortion(size_t bits) {
    return bits == 2 ? 0.17f : bits == 3 ? 0.043f : bits == 4 ? 0.011f : 0.17f;
}

uint64_t or_splitmix64_next(uint64_t* state) {
    /* :725-731 */
    *state += 0x9E3779B97F4A7C15ULL;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

float or_splitmix64_gaussian(uint64_t* state) {
    /* :733-745: u1 = max(next_f64, 1e-10), Box-Muller cosine branch in f64, rounded to f32 */
    double u1 = (double)(or_splitmix64_next(state) >> 11) / (double)(1ULL << 53);
    double u2 = (double)(or_splitmix64_next(state) >> 11) / (double)(1ULL << 53);
    if (u1 < 1e-10) u1 = 1e-10;
    double r = sqrt(-2.0 * log(u1));
    double theta = 2.0 * 3.14159265358979323846 * u2;
    return (float)(r * cos(theta));
}

void or_tq_gaussian_matrix(float* m, size_t rows, size_t cols, uint64_t seed) {
    uint64_t st = seed;
    for (size_t i = 0; i < rows * cols; ++i) m[i] = or_splitmix64_gaussian(&st);
}

void or_tq_orthogonal(float* q, size_t dim, uint64_t seed) {
    /* :657-701: Gaussian A (row-major), then per column j: q_j = a_j minus its projections
     * (dot taken against the original column a_j) on q_0..q_{j-1}, then q_j /= |q_j|. */
    float* a = (float*)malloc(dim * dim * sizeof(float));
    or_tq_gaussian_matrix(a, dim, dim, seed);
    for (size_t j = 0; j < dim; ++j) {
        for (size_t i = 0; i < dim; ++i) q[i * dim + j] = a[i * dim + j];
        for (size_t k = 0; k < j; ++k) {
            float dot = 0.0f;
            for (size_t i = 0; i < dim; ++i) dot += q[i * dim + k] * a[i * dim + j];
            for (size_t i = 0; i < dim; ++i) q[i * dim + j] -= dot * q[i * dim + k];
        }
        float norm = 0.0f;
        for (size_t i = 0; i < dim; ++i) norm += q[i * dim + j] * q[i * dim + j];
        norm = sqrtf(norm);
        if (norm > 1e-10f)
            for (size_t i = 0; i < dim; ++i) q[i * dim + j] /= norm;
    }
    free(a);
}

size_t or_tq_compressed_bytes(size_t bits, size_t dim, size_t qjl_bits) {
    return (bits * dim + 7) / 8 + (qjl_bits + 7) / 8;
}

void or_tq_pack(uint8_t* out, const uint8_t* idx, size_t n, size_t bits, const uint8_t* signs,
                size_t n_signs) {
    /* :591-617 (pack_indices :572-588 is the n_signs == 0 case) */
    memset(out, 0, (n * bits + n_signs + 7) / 8);
    size_t pos = 0;
    for (size_t i = 0; i < n; ++i)
        for (size_t b = 0; b < bits; ++b, ++pos)
            if ((idx[i] >> b) & 1) out[pos / 8] |= (uint8_t)(1u << (pos % 8));
    for (size_t i = 0; i < n_signs; ++i, ++pos)
        if (signs[i]) out[pos / 8] |= (uint8_t)(1u << (pos % 8));
}

void or_tq_unpack(uint8_t* idx, uint8_t* signs, const uint8_t* packed, size_t n, size_t bits,
                  size_t n_signs) {
    /* :620-654 */
    size_t pos = 0;
    for (size_t i = 0; i < n; ++i) {
        idx[i] = 0;
        for (size_t b = 0; b < bits; ++b, ++pos)
            if ((packed[pos / 8] >> (pos % 8)) & 1) idx[i] |= (uint8_t)(1u << b);
    }
    for (size_t i = 0; i < n_signs; ++i, ++pos)
        if (signs) signs[i] = (packed[pos / 8] >> (pos % 8)) & 1;
}

void or_tq_quantize(uint8_t* packed, const float* x, const float* R, const float* G, size_t dim,
                    size_t bits, size_t qjl_bits) {
    /* :128-187 */
    const float* c = tq_centroids(bits);
    const size_t nc = (size_t)1 << bits;
    float* rot = (float*)malloc(dim * sizeof(float));
    uint8_t* idx = (uint8_t*)malloc(dim);
    const float scale = sqrtf((float)dim);
    for (size_t i = 0; i < dim; ++i) {
        float sum = 0.0f;
        for (size_t j = 0; j < dim; ++j) sum += R[i * dim + j] * x[j];
        rot[i] = sum;
    }
    for (size_t i = 0; i < dim; ++i) rot[i] *= scale;
    for (size_t i = 0; i < dim; ++i) {
        uint8_t best = 0;
        float best_d = 3.40282347e+38f;
        for (size_t j = 0; j < nc; ++j) {
            const float d = fabsf(rot[i] - c[j]);
            if (d < best_d) {
                best_d = d;
                best = (uint8_t)j;
            }
        }
        idx[i] = best;
    }
    if (qjl_bits == 0) {
        or_tq_pack(packed, idx, dim, bits, NULL, 0);
    } else {
        uint8_t* sg = (uint8_t*)malloc(qjl_bits);
        for (size_t i = 0; i < dim; ++i) rot[i] = rot[i] - c[idx[i]]; /* residual */
        for (size_t i = 0; i < qjl_bits; ++i) {
            float proj = 0.0f;
            for (size_t j = 0; j < dim; ++j) proj += G[i * dim + j] * rot[j];
            sg[i] = proj >= 0.0f;
        }
        or_tq_pack(packed, idx, dim, bits, sg, qjl_bits);
        free(sg);
    }
    free(idx);
    free(rot);
}

void or_tq_dequantize(float* out, const uint8_t* packed, const float* R, size_t dim, size_t bits) {
    /* :194-216 */
    const float* c = tq_centroids(bits);
    uint8_t* idx = (uint8_t*)malloc(dim);
    float* rec = (float*)malloc(dim * sizeof(float));
    or_tq_unpack(idx, NULL, packed, dim, bits, 0);
    const float inv_scale = 1.0f / sqrtf((float)dim);
    for (size_t i = 0; i < dim; ++i) rec[i] = c[idx[i]] * inv_scale;
    for (size_t i = 0; i < dim; ++i) {
        float sum = 0.0f;
        for (size_t j = 0; j < dim; ++j) sum += R[j * dim + i] * rec[j];
        out[i] = sum;
    }
    free(rec);
    free(idx);
}

float or_tq_dot(const float* q, const uint8_t* packed, const float* R, const float* G, size_t dim,
                size_t bits, size_t qjl_bits) {
    if (qjl_bits == 0) { /* :229-238 */
        float* kd = (float*)malloc(dim * sizeof(float));
        or_tq_dequantize(kd, packed, R, dim, bits);
        float dot = 0.0f;
        for (size_t i = 0; i < dim; ++i) dot += q[i] * kd[i];
        free(kd);
        return dot;
    }
    /* asymmetric_dot (:323-369) */
    const float* c = tq_centroids(bits);
    uint8_t* idx = (uint8_t*)malloc(dim);
    uint8_t* sg = (uint8_t*)malloc(qjl_bits);
    float* qr = (float*)malloc(dim * sizeof(float));
    or_tq_unpack(idx, sg, packed, dim, bits, qjl_bits);
    const float inv_scale = 1.0f / sqrtf((float)dim);
    for (size_t i = 0; i < dim; ++i) {
        float sum = 0.0f;
        for (size_t j = 0; j < dim; ++j) sum += R[i * dim + j] * q[j];
        qr[i] = sum;
    }
    float mse = 0.0f;
    for (size_t i = 0; i < dim; ++i) mse += qr[i] * c[idx[i]] * inv_scale;
    const float residual_norm = sqrtf(tq_distortion(bits) * inv_scale);
    float qjl = 0.0f;
    for (size_t i = 0; i < qjl_bits; ++i) {
        float proj = 0.0f;
        for (size_t j = 0; j < dim; ++j) proj += G[i * dim + j] * qr[j];
        qjl += proj * (sg[i] ? 1.0f : -1.0f);
    }
    const float qjl_scale = sqrtf(3.14159274f / (2.0f * (float)qjl_bits));
    const float corr = residual_norm * qjl_scale * qjl * inv_scale;
    free(qr);
    free(sg);
    free(idx);
    return mse + corr;
}

void or_tq_precompute_query(float* q_rot, float* qjl_proj, const float* q, const float* R,
                            const float* G, size_t dim, size_t qjl_bits) {
    /* :244-278 */
    const float scale = sqrtf((float)dim);
    const float inv_scale = 1.0f / scale;
    for (size_t i = 0; i < dim; ++i) {
        float sum = 0.0f;
        for (size_t j = 0; j < dim; ++j) sum += R[i * dim + j] * q[j];
        q_rot[i] = sum;
    }
    for (size_t i = 0; i < qjl_bits; ++i) {
        float proj = 0.0f;
        for (size_t j = 0; j < dim; ++j) proj += G[i * dim + j] * q_rot[j];
        qjl_proj[i] = proj * inv_scale;
    }
    for (size_t i = 0; i < dim; ++i) q_rot[i] *= inv_scale;
}

float or_tq_dot_precomputed(const float* q_rot, const float* qjl_proj, const uint8_t* packed,
                            size_t dim, size_t bits, size_t qjl_bits) {
    /* :281-320 */
    const float* c = tq_centroids(bits);
    uint8_t* idx = (uint8_t*)malloc(dim);
    uint8_t* sg = (uint8_t*)malloc(qjl_bits ? qjl_bits : 1);
    or_tq_unpack(idx, sg, packed, dim, bits, qjl_bits);
    float mse = 0.0f;
    for (size_t i = 0; i < dim; ++i) mse += q_rot[i] * c[idx[i]];
    float res = mse;
    if (qjl_bits > 0) {
        const float inv_scale = 1.0f / sqrtf((float)dim);
        const float residual_norm = sqrtf(tq_distortion(bits) * inv_scale);
        float qjl = 0.0f;
        for (size_t i = 0; i < qjl_bits; ++i) qjl += qjl_proj[i] * (sg[i] ? 1.0f : -1.0f);
        const float qjl_scale = sqrtf(3.14159274f / (2.0f * (float)qjl_bits));
        res = mse + residual_norm * qjl_scale * qjl;
    }
    free(sg);
    free(idx);
    return res;
}

void or_tq_cache_append_keys(uint8_t* packed, float* norms, const float* keys, const float* R,
                             const float* G, size_t n_kv, size_t dim) {
    /* :455-486 with TurboQuant::new(3, dim, dim, .) per head (:430-437) */
    const size_t nb = or_tq_compressed_bytes(3, dim, dim);
    float* xn = (float*)malloc(dim * sizeof(float));
    for (size_t h = 0; h < n_kv; ++h) {
        const float* x = keys + h * dim;
        float ss = 0.0f;
        for (size_t i = 0; i < dim; ++i) ss += x[i] * x[i];
        const float norm = sqrtf(ss);
        const float inv = norm > 1e-12f ? 1.0f / norm : 0.0f;
        for (size_t i = 0; i < dim; ++i) xn[i] = x[i] * inv;
        or_tq_quantize(packed + h * nb, xn, R + h * dim * dim, G + h * dim * dim, dim, 3, dim);
        norms[h] = norm;
    }
    free(xn);
}

/* IEEE binary16 bits -> float (exact). */
static float half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else { /* subnormal: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-08f;
            return (h >> 15) ? -f : f;
        }
    } else if (e == 31) {
        bits = s | 0x7F800000u | (m << 13);
    } else {
        bits = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

void or_tq_cache_attend(float* out, const float* q_head, const uint8_t* packed, const float* norms,
                        const uint16_t* values, const float* R, const float* G, size_t T,
                        size_t n_kv, size_t kv_h, size_t dim) {
    /* attention_scores (:489-516) with the precomputed query, ops::softmax (src/ops.rs:160-180),
     * weighted_value_sum (:519-536), which skips weights below 1e-7. */
    const size_t nb = or_tq_compressed_bytes(3, dim, dim);
    const float scale = 1.0f / sqrtf((float)dim);
    float* qr = (float*)malloc(dim * sizeof(float));
    float* qp = (float*)malloc(dim * sizeof(float));
    float* sc = (float*)malloc((T ? T : 1) * sizeof(float));
    or_tq_precompute_query(qr, qp, q_head, R, G, dim, dim);
    for (size_t t = 0; t < T; ++t) {
        const float kn = norms[t * n_kv + kv_h];
        sc[t] = kn * or_tq_dot_precomputed(qr, qp, packed + (t * n_kv + kv_h) * nb, dim, 3, dim) *
                scale;
    }
    or_softmax(sc, T);
    for (size_t d = 0; d < dim; ++d) out[d] = 0.0f;
    for (size_t t = 0; t < T; ++t) {
        const float w = sc[t];
        if (w < 1e-7f) continue;
        const uint16_t* v = values + (t * n_kv + kv_h) * dim;
        for (size_t d = 0; d < dim; ++d) out[d] += w * half_to_float(v[d]);
    }
    free(sc);
    free(qp);
    free(qr);
}

/*
 * oracle.h -- CPU restatement of PowerInfer_x64's attention + gated-DeltaNet path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the timed CPU baseline of bench.py.  Only tests/, the smoke() entry
 * and bench.py's cpu_baseline leg may load it; the product library never
 * links, loads or falls back to it.
 *
 * Every function restates one reference function (file:line relative to the
 * PowerInfer_x64 repository root) in plain C with the same loop order and f32
 * arithmetic: separate multiply and add (built with -ffp-contract=off, as Rust
 * never contracts a*b+c), the same reduction order (4-lane SSE accumulators
 * where the reference uses src/simd.rs, a left fold where it uses
 * Iterator::sum), and the same libm calls (Rust's f32::{exp,ln,powf,sin,cos}
 * lower to the glibc expf/logf/powf/sinf/cosf this file calls).
 *
 * Pins (tests/test_oracle_pins.py): the reference's own known-answer tests
 * (src/ops.rs:303-395, src/simd.rs:242-354, tests/smoke.rs:46-61,
 * src/bin/layer_trace.rs:180-196), closed forms, invariants and float64
 * brute force on tiny shapes.  Functions whose only pin is a property test are
 * noted below; none is "parity unpinned".
 */
#ifndef PI_ORACLE_H
#define PI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/simd.rs:14-53 + :189-197 -- 4 lane accumulators over i step 4,
 * horizontal sum (l0+l1)+(l2+l3), then scalar tail. */
float or_dot_product(const float* a, const float* b, size_t n);
/* src/simd.rs:115-135 -- same lane structure as the dot product. */
float or_sum_squares(const float* a, size_t n);
/* src/simd.rs:139-156 -- out = a * s. */
void or_scale(float* out, const float* a, float s, size_t n);

/* src/ops.rs:13-27 */
void or_rms_norm(float* out, const float* x, const float* w, size_t n, float eps);
/* src/ops.rs:35-67 -- adjacent-pair (2i, 2i+1) rotary on one q head and one k head. */
void or_apply_rope(float* q, float* k, size_t position, size_t head_dim, size_t rope_dim, float base);
/* src/ops.rs:78-122 -- writes n_rot/2 frequencies. */
void or_compute_imrope_freqs(float base, size_t n_rot, const int32_t sections[4], float* freqs);
/* src/ops.rs:130-157 -- NeoX pairing (i, i+n_freqs). */
void or_apply_rope_with_freqs(float* q, float* k, size_t position, size_t head_dim,
                              const float* freqs, size_t n_freqs);
/* src/ops.rs:160-180 */
void or_softmax(float* x, size_t n);
/* src/ops.rs:213-247 -- scalar dot, contiguous [seq_len][head_dim] caches. */
void or_attention_head(float* out, const float* q, const float* k_cache, const float* v_cache,
                       size_t seq_len, size_t head_dim);

/* src/model/mod.rs:1148-1190 -- the decode attention core for one query token.
 * q: [n_heads][q_head_dim] (already normed and rotated); caches are the
 * reference's token-major [total_seq][n_kv_heads][kv_head_dim|v_head_dim];
 * kv head of q head h is h % n_kv_heads; out: [n_heads][kv_head_dim]. */
void or_attn_decode(float* out, const float* q, size_t q_head_dim,
                    const float* key_cache, const float* value_cache, size_t total_seq,
                    size_t n_heads, size_t n_kv_heads, size_t kv_head_dim, size_t v_head_dim);

/* src/model/mod.rs:1192-1196 -- out[i] *= 1/(1+exp(-gate[i])), i < n. */
void or_apply_gate(float* out, const float* gate, size_t n);

/* src/model/mod.rs:1035-1138 for n_tokens consecutive tokens: the optional
 * per-head Q/K RMSNorm and the RoPE driver (Q heads at every position, K head
 * h rotated only when h < n_kv_heads), in place, without appending or
 * attending.  Token i sits at position pos0 + i.  q may be NULL (K only). */
void or_attn_prepare(float* q, float* k, size_t n_tokens, size_t n_heads, size_t n_kv_heads,
                     size_t q_head_dim, size_t kv_head_dim, const float* q_norm_w,
                     const float* k_norm_w, float eps, size_t rope_dim, float rope_base,
                     const float* freqs, size_t n_freqs, size_t pos0);

/* src/model/mod.rs:1035-1196 for n_tokens consecutive tokens of one sequence:
 * per token (src/model/mod.rs:668 loop) optional per-head Q/K RMSNorm
 * (:1035-1070), RoPE driver (:1072-1138; NORM mode when freqs == NULL,
 * sectioned/NeoX mode otherwise), append to the caches (:1140-1146; the caches
 * must have room for prev_seq_len + n_tokens tokens), attention over
 * prev_seq_len + pos + 1 keys (:1148-1190), optional sigmoid gate (:1192-1196).
 * q/k are modified in place (normed + rotated), as in the reference. */
void or_attn_layer_tokens(float* out, float* q, const float* gate, float* k, const float* v,
                          size_t n_tokens, size_t n_heads, size_t n_kv_heads,
                          size_t q_head_dim, size_t kv_head_dim, size_t v_head_dim,
                          const float* q_norm_w, const float* k_norm_w, float eps,
                          size_t rope_dim, float rope_base, const float* freqs, size_t n_freqs,
                          float* key_cache, float* value_cache, size_t prev_seq_len);

/* src/model/mod.rs:796-839 -- beta = sigmoid(beta_raw); g = ssm_a * softplus(a_raw + dt_bias),
 * softplus(x) = x for x > 10.  All arrays are [n_v_heads]. */
void or_gdn_gates(float* beta, float* g, const float* beta_raw, const float* a_raw,
                  const float* ssm_a, const float* dt_bias, size_t n_v_heads);

/* src/model/mod.rs:841-916 -- one token of the gated delta rule.
 * q_raw/k_raw: [n_k_heads][k_hd] (pre-norm), v: [n_v_heads][v_hd], beta/g: [n_v_heads],
 * state: [n_v_heads][k_hd][v_hd] in/out, out: [n_v_heads][v_hd] (pre RMSNormGated). */
void or_gdn_step(float* out, float* state, const float* q_raw, const float* k_raw,
                 const float* v, const float* beta, const float* g,
                 size_t n_k_heads, size_t n_v_heads, size_t k_hd, size_t v_hd);

/* n_tokens consecutive calls of or_gdn_step (the reference's per-token prefill,
 * src/model/mod.rs:668 loop).  Arrays are token-major. */
void or_gdn_tokens(float* out, float* state, const float* q_raw, const float* k_raw,
                   const float* v, const float* beta, const float* g, size_t n_tokens,
                   size_t n_k_heads, size_t n_v_heads, size_t k_hd, size_t v_hd);

/* src/model/mod.rs:918-932 -- per v head: o * (1/sqrt(mean(o^2)+eps)) * w * silu(z). */
void or_rmsnorm_gated(float* o, const float* z, const float* w, size_t n_v_heads, size_t v_hd,
                      float eps);

/* src/ssm/mod.rs:40-157 -- ssm_forward, one token of the Mamba-2-style scan.
 * x, dt_bias: [d_inner]; ssm_a, state: [d_state * d_inner] (state in/out);
 * alpha: [d_inner * d_inner]; conv1d / beta / out_w at the given lengths select
 * the reference's branches.  y: [d_inner]. */
void or_ssm_forward(float* y, const float* x, const float* conv1d, size_t conv1d_len,
                    const float* ssm_a, const float* dt_bias, const float* alpha,
                    const float* beta, size_t beta_len, const float* out_w, size_t out_len,
                    float* state, size_t d_inner, size_t d_state, size_t d_conv);

/* src/model/mod.rs:750-776 -- depthwise causal conv1d + SiLU for one token.
 * hist: [d_conv-1][conv_dim] previous inputs, oldest first (zeros at start);
 * x: [conv_dim] new input, overwritten with the activation; hist is shifted. */
void or_conv1d_silu(float* x, float* hist, const float* w, size_t conv_dim, size_t d_conv);

/* ---- TurboQuant compressed KV (src/turboquant/mod.rs) ---------------------------------- */
/* SplitMix64 step and its Box-Muller Gaussian (:719-746). */
uint64_t or_splitmix64_next(uint64_t* state);
float or_splitmix64_gaussian(uint64_t* state);
/* Random orthogonal [dim x dim] by Gram-Schmidt of a seeded Gaussian matrix (:657-701). */
void or_tq_orthogonal(float* q, size_t dim, uint64_t seed);
/* Seeded Gaussian [rows x cols] (:704-711). */
void or_tq_gaussian_matrix(float* m, size_t rows, size_t cols, uint64_t seed);
/* Lloyd-Max centroid j of the bits-wide codebook (:27-40). */
float or_tq_centroid(size_t bits, size_t j);
/* Packed bytes of one vector (:111-118). */
size_t or_tq_compressed_bytes(size_t bits, size_t dim, size_t qjl_bits);
/* Bit packing, LSB first: indices then sign bits (:572-654). */
void or_tq_pack(uint8_t* out, const uint8_t* idx, size_t n, size_t bits, const uint8_t* signs,
                size_t n_signs);
void or_tq_unpack(uint8_t* idx, uint8_t* signs, const uint8_t* packed, size_t n, size_t bits,
                  size_t n_signs);
/* quantize_vector (:128-187): rotation R [dim][dim], QJL matrix G [qjl_bits][dim] (NULL
 * when qjl_bits == 0); writes or_tq_compressed_bytes() bytes. */
void or_tq_quantize(uint8_t* packed, const float* x, const float* R, const float* G, size_t dim,
                    size_t bits, size_t qjl_bits);
/* dequantize_vector (:194-216). */
void or_tq_dequantize(float* out, const uint8_t* packed, const float* R, size_t dim, size_t bits);
/* dot (:225-241) -- MSE-only dequantize-and-dot, or the asymmetric QJL estimator (:323-369). */
float or_tq_dot(const float* q, const uint8_t* packed, const float* R, const float* G, size_t dim,
                size_t bits, size_t qjl_bits);
/* precompute_query (:244-278) and dot_precomputed (:281-320). */
void or_tq_precompute_query(float* q_rot, float* qjl_proj, const float* q, const float* R,
                            const float* G, size_t dim, size_t qjl_bits);
float or_tq_dot_precomputed(const float* q_rot, const float* qjl_proj, const uint8_t* packed,
                            size_t dim, size_t bits, size_t qjl_bits);
/* CompressedKVCache::append for one token (:455-486), keys only: per KV head the L2 norm and
 * the 3-bit + QJL packed key.  R, G: [n_kv][dim][dim].  packed: [n_kv][bytes]. */
void or_tq_cache_append_keys(uint8_t* packed, float* norms, const float* keys, const float* R,
                             const float* G, size_t n_kv, size_t dim);
/* attention_scores (:489-516) + ops::softmax + weighted_value_sum (:519-536) for one query
 * head over T tokens of KV head kv_h.  packed [T][n_kv][bytes], norms [T][n_kv], values
 * [T][n_kv][dim] as f16 bits, R, G of that KV head. */
void or_tq_cache_attend(float* out, const float* q_head, const uint8_t* packed, const float* norms,
                        const uint16_t* values, const float* R, const float* G, size_t T,
                        size_t n_kv, size_t kv_h, size_t dim);

#ifdef __cplusplus
}
#endif
#endif

/*
 * pi_attn.h -- C ABI of the MI355X (gfx950) attention + gated-DeltaNet path.
 *
 * Drop-in boundary for PowerInfer_x64's CPU attention / SSM path.  Each entry
 * point names the reference code it replaces (paths relative to the
 * PowerInfer_x64 repository root).  Conventions:
 *   - every function returns pi_status (0 = PI_OK); on failure the text is in
 *     pi_last_error(handle) -- the analogue of the reference's
 *     Option<Result<(), String>> offload seam (src/cuda/mod.rs:527-537,
 *     src/model/mod.rs:612-626): PI_OK = Some(Ok), an error = Some(Err(text)),
 *     and a caller without a handle takes the CPU path (None);
 *   - status classes follow BackendError (src/runtime/mod.rs:6-18);
 *   - pointers named d_* are device pointers (HBM), h_* are host pointers;
 *   - `stream` is a hipStream_t; NULL is HIP's default (null) stream, as for
 *     every HIP API, not the handle's stream.  The null stream is the legacy
 *     one: work on it waits for, and holds back, work on every blocking stream
 *     of the device, so a caller that wants its calls isolated from other
 *     streams passes a non-blocking stream of its own.  Calls are
 *     asynchronous on that stream except the h_* "sync" wrappers, which run on
 *     the handle's own (non-blocking) stream and synchronise before
 *     returning, like GpuDevice::matvec (src/cuda/mod.rs:244-330);
 *   - one handle per host thread; the library takes no locks.  A handle's
 *     workspaces (decode partials, GDN prefill buffers) may serve calls on
 *     different streams: a call on another stream than the previous
 *     workspace user waits (on the device) for that use first;
 *   - all arithmetic is fp32 except where a dtype argument says otherwise;
 *   - page_tokens is 16; head_dim is 64, 128 or 256.
 */
#ifndef PI_ATTN_H
#define PI_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PI_ATTN_ABI_VERSION 1

/* src/runtime/mod.rs:6-18 (BackendError) */
typedef enum pi_status {
    PI_OK = 0,
    PI_ERR_INVALID_ARG = 1,    /* bad pointer / shape (debug_assert_eq! in src/ops.rs:14-15) */
    PI_ERR_OUT_OF_MEMORY = 2,  /* BackendError::OutOfMemory */
    PI_ERR_INVALID_KERNEL = 3, /* BackendError::InvalidKernel: no gfx950 code object / launch failed */
    PI_ERR_DEVICE = 4,         /* BackendError::CudaError(String): HIP runtime error */
    PI_ERR_UNSUPPORTED = 5     /* BackendError::Unsupported: shape/dtype outside the kernels */
} pi_status;

typedef enum pi_dtype { PI_F32 = 0, PI_F16 = 1, PI_BF16 = 2 } pi_dtype;

/* Q head h reads KV head h % n_kv_heads (src/model/mod.rs:1155, the reference's
 * mapping) or h / (n_q_heads / n_kv_heads) (the usual grouped layout). */
typedef enum pi_gqa_mode { PI_GQA_MODULO = 0, PI_GQA_GROUPED = 1 } pi_gqa_mode;

typedef struct pi_handle_s* pi_handle;
typedef struct pi_kv_pool_s* pi_kv_pool;

/* ---- handle ---------------------------------------------------------------
 * Replaces GpuDevice::new / GpuResources::init (src/cuda/mod.rs:196-242,
 * :387-460): binds a device, creates the handle's stream and lazily-grown
 * workspace (the reference's RefCell scratch, src/cuda/mod.rs:152,257-278). */
int pi_create(int device, pi_handle* out);
/* Drop ordering of src/cuda/mod.rs:166-178,540-573: frees with the device current. */
void pi_destroy(pi_handle h);
/* Text of the last error on this handle (or of the last pi_create failure when h is NULL). */
const char* pi_last_error(pi_handle h);
/* stream.synchronize() (src/cuda/mod.rs:312-314). */
int pi_sync(pi_handle h, void* stream);
int pi_abi_version(void);

/* ---- paged KV cache --------------------------------------------------------
 * Replaces LayerCache (src/model/mod.rs:73-106): instead of a growing f32
 * Vec [T][n_kv][D], a pool of fixed 16-token pages in HBM, one K and one V
 * block of 16 x head_dim per (page, kv head).  Sequences own pages through a
 * caller-provided int32 page table [n_seq][max_pages]. */
int pi_kv_pool_create(pi_handle h, int32_t n_pages, int32_t page_tokens, int32_t n_kv_heads,
                      int32_t head_dim, int32_t dtype, pi_kv_pool* out);
void pi_kv_pool_destroy(pi_kv_pool pool);
/* Total bytes of the K and V blocks (for capacity planning on 288 GB). */
size_t pi_kv_pool_bytes(pi_kv_pool pool);

/* Append (src/model/mod.rs:1140-1146, extend_from_slice): sequence s writes
 * n_tok tokens at positions d_start_pos[s] .. +n_tok-1.  d_k/d_v:
 * [n_seq][n_tok][n_kv_heads][head_dim] in src_dtype (converted, RNE, to the
 * pool dtype). */
int pi_kv_append(pi_handle h, pi_kv_pool pool, const void* d_k, const void* d_v, int32_t src_dtype,
                 const int32_t* d_page_table, int32_t max_pages, const int32_t* d_start_pos,
                 int32_t n_seq, int32_t n_tok, void* stream);
/* Read tokens [start, start+n_tok) of sequence `seq` back as f32 [n_tok][n_kv][D]
 * (the reference cache layout; used for dumps and parity checks). */
int pi_kv_read(pi_handle h, pi_kv_pool pool, const int32_t* d_page_table, int32_t max_pages,
               int32_t seq, int32_t start, int32_t n_tok, float* d_k_out, float* d_v_out,
               void* stream);
/* reset() (src/model/mod.rs:1847-1873) needs no device work: a sequence is
 * reset by giving it length 0; pages are owned by the caller's table. */

/* ---- decode prologue -------------------------------------------------------
 * Per-head RMSNorm in place (ops::rms_norm, src/ops.rs:13-27, as called at
 * src/model/mod.rs:1035-1070): rows of `dim` values (any dim) at stride
 * `row_stride`. */
int pi_head_rmsnorm(pi_handle h, float* d_x, const float* d_w, int32_t n_rows, int32_t dim,
                    int32_t row_stride, float eps, void* stream);
/* RoPE in place on q [n_tok][n_q_heads][head_dim] and k [n_tok][n_kv_heads][head_dim]
 * at positions d_pos[n_tok].  h_sections == NULL: ops::apply_rope (src/ops.rs:35-67,
 * adjacent pairs, rope_dim dims).  Otherwise ops::compute_imrope_freqs +
 * apply_rope_with_freqs (src/ops.rs:78-157, NeoX pairs over rope_dim dims).
 * Frequencies are built on the host with the reference's f32 formula.  d_k may
 * be NULL (rotate q only, the src/model/mod.rs:1113-1134 dummy-k branch). */
int pi_rope(pi_handle h, float* d_q, float* d_k, const int32_t* d_pos, int32_t n_tok,
            int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t rope_dim,
            float base, const int32_t* h_sections, void* stream);

/* The whole prologue of a full-attention layer step in one launch
 * (src/model/mod.rs:1035-1146): for token t of sequence s at position
 * d_start_pos[s] + t, per-head RMSNorm of q and k (when d_q_norm_w /
 * d_k_norm_w are non-NULL, [head_dim] each), RoPE (as pi_rope: NORM pairs, or
 * IMRoPE NeoX pairs when h_sections != NULL), q and k rewritten in place, and
 * k and v appended to the pool (append-then-attend).  d_q
 * [n_seq][n_tok][n_q_heads][D], d_k/d_v [n_seq][n_tok][n_kv_heads][D] f32,
 * D = the pool's head_dim. */
int pi_attn_prologue(pi_handle h, float* d_q, float* d_k, const float* d_v,
                     const float* d_q_norm_w, const float* d_k_norm_w, float eps,
                     int32_t rope_dim, float rope_base, const int32_t* h_sections,
                     pi_kv_pool pool, const int32_t* d_page_table, int32_t max_pages,
                     const int32_t* d_start_pos, int32_t n_seq, int32_t n_tok,
                     int32_t n_q_heads, void* stream);

/* ---- attention ---------------------------------------------------------------
 * Decode: one query token per sequence against its paged cache
 * (src/model/mod.rs:1148-1190; append-then-attend: the caller appends the
 * token's K/V first, so d_ctx_len counts it).  d_q [batch][n_q_heads][D] f32
 * (normed, rotated); out [batch][n_q_heads][D] f32.  scale multiplies q.k
 * (1/sqrt(D) in the reference).  d_gate (nullable) [batch][n_q_heads][D]:
 * out *= sigmoid(gate) (src/model/mod.rs:1192-1196).  Split-K flash decoding,
 * one launch.  Any head counts with the modulo map (a KV head's query heads
 * ride in the MFMA columns, up to 16 per pass); the grouped map needs n_q_heads
 * a multiple of n_kv_heads.  d_q, d_out and d_gate are 16-byte aligned (the
 * kernels move them in 16-byte groups).  Device tables are read, not
 * trusted: d_ctx_len[b] is clamped to [0, 16 * max_pages], and a page id
 * outside [0, n_pages) holds no tokens (its keys are masked; a sequence with
 * no unmasked key gets zeros, as an empty context does). */
int pi_attn_decode(pi_handle h, const float* d_q, pi_kv_pool pool, const int32_t* d_page_table,
                   int32_t max_pages, const int32_t* d_ctx_len, int32_t batch,
                   int32_t n_q_heads, int32_t gqa_mode, float scale, const float* d_gate,
                   float* d_out, void* stream);

/* No counterpart in the reference.  pi_attn_decode for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): same arguments, kernels and results, but
 * the split-run partials live in a fixed 16 MiB scratch array per GPU instead
 * of the handle's grow-on-demand workspace, so the call allocates nothing.
 * The scratch needs (batch * n_kv_heads + CUs * resident workgroups) *
 * (n_q_heads / n_kv_heads) * (head_dim + 2) floats (at most 1023 workgroups);
 * a launch needing more fails with PI_ERR_UNSUPPORTED and launches nothing.
 * Every no-alloc call on one GPU, from any handle or stream, shares that
 * array: calls that overlap on one GPU race and must be ordered by the
 * caller. */
int pi_attn_decode_noalloc(pi_handle h, const float* d_q, pi_kv_pool pool,
                           const int32_t* d_page_table, int32_t max_pages,
                           const int32_t* d_ctx_len, int32_t batch, int32_t n_q_heads,
                           int32_t gqa_mode, float scale, const float* d_gate, float* d_out,
                           void* stream);

/* Causal prefill of a whole prompt: row i attends keys 0..i, which is what the
 * reference's per-token loop computes (src/model/mod.rs:668,1140-1190).
 * d_q [batch][seq_len][n_q_heads][D], d_k/d_v [batch][seq_len][n_kv_heads][D]
 * in dtype (PI_BF16 or PI_F16); d_out [batch][seq_len][n_q_heads][D] f32.
 * MFMA flash attention with fp32 softmax/accumulation.  D = head_dim is 1..256:
 * 64, 128 and 256 run directly; another width runs zero-padded to the next of
 * them (q, k, v copied into padded rows of a handle workspace, the output cut
 * back; zero dims change no q.k), at that width's cost.  Head counts as
 * pi_attn_decode. */
int pi_attn_prefill(pi_handle h, const void* d_q, const void* d_k, const void* d_v, int32_t dtype,
                    int32_t batch, int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads,
                    int32_t head_dim, int32_t causal, int32_t gqa_mode, float scale, float* d_out,
                    void* stream);

/* Causal prefill of a chunk that continues a sequence, over its paged cache
 * (src/model/mod.rs:668 token loop over :1140-1190 with prev_seq_len =
 * start_pos): query row i sits at position start_pos + i and attends keys
 * 0 .. start_pos + i, read from the f16 pool through the sequence's page-table
 * row d_page_table[max_pages] (the chunk's own K/V appended first, as the
 * reference appends before it attends).  d_q [n_tok][n_q_heads][D] in the
 * pool's dtype (normed, rotated), d_out [n_tok][n_q_heads][D] f32.  f16 pool
 * (D = 64, 128 or 256): the flash prefill reads K/V straight from the pages
 * (no copy of the history; the handle's workspace holds only the key splits'
 * partials of the chunk's rows).  f32 pool (D = 64, 128 or 256): a kernel
 * reads the pages directly and keeps f32 accuracy (bf16 hi + lo operand splits
 * on the MFMA).  A page id outside [0, n_pages) holds no tokens: its keys are
 * left out of the softmax, as in pi_attn_decode. */
int pi_attn_prefill_paged(pi_handle h, const void* d_q, pi_kv_pool pool,
                          const int32_t* d_page_table, int32_t max_pages, int32_t start_pos,
                          int32_t n_tok, int32_t n_q_heads, int32_t gqa_mode, float scale,
                          float* d_out, void* stream);

/* ---- gated DeltaNet ----------------------------------------------------------
 * Gates (src/model/mod.rs:796-839): beta = sigmoid(beta_raw),
 * g = ssm_a * softplus(a_raw + dt_bias) (identity above 10).
 * beta_raw/a_raw/beta/g: [n_tok][n_v_heads]; ssm_a/dt_bias: [n_v_heads]. */
int pi_gdn_gates(pi_handle h, const float* d_beta_raw, const float* d_a_raw, const float* d_ssm_a,
                 const float* d_dt_bias, float* d_beta, float* d_g, int32_t n_tok,
                 int32_t n_v_heads, void* stream);
/* Depthwise causal conv1d + SiLU over the QKV channels (src/model/mod.rs:750-776)
 * for n_tok tokens of n_seq sequences.  d_x, d_out [n_seq][n_tok][conv_dim]
 * (d_out must not alias d_x); d_conv_state [n_seq][d_conv-1][conv_dim] in/out
 * holds the previous d_conv-1 raw inputs, oldest first (the reference's
 * ssm_conv_states ring, :125-127; zero-initialised, as its lazy init at
 * :752-756); d_w [conv_dim][d_conv] (GGML [ne0=d_conv, ne1=conv_dim]).
 * out[t][i] = silu(sum_k w[i][k] * window[k][i]). */
int pi_gdn_conv1d(pi_handle h, const float* d_x, float* d_conv_state, const float* d_w,
                  float* d_out, int32_t n_seq, int32_t n_tok, int32_t conv_dim, int32_t d_conv,
                  void* stream);
/* RMSNormGated in place (src/model/mod.rs:918-932): for each row and V head,
 * o = o * (1/sqrt(mean(o^2) + eps)) * w * silu(z).  d_o, d_z
 * [n_rows][n_v_heads][v_hd], d_w [v_hd]. */
int pi_gdn_rmsnorm_gated(pi_handle h, float* d_o, const float* d_z, const float* d_w,
                         int32_t n_rows, int32_t n_v_heads, int32_t v_hd, float eps,
                         void* stream);
/* One recurrent step per sequence (src/model/mod.rs:841-916): q/k raw
 * [batch][n_k_heads][k_hd], v [batch][n_v_heads][v_hd], beta/g [batch][n_v_heads],
 * state [batch][n_v_heads][k_hd][v_hd] f32 in/out (ssm::create_ssm_state,
 * src/ssm/mod.rs:164-166: zero-initialised by the caller), out
 * [batch][n_v_heads][v_hd] (before RMSNormGated).  Any k_hd <= 1024 and v_hd, any head
 * counts (V head vh reads K head vh % n_k_heads); k_hd = v_hd = 128 runs the tuned kernel,
 * other widths a per-token kernel (one wavefront per 8 state columns, 2 above k_hd 256). */
int pi_gdn_decode(pi_handle h, const float* d_q, const float* d_k, const float* d_v,
                  const float* d_beta, const float* d_g, float* d_state, float* d_out,
                  int32_t batch, int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd,
                  int32_t v_hd, void* stream);
/* n_tok tokens of one sequence, equal to n_tok consecutive pi_gdn_decode steps
 * (the reference's per-token prefill).  chunk 64: the chunked (WY) form when
 * k_hd = v_hd = 128; chunk 1, or other widths: token by token on the device.
 * Other chunk values are PI_ERR_UNSUPPORTED.  Layouts as pi_gdn_decode with
 * batch replaced by n_tok; state in/out. */
int pi_gdn_prefill(pi_handle h, const float* d_q, const float* d_k, const float* d_v,
                   const float* d_beta, const float* d_g, float* d_state, float* d_out,
                   int32_t n_tok, int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd,
                   int32_t v_hd, int32_t chunk, void* stream);

/* ---- host-slice drop-ins (synchronous) ---------------------------------------
 * ops::attention_head (src/ops.rs:213-247) with host slices: copies in,
 * runs the decode kernel, copies out.  k/v caches [seq_len][head_dim],
 * head_dim 1..128 (rows are zero-padded to the kernel's 64 or 128; the scale
 * stays 1/sqrt(head_dim)). */
int pi_ops_attention_head(pi_handle h, float* h_out, const float* h_q, const float* h_k_cache,
                          const float* h_v_cache, size_t seq_len, size_t head_dim);
/* ops::rms_norm (src/ops.rs:13-27): out = x * (1/sqrt(sum(x^2)/n + eps)) * w, n values. */
int pi_ops_rms_norm(pi_handle h, float* h_out, const float* h_x, const float* h_w, size_t n,
                    float eps);
/* ops::softmax (src/ops.rs:160-180), in place; n == 0 is a no-op. */
int pi_ops_softmax(pi_handle h, float* h_x, size_t n);
/* ops::apply_rope (src/ops.rs:35-67): one q head and one k head in place,
 * adjacent pairs (2i, 2i+1) for i < rope_dim/2 with 2i+1 < head_dim. */
int pi_ops_apply_rope(pi_handle h, float* h_q, float* h_k, size_t position, size_t head_dim,
                      size_t rope_dim, float base_freq);
/* ops::apply_rope_with_freqs (src/ops.rs:130-157): NeoX pairs (i, i+n_freqs). */
int pi_ops_apply_rope_with_freqs(pi_handle h, float* h_q, float* h_k, size_t position,
                                 size_t head_dim, const float* h_freqs, size_t n_freqs);
/* ops::compute_imrope_freqs (src/ops.rs:78-122), host only: writes n_rot/2
 * values theta_scale^k by repeated f32 multiplication.  `sections` is the
 * reference's argument; for text (all position tracks equal) it does not
 * change the values.  Errors are reported through pi_last_error(NULL). */
int pi_compute_imrope_freqs(float base, size_t n_rot, const int32_t* sections, float* out);
/* One gated-delta step on host slices (src/model/mod.rs:841-916 for one
 * token): q/k raw [n_k_heads][k_hd], v [n_v_heads][v_hd], beta/g [n_v_heads],
 * state [n_v_heads][k_hd][v_hd] in/out (ssm::create_ssm_state layout,
 * src/ssm/mod.rs:164-166), out [n_v_heads][v_hd]. */
int pi_ssm_gated_delta_step(pi_handle h, float* h_out, float* h_state, const float* h_q,
                            const float* h_k, const float* h_v, const float* h_beta,
                            const float* h_g, int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd,
                            int32_t v_hd);
/* ssm::ssm_forward (src/ssm/mod.rs:40-157): one token of the Mamba-2-style
 * selective scan on host slices, computed on the device.  x, dt_bias [d_inner];
 * ssm_a, state [d_state * d_inner] (state in/out); alpha [d_inner * d_inner];
 * conv1d, beta and out_w are taken at the lengths passed, and as in the
 * reference the conv taps apply only when conv1d_len = d_inner * d_conv, the
 * input-dependent B only when beta_len = d_state * d_inner, the output
 * projection only when out_len = d_inner * d_inner.  y [d_inner]. */
int pi_ssm_forward(pi_handle h, float* h_y, const float* h_x, const float* h_conv1d,
                   size_t conv1d_len, const float* h_ssm_a, const float* h_dt_bias,
                   const float* h_alpha, const float* h_beta, size_t beta_len,
                   const float* h_out_w, size_t out_len, float* h_state, size_t d_inner,
                   size_t d_state, size_t d_conv);

/* ---- Attention layer cache (the seam in InferenceContext::forward) -------------------
 * LayerCache (src/model/mod.rs:73-106) of one attention layer for one sequence, held on the
 * device: a paged pool of max_tokens tokens, the per-head Q/K RMSNorm weights (NULL when the
 * layer has none, src/model/mod.rs:1035-1070), the RoPE mode (NORM when h_sections is NULL,
 * else the sectioned NeoX rotation, :1072-1138) and the KV dtype (PI_F32 or PI_F16).
 * head_dim is 1..256: a width other than 64, 128 or 256 runs zero-padded to the next of them
 * (the pool's rows and the step's kernels at that width; zero dims change no q.k, the output
 * is cut back to head_dim, and the Q/K RMSNorm, RoPE and the 1/sqrt(head_dim) scale use
 * head_dim itself). */
typedef struct pi_attn_layer_s* pi_attn_layer;
int pi_attn_layer_create(pi_handle h, int32_t max_tokens, int32_t n_heads, int32_t n_kv_heads,
                         int32_t head_dim, int32_t kv_dtype, const float* h_q_norm_w,
                         const float* h_k_norm_w, float eps, int32_t rope_dim, float rope_base,
                         const int32_t* h_sections, int32_t gqa_mode, pi_attn_layer* out);
/* The same layer with the reference's separate head widths (src/model/mod.rs:976-982,
 * 1043-1190): query heads of q_head_dim >= head_dim values of which attention, the Q norm and
 * RoPE use the first head_dim (the rest pass through untouched); key heads of head_dim
 * (1..256); value heads of v_head_dim, of which the first min(head_dim,
 * v_head_dim) reach the output.  forward then takes q and gate [n][n_heads][q_head_dim], k
 * [n][n_kv_heads][head_dim], v [n][n_kv_heads][v_head_dim] and writes out
 * [n][n_heads][head_dim] (dims at or past v_head_dim zero); the gate multiplies the flat
 * output index i by sigmoid of the gate's flat index i, as :1192-1196 does.  q_norm_w and
 * k_norm_w hold head_dim values. */
int pi_attn_layer_create_dims(pi_handle h, int32_t max_tokens, int32_t n_heads,
                              int32_t n_kv_heads, int32_t q_head_dim, int32_t head_dim,
                              int32_t v_head_dim, int32_t kv_dtype, const float* h_q_norm_w,
                              const float* h_k_norm_w, float eps, int32_t rope_dim,
                              float rope_base, const int32_t* h_sections, int32_t gqa_mode,
                              pi_attn_layer* out);
void pi_attn_layer_destroy(pi_attn_layer layer);
/* src/model/mod.rs:1035-1196 for n_tokens consecutive tokens of the sequence (the :668 token
 * loop as one call): norm, RoPE at positions seq_len .. seq_len + n_tokens - 1, append, then
 * for every token attention over all cached keys up to and including its own, and the sigmoid
 * gate when h_gate is not NULL.  Host slices: q [n_tokens][n_heads][head_dim] and k
 * [n_tokens][n_kv_heads][head_dim] are normalised and rotated in place, as in the reference;
 * v like k; gate and out like q.  A full cache fails with PI_ERR_OUT_OF_MEMORY and changes
 * nothing.  Synchronous. */
int pi_attn_layer_forward(pi_handle h, pi_attn_layer layer, float* h_q, float* h_k,
                          const float* h_v, const float* h_gate, int32_t n_tokens, float* h_out);
/* pi_attn_layer_forward with device pointers (same layouts), enqueued on `stream` without
 * host copies or waits: the layer's sequence length advances when the call returns.  A
 * prompt or a continued chunk (more than one token) runs the flash prefill over the layer's
 * pages, as pi_attn_prefill_paged (f16 cache: straight from the pages at head_dim 64 / 128;
 * f32 cache: the f32 prefill); a single token runs the decode.  Calls on one layer must be
 * ordered on one stream. */
int pi_attn_layer_forward_dev(pi_handle h, pi_attn_layer layer, float* d_q, float* d_k,
                              const float* d_v, const float* d_gate, int32_t n_tokens,
                              float* d_out, void* stream);
/* LayerCache::reset (src/model/mod.rs:1854-1856): the sequence restarts at position 0. */
void pi_attn_layer_reset(pi_attn_layer layer);
int32_t pi_attn_layer_seq_len(pi_attn_layer layer);

/* ---- Gated-DeltaNet layer state (the seam in InferenceContext::forward) ----------------
 * One GDN layer of one sequence on the device: the rolling conv state ssm_conv_states[layer]
 * (src/model/mod.rs:125-127) and the recurrent state ssm_states[layer] (:122-124), both zero,
 * with the layer's conv1d weights [conv_dim][d_conv] (GGML layout, :765-769), ssm_a and
 * dt_bias [n_v_heads], and the RMSNormGated weight [v_hd]; conv_dim = 2 n_k_heads k_hd +
 * n_v_heads v_hd. */
typedef struct pi_gdn_layer_s* pi_gdn_layer;
int pi_gdn_layer_create(pi_handle h, int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd,
                        int32_t v_hd, int32_t d_conv, const float* h_conv_w, const float* h_ssm_a,
                        const float* h_dt_bias, const float* h_norm_w, float eps,
                        pi_gdn_layer* out);
void pi_gdn_layer_destroy(pi_gdn_layer layer);
/* src/model/mod.rs:750-932 for n_tokens consecutive tokens: conv1d + SiLU over the projected
 * qkv rows [n_tokens][conv_dim], split into q, k, v, beta / g from beta_raw, a_raw
 * [n_tokens][n_v_heads], the gated delta rule (chunked for n_tokens > 1), and
 * RMSNormGated x SiLU(z) with z [n_tokens][n_v_heads][v_hd]; out like z.  Synchronous. */
int pi_gdn_layer_forward(pi_handle h, pi_gdn_layer layer, const float* h_qkv, const float* h_z,
                         const float* h_beta_raw, const float* h_a_raw, int32_t n_tokens,
                         float* h_out);
/* pi_gdn_layer_forward with device pointers (same layouts), enqueued on `stream` without
 * host copies or waits.  Calls on one layer must be ordered on one stream.  With k_hd = v_hd
 * = 128 and d_conv 4, a one-token call is one kernel launch (16-byte aligned d_z and d_out;
 * otherwise the general path runs). */
int pi_gdn_layer_forward_dev(pi_handle h, pi_gdn_layer layer, const float* d_qkv,
                             const float* d_z, const float* d_beta_raw, const float* d_a_raw,
                             int32_t n_tokens, float* d_out, void* stream);
/* The GDN part of InferenceContext::reset (src/model/mod.rs:1867-1869): both states to zero.
 * It first waits for all work queued on the device (so forward_dev steps still pending on any
 * stream, a caller's non-blocking stream included, finish before the states are cleared),
 * then zeroes the conv state (both buffers of the one-launch step) and the recurrent state,
 * and returns when they are zero.  Synchronous. */
int pi_gdn_layer_reset(pi_handle h, pi_gdn_layer layer);

/* ---- TurboQuant compressed KV (src/turboquant/mod.rs:408-566) -------------------------
 * CompressedKVCache with head_dim D = 1..256: per KV head h a TurboQuant(3 bits, D, D QJL
 * bits, seed 0xCAFEBABE + h) key quantizer (:430-437) and f16 values.  Keys are stored as
 * ceil(4D/8)-byte records (3-bit Lloyd-Max codes of the rotated unit key, then the D QJL sign
 * bits, LSB first, byte-identical to quantize_vector / pack_compressed, :128-187,591-617)
 * plus their f32 L2 norm, in pages of 16 tokens addressed by the caller's page table, like
 * pi_kv_pool. */
typedef struct pi_tq_pool_s* pi_tq_pool;
/* Host only: the rotation [dim][dim] and QJL matrix [dim][dim] of TurboQuant::new(bits, dim,
 * dim, seed) (:76-103: Gram-Schmidt of a SplitMix64 / Box-Muller Gaussian matrix, and a
 * Gaussian matrix of seed ^ 0xDEADBEEF).  Errors through pi_last_error(NULL). */
int pi_tq_generate(int32_t dim, uint64_t seed, float* h_rotation, float* h_qjl);
/* CompressedKVCache::new (:430-447) over a paged pool: n_pages pages of 16 tokens.  Besides
 * the rotation R and QJL matrix G of each KV head, the pool keeps G.R (computed on the host at
 * creation), so a query's virtual query is one product; pi_tq_pool_bytes counts all three. */
int pi_tq_pool_create(pi_handle h, int32_t n_pages, int32_t page_tokens, int32_t n_kv_heads,
                      int32_t head_dim, pi_tq_pool* out);
void pi_tq_pool_destroy(pi_tq_pool pool);
size_t pi_tq_pool_bytes(pi_tq_pool pool);
/* CompressedKVCache::append (:455-486) for n_tok tokens of n_seq sequences: k, v f32
 * [n_seq][n_tok][n_kv_heads][D]; token t of sequence s goes to position start_pos[s] + t. */
int pi_tq_append(pi_handle h, pi_tq_pool pool, const float* d_k, const float* d_v,
                 const int32_t* d_page_table, int32_t max_pages, const int32_t* d_start_pos,
                 int32_t n_seq, int32_t n_tok, void* stream);
/* The stored records of positions start .. start+n_tok-1 of sequence `seq`: keys
 * [n_tok][n_kv_heads][ceil(4D/8)] bytes, norms [n_tok][n_kv_heads] f32, values [n_tok][n_kv_heads][D]
 * as f16 bits. */
int pi_tq_read(pi_handle h, pi_tq_pool pool, const int32_t* d_page_table, int32_t max_pages,
               int32_t seq, int32_t start, int32_t n_tok, uint8_t* d_keys_out, float* d_norms_out,
               uint16_t* d_values_out, void* stream);
/* The compressed-cache branch of the decode attention (src/model/mod.rs:1161-1166:
 * attention_scores with the precomputed query, softmax, weighted_value_sum) for every query
 * head, with the optional sigmoid gate (:1192-1196).  q [batch][n_q_heads][D], out likewise;
 * modulo (PI_GQA_MODULO) or grouped head map; the score scale is 1/sqrt(D) (:490).  D = 128
 * and 256 run the MFMA decode, which keeps every weight (the reference skips weights below
 * 1e-7 in the value sum, :526-529: a difference below the 1e-7-per-token mass it drops);
 * every other D runs the reference's order (all scores, the softmax, then the value sum
 * without the weights below 1e-7), one workgroup per (sequence, query head), with a
 * workspace of batch * n_q_heads * max_pages * 16 floats. */
int pi_tq_attn_decode(pi_handle h, const float* d_q, pi_tq_pool pool, const int32_t* d_page_table,
                      int32_t max_pages, const int32_t* d_ctx_len, int32_t batch,
                      int32_t n_q_heads, int32_t gqa_mode, const float* d_gate, float* d_out,
                      void* stream);

#ifdef __cplusplus
}
#endif
#endif /* PI_ATTN_H */

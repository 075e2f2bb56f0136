// pi_launch.hpp -- host-side launchers implemented in the .hip files and
// called by the C ABI layer (api.cpp).  Arguments are validated by the
// caller; launchers only check what the kernels themselves assume.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace pi {

constexpr int kPageTokens = 16;  // tokens per KV page
constexpr int kItemPages = 16;   // max pages per decode work item (the balancing unit)
constexpr int kMaxBatch = 4096;  // sequences per decode launch (LDS prefix scan)
constexpr int kTqDtype = 3;      // KvGeom::dtype of a TurboQuant pool (head_dim 1..256)
constexpr int kTqMaxDim = 256;
// Bytes of one packed TurboQuant key of head_dim d: 3 d code bits + d QJL sign bits.
// bytes of a TurboQuant key record: 3 code bits and 1 QJL sign bit per coordinate
constexpr int tq_key_bytes(int d) { return (4 * d + 7) / 8; }
// head widths whose decode runs on the MFMA tile (the others on the in-order kernels)
constexpr bool tq_mfma_dim(int d) { return d == 128 || d == 256; }

// KV pool geometry: one K and one V block of kPageTokens x head_dim elements
// per (page, kv head).  K block layout: [head_dim/E][16 tokens][E] with
// E = 16 bytes / element size (16-byte chunks, chunk-major), V block layout:
// [head_dim][16 tokens] (dim-major).  Both match the MFMA operand order the
// decode kernel loads with one linear 16-byte (K) or 8/16-byte (V) access
// per lane.  Block (page, kv head) i = page * n_kv_heads + kv head starts at
// k + i * kstride and v + i * vstride bytes.  The f16 / f32 pool interleaves
// them: K block, then V block, per (page, kv head), so one segment's page is
// one contiguous run of 2 x 16 x D elements (v = k + one block, strides = two).
struct KvGeom {
    void* k;            // device base of K blocks
    void* v;            // device base of V blocks
    int32_t n_pages;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t dtype;      // PI_F32 / PI_F16
    int32_t elem_bytes;
    size_t kstride;     // bytes from one K block to the next
    size_t vstride;     // bytes from one V block to the next
};

// TurboQuant compressed pool (head_dim d = 1..256): g.k holds per (page,
// KV head) 16 packed keys of tq_key_bytes(d) then their 16 f32 norms, g.v the
// f16 V block [d][16]; rt / gt are the per-head rotation and QJL matrices,
// transposed ([h][j][i] = M[h][i][j]) so that lane i reads row i coalesced.
struct TqPool {
    KvGeom g;
    float* rt;
    float* gt;
    float* grt;   // (G.R) transposed per head, for the one-pass virtual query (nullable)
    float scale;  // sqrt(d) in f32: the quantizer's per-coordinate scale
    float corr;   // residual_norm * qjl_scale of the 3-bit estimator
};

struct DecodeWorkspace {
    float* partial_o;     // [slot][G][D]: slot = segment (b * Hkv + kvh) or batch * Hkv + workgroup
    float* partial_ml;    // [slot][G][2]  (running max, sum) in log2 units
    int32_t* seg_runs;    // [segment][2]: (workgroup of run 1, number of runs), set by the
                          // workgroup that starts the segment
    size_t capacity_o;    // floats
    size_t capacity_ml;   // floats
    size_t capacity_runs; // int32 entries
};

struct DecodeParams {
    const float* q;
    const int32_t* page_table;
    const int32_t* ctx_len;
    const float* gate;
    float* out;
    int32_t max_pages;
    int32_t batch;
    int32_t n_q_heads;
    int32_t gqa_mode;
    float scale;
    int32_t item_pages;  // pages per work item (power of 2, <= kItemPages), set by decode_plan
    // Query heads of a KV head ride in the MFMA columns, `cols` (<= 16, cols * D <= 2048) to
    // a segment; a KV head with more splits into n_cb column blocks, each its own segment.
    // group: query heads per KV head for the head map (modulo: ceil(n_q_heads / n_kv_heads),
    // columns whose head would be >= n_q_heads are off).  Set by decode_plan.
    int32_t group;
    int32_t cols;
    int32_t n_cb;
};

struct DecodePlan {
    int32_t grid;        // persistent workgroups (CUs x resident workgroups per CU)
    int32_t batch;
    long long n_slots;   // partial slots: batch * segments per sequence + grid
    int32_t group;       // query heads per KV head of the head map
    int32_t cols;        // query heads per segment
    int32_t n_cb;        // segments (column blocks) per KV head
    int32_t item_pages;  // pages per work item
};
// Floats of the per-GPU fixed scratch behind pi_attn_decode_noalloc (16 MiB).
constexpr size_t kDecodeScratchFloats = (size_t)4 << 20;
// Device address of that scratch on `device`, which must be current; looked up
// once per device with hipGetSymbolAddress.
hipError_t decode_scratch(int device, float** ptr);

// Grid size, head blocking and workspace bound of a decode launch on `device`.  max_tokens
// bounds the tokens any sequence holds (<= 0: 16 * max_pages); it sizes the work items.
DecodePlan decode_plan(const KvGeom& g, int32_t batch, int32_t max_pages, int32_t n_q_heads,
                       int32_t gqa_mode, int device, int32_t max_tokens = 0);
size_t decode_ws_floats_o(const KvGeom& g, const DecodePlan& plan);
// int32 entries of the per-segment run table (2 per (sequence, KV head)).
size_t decode_ws_ints_runs(const KvGeom& g, const DecodePlan& plan);
hipError_t launch_decode(const KvGeom& g, const DecodeParams& p, const DecodeWorkspace& ws,
                         const DecodePlan& plan, hipStream_t s);

hipError_t launch_kv_append(const KvGeom& g, const void* k, const void* v, int32_t src_dtype,
                            const int32_t* page_table, int32_t max_pages,
                            const int32_t* start_pos, int32_t n_seq, int32_t n_tok,
                            hipStream_t s);
hipError_t launch_kv_read(const KvGeom& g, const int32_t* page_table, int32_t max_pages,
                          int32_t seq, int32_t start, int32_t n_tok, float* k_out, float* v_out,
                          hipStream_t s);

hipError_t launch_tq_append(const TqPool& t, const float* k, const float* v,
                            const int32_t* page_table, int32_t max_pages, const int32_t* start_pos,
                            int32_t n_seq, int32_t n_tok, hipStream_t s);
hipError_t launch_tq_read(const TqPool& t, const int32_t* page_table, int32_t max_pages,
                          int32_t seq, int32_t start, int32_t n_tok, uint8_t* keys_out,
                          float* norms_out, uint16_t* v_out, hipStream_t s);
// Virtual queries [batch][n_q_heads][2 head_dim] for the TurboQuant decode.
hipError_t launch_tq_query(const TqPool& t, const float* q, float* qv, int32_t batch,
                           int32_t n_q_heads, int32_t gqa_mode, hipStream_t s);
// The decode of a pool whose head_dim has no MFMA tile (tq_mfma_dim false): qv from
// launch_tq_query ([q_rot | qjl_proj] / sqrt(d) per head row), scores a workspace of
// batch * n_q_heads * max_pages * 16 floats.
hipError_t launch_tq_decode_any(const TqPool& t, const float* qv, const int32_t* page_table,
                                int32_t max_pages, const int32_t* ctx_len, int32_t batch,
                                int32_t n_q_heads, int32_t gqa_mode, const float* gate, float* out,
                                float* scores, hipStream_t s);

struct RopeFreqs {
    float f[128];  // up to head_dim 256 -> 128 pairs
};
hipError_t launch_rope(float* q, float* k, const int32_t* pos, int32_t n_tok, int32_t n_q_heads,
                       int32_t n_kv_heads, int32_t head_dim, int32_t n_pairs, int32_t neox,
                       const RopeFreqs& freqs, hipStream_t s);
hipError_t launch_head_rmsnorm(float* x, const float* w, int32_t n_rows, int32_t dim,
                               int32_t row_stride, float eps, hipStream_t s);
hipError_t launch_softmax(float* x, int32_t n, hipStream_t s);
hipError_t launch_apply_gate(float* out, const float* gate, size_t n, hipStream_t s);
hipError_t launch_fill_iota(int32_t* dst, int32_t n, int32_t first, hipStream_t s);
hipError_t launch_fill_zero(float* dst, size_t n, hipStream_t s);
// Row (t, r), t < n_tok, r < n_rows: `width` floats from src + t * s_tok + r * s_row to
// dst + t * d_tok + r * d_row, zero-filled out to `pad` floats (width <= pad; src and dst
// must not overlap).
hipError_t launch_pack_rows(float* dst, const float* src, int32_t n_tok, int32_t n_rows,
                           int32_t width, int32_t pad, size_t s_tok, size_t s_row, size_t d_tok,
                           size_t d_row, hipStream_t s);
// The same for 16-bit elements (f16 / bf16 bits; zero bits are +0 in both).
hipError_t launch_pack_rows16(uint16_t* dst, const uint16_t* src, int32_t n_tok, int32_t n_rows,
                             int32_t width, int32_t pad, size_t s_tok, size_t s_row, size_t d_tok,
                             size_t d_row, hipStream_t s);
hipError_t launch_attn_prologue(float* q, float* k, const float* v, const float* q_norm_w,
                                const float* k_norm_w, float eps, const RopeFreqs& freqs,
                                int32_t n_pairs, int32_t neox, const KvGeom& g,
                                const int32_t* page_table, int32_t max_pages,
                                const int32_t* start_pos, int32_t n_seq, int32_t n_tok,
                                int32_t n_q_heads, hipStream_t s, int32_t start_scalar = 0,
                                int32_t* ctx_out = nullptr, int32_t n_ctx = 0, int32_t norm_dim = 0);
// norm_dim: the divisor of the per-head RMSNorm's mean square (0: g.head_dim).  A head
// narrower than the pool's head_dim sits in the first norm_dim dims of its row, the rest
// zero; the norm weights past norm_dim are zero so the padding stays zero.

// Causal (or full) flash attention of seq_len query rows per sequence over
// n_keys keys; query row i sits at key position q_off + i (a fresh prompt:
// n_keys = seq_len, q_off = 0).  q / out [batch][seq_len][Hq][D],
// k / v [batch][n_keys][Hkv][D].
// ws: the key-split partials of a launch with fewer workgroups than CUs (floats from
// prefill_ws_floats; 0 = no split).  With ws null or short the launch runs unsplit.
size_t prefill_ws_floats(int32_t batch, int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads,
                         int32_t head_dim, int32_t causal);
hipError_t launch_prefill(const void* q, const void* k, const void* v, int32_t dtype,
                          int32_t batch, int32_t seq_len, int32_t n_keys, int32_t q_off,
                          int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t causal,
                          int32_t gqa_mode, float scale, float* out, float* ws, size_t ws_floats,
                          hipStream_t s, const float* gate = nullptr);
// Causal attention of n_tok f32 query rows [n_tok][Hq][D] at positions q_off ..
// q_off + n_tok - 1 over an f32 pool (D = 64 / 128 / 256), keys read through the
// sequence's page-table row; products at f32 accuracy (bf16 hi + lo splits).
// Causal prefill of n_tok query rows at positions q_off .. of one sequence, its keys 0 ..
// q_off + n_tok - 1 read straight from the f16 pool's pages (head_dim 64, 128 or 256) through
// the sequence's page-table row; q [n_tok][n_q_heads][D] in f32 (q_f32) or f16.  ws: the
// key-split partials (prefill_ws_floats(1, n_tok, ...)).
hipError_t launch_prefill_pool(const KvGeom& g, const void* q, int32_t q_f32, const int32_t* page_table,
                               int32_t q_off, int32_t n_tok, int32_t n_q_heads, int32_t gqa_mode,
                               float scale, float* out, float* ws, size_t ws_floats, hipStream_t s,
                               const float* gate = nullptr);
hipError_t launch_prefill_f32(const KvGeom& g, const float* q, const int32_t* page_table,
                              int32_t max_pages, int32_t q_off, int32_t n_tok, int32_t n_q_heads,
                              int32_t gqa_mode, float scale, float* out, hipStream_t s,
                              const float* gate = nullptr);

hipError_t launch_gdn_gates(const float* beta_raw, const float* a_raw, const float* ssm_a,
                            const float* dt_bias, float* beta, float* g, int32_t n_tok,
                            int32_t n_v_heads, hipStream_t s);
hipError_t launch_gdn_conv1d(const float* x, float* state, const float* w, float* out,
                             int32_t n_seq, int32_t n_tok, int32_t conv_dim, int32_t d_conv,
                             hipStream_t s);
hipError_t launch_gdn_rmsnorm_gated(float* o, const float* z, const float* w, int32_t n_rows,
                                    int32_t n_v_heads, int32_t v_hd, float eps, hipStream_t s);
// One GDN layer step of one token, k_hd = v_hd = 128, d_conv 4: conv1d + SiLU
// (state cs_in -> cs_out, [3][conv_dim] each), gates, delta rule and
// RMSNormGated x SiLU(z) into out [n_v_heads][128], in one launch.
hipError_t launch_gdn_step(const float* x, const float* cs_in, float* cs_out, const float* w,
                           const float* z, const float* beta_raw, const float* a_raw,
                           const float* ssm_a, const float* dt_bias, const float* norm_w, float eps,
                           float* state, float* out, int32_t n_k_heads, int32_t n_v_heads,
                           hipStream_t s);
// Largest key head width of the gated-DeltaNet kernels; k_hd = v_hd = 128
// run the tuned decode / chunked kernels, other widths the per-token kernel.
constexpr int kGdnMaxKhd = 1024;
hipError_t launch_gdn_decode(const float* q, const float* k, const float* v, const float* beta,
                             const float* g, float* state, float* out, int32_t batch,
                             int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd, int32_t v_hd,
                             hipStream_t s);
// The per-token recurrence for any k_hd <= kGdnMaxKhd and v_hd: `batch`
// sequences of one token each, or one sequence of n_tok tokens.
hipError_t launch_gdn_recur(const float* q, const float* k, const float* v, const float* beta,
                            const float* g, float* state, float* out, int32_t batch, int32_t n_tok,
                            int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd, int32_t v_hd,
                            hipStream_t s);

// ssm::ssm_forward of one token (src/ssm/mod.rs:40-157) on device buffers;
// has_* are the reference's slice-length tests, decided by the caller.
struct SsmArgs {
    const float *x, *conv_w, *a, *dt_bias, *alpha, *beta, *out_w;
    float *state, *y;
    float *conv_out, *dt, *bv, *colsum;  // scratch: d_inner, d_inner, d_state, d_inner floats
    int32_t d_inner, d_state, d_conv, has_conv, has_b, has_out;
};
hipError_t launch_ssm_forward(const SsmArgs& a, hipStream_t s);

struct GdnWorkspace {
    float* buf;
    size_t capacity;  // floats
};
size_t gdn_prefill_ws_floats(int32_t n_tok, int32_t n_k_heads, int32_t n_v_heads, int32_t chunk);
hipError_t launch_gdn_prefill(const float* q, const float* k, const float* v, const float* beta,
                              const float* g, float* state, float* out, int32_t n_tok,
                              int32_t n_k_heads, int32_t n_v_heads, int32_t chunk,
                              const GdnWorkspace& ws, hipStream_t s);

}  // namespace pi

// turboquant.hip -- TurboQuant compressed KV cache on gfx950: key
// quantization on append, the per-query precompute, and a read-back of the
// stored records.  The decode itself is decode_kernel with the TurboQuant
// tile (decode.hip).
//
// Replaces CompressedKVCache (src/turboquant/mod.rs:408-566) for head_dim
// D = 1..256 (128 and 256 on the MFMA decode; any other width on the in-order
// kernels at the end of this file): keys are L2-normalised, rotated by the head's orthogonal
// matrix R, scaled by sqrt(D), coded with the 3-bit Lloyd-Max codebook, and
// the residual's D projections on the QJL matrix G keep their signs
// (quantize_vector, :128-187); values are stored as f16 (:481-483).
//
// tq_append_kernel reproduces quantize_vector bit for bit: every sum is the
// reference's sequential f32 loop with a separate multiply and add (this
// file is built with -ffp-contract=off), sqrt and divide are correctly
// rounded, the nearest
// centroid takes the first strict minimum, and a QJL bit is set for a
// projection >= 0.  One wavefront per (sequence, token, KV
// head); lane i owns rotated coordinates i + 64 j, j < D / 64.
#include "pi_device.hpp"
#include "pi_launch.hpp"

namespace pi {
namespace {

__constant__ float kCentroids3[8] = {-2.1520f, -1.3440f, -0.7560f, -0.2451f,
                                     0.2451f,  0.7560f,  1.3440f,  2.1520f};

// Correctly rounded f32 square root of x >= 0: the hardware estimate is
// within one ulp; each neighbour is taken when x lies beyond the midpoint
// between the two, tested in f64, where the squared midpoint (25 significant
// bits) is exact.  A float square root is never exactly such a midpoint.
__device__ __forceinline__ float sqrt_rn(float x) {
    float y = __builtin_sqrtf(x);
    if (!(x > 0.0f) || !(x < 3.0e38f)) return y;
    const double xd = (double)x;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const float up = __int_as_float(__float_as_int(y) + 1);
        const double mu = 0.5 * ((double)y + (double)up);
        if (xd > mu * mu) y = up;
        const float dn = __int_as_float(__float_as_int(y) - 1);
        const double md = 0.5 * ((double)y + (double)dn);
        if (xd < md * md) y = dn;
    }
    return y;
}

__device__ __forceinline__ int nearest_centroid(float x) {
    int best = 0;
    float bd = 3.40282347e+38f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float d = fabsf(__fsub_rn(x, kCentroids3[j]));
        if (d < bd) {
            bd = d;
            best = j;
        }
    }
    return best;
}

template <int D>
__global__ __launch_bounds__(256) void tq_append_kernel(TqPool t, const float* __restrict__ k,
                                                        const float* __restrict__ v,
                                                        const int32_t* __restrict__ page_table,
                                                        int max_pages,
                                                        const int32_t* __restrict__ start_pos,
                                                        int n_seq, int n_tok) {
    constexpr int NJ = D / 64;          // coordinates per lane
    constexpr int CW = 3 * D / 32;      // record dwords of the 3-bit codes
    constexpr int KB = tq_key_bytes(D);
    __shared__ float s_x[4][D];
    __shared__ uint32_t s_bits[4][CW];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n_kv = t.g.n_kv_heads;
    const long long item = (long long)blockIdx.x * 4 + w;
    const bool on = item < (long long)n_seq * n_tok * n_kv;
    const long long it = on ? item : 0;
    const int kvh = (int)(it % n_kv);
    const int tok = (int)((it / n_kv) % n_tok);
    const int seq = (int)(it / ((long long)n_kv * n_tok));
    const size_t row = (((size_t)seq * n_tok + tok) * n_kv + kvh) * D;

    // L2 norm: sequential f32 sum of squares (:466-468)
#pragma unroll
    for (int j = 0; j < NJ; ++j) s_x[w][lane + 64 * j] = k[row + lane + 64 * j];
    if (lane < CW) s_bits[w][lane] = 0u;
    __syncthreads();
    float ss = 0.f;
    for (int j = 0; j < D; ++j) ss = __fadd_rn(ss, __fmul_rn(s_x[w][j], s_x[w][j]));
    const float norm = sqrt_rn(ss);
    const float inv = norm > 1e-12f ? __fdiv_rn(1.0f, norm) : 0.0f;
    float x[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) x[j] = __fmul_rn(s_x[w][lane + 64 * j], inv);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NJ; ++j) s_x[w][lane + 64 * j] = x[j];
    __syncthreads();

    // rotation rows lane + 64 j, then the sqrt(d) scale (:131-146)
    const float* rt = t.rt + (size_t)kvh * D * D;
    float r[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) r[j] = 0.f;
    for (int i = 0; i < D; ++i) {
        const float xi = s_x[w][i];
#pragma unroll
        for (int j = 0; j < NJ; ++j) r[j] = __fadd_rn(r[j], __fmul_rn(rt[i * D + lane + 64 * j], xi));
    }
    int c[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        r[j] = __fmul_rn(r[j], t.scale);
        c[j] = nearest_centroid(r[j]);
    }
    __syncthreads();
    // residual (:170-173); codes: coordinate i occupies bits 3i .. 3i+2 of the record
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int i = lane + 64 * j;
        s_x[w][i] = __fsub_rn(r[j], kCentroids3[c[j]]);
        const uint32_t cv = (uint32_t)c[j];
        const int bit = 3 * i, wd = bit >> 5, off = bit & 31;
        atomicOr(&s_bits[w][wd], cv << off);
        if (off > 29) atomicOr(&s_bits[w][wd + 1], cv >> (32 - off));
    }
    __syncthreads();

    // QJL signs of G . residual (:176-184), one ballot per 64 projections
    const float* gt = t.gt + (size_t)kvh * D * D;
    float pr[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) pr[j] = 0.f;
    for (int i = 0; i < D; ++i) {
        const float ri = s_x[w][i];
#pragma unroll
        for (int j = 0; j < NJ; ++j) pr[j] = __fadd_rn(pr[j], __fmul_rn(gt[i * D + lane + 64 * j], ri));
    }
    uint64_t m[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) m[j] = __ballot(pr[j] >= 0.0f);
    if (!on) return;

    const int pos = start_pos[seq] + tok;
    if (pos < 0 || pos / kPageTokens >= max_pages) return;  // outside the sequence's table
    const int page = page_table[(size_t)seq * max_pages + pos / kPageTokens];
    if (page < 0 || page >= t.g.n_pages) return;
    const int slot = pos % kPageTokens;
    const size_t blk = (size_t)page * n_kv + kvh;
    char* kb = reinterpret_cast<char*>(t.g.k) + blk * (kPageTokens * (KB + 4));
    uint32_t* rec = reinterpret_cast<uint32_t*>(kb + slot * KB);
    if (lane < CW) rec[lane] = s_bits[w][lane];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        if (lane == CW + 2 * j) rec[CW + 2 * j] = (uint32_t)m[j];
        if (lane == CW + 2 * j + 1) rec[CW + 2 * j + 1] = (uint32_t)(m[j] >> 32);
    }
    if (lane == 63) reinterpret_cast<float*>(kb + kPageTokens * KB)[slot] = norm;
    // values as f16 (round to nearest even), V block [dim][16 tokens]
    f16* vb = reinterpret_cast<f16*>(t.g.v) + blk * (kPageTokens * D);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
        vb[(lane + 64 * j) * kPageTokens + slot] = to_f16(v[row + lane + 64 * j]);
}

// Stored records of tokens start .. start+n_tok-1 of one sequence: keys
// [n_tok][Hkv][ceil(D/2)] bytes, norms [n_tok][Hkv], values [n_tok][Hkv][D] f16.
__global__ __launch_bounds__(256) void tq_read_kernel(TqPool t, const int32_t* __restrict__ page_table,
                                                      int max_pages, int seq, int start, int n_tok,
                                                      uint8_t* __restrict__ keys_out,
                                                      float* __restrict__ norms_out,
                                                      uint16_t* __restrict__ v_out) {
    const int D = t.g.head_dim, KB = tq_key_bytes(D);
    const int n_kv = t.g.n_kv_heads;
    const long long total = (long long)n_tok * n_kv * D;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const int d = (int)(e % D);
        const int kvh = (int)((e / D) % n_kv);
        const int i = (int)(e / ((long long)D * n_kv));
        const int pos = start + i;
        if (pos / kPageTokens >= max_pages) continue;
        const int page = page_table[(size_t)seq * max_pages + pos / kPageTokens];
        if (page < 0 || page >= t.g.n_pages) continue;
        const int slot = pos % kPageTokens;
        const size_t blk = (size_t)page * n_kv + kvh;
        const char* kb = reinterpret_cast<const char*>(t.g.k) + blk * (kPageTokens * (KB + 4));
        const uint16_t* vb = reinterpret_cast<const uint16_t*>(t.g.v) + blk * (kPageTokens * D);
        const size_t o = (size_t)i * n_kv + kvh;
        v_out[o * D + d] = vb[d * kPageTokens + slot];
        if (d < KB) keys_out[o * KB + d] = (uint8_t)kb[slot * KB + d];
        if (d == 0) norms_out[o] = reinterpret_cast<const float*>(kb + kPageTokens * KB)[slot];
    }
}

// Virtual query of (sequence b, query head h) (precompute_query,
// :244-278): [R.q / sqrt(d) | corr * G.(R.q) / sqrt(d)], corr =
// residual_norm * qjl_scale of the 3-bit estimator (:297-316).
//
// One workgroup of 256 threads per (sequence, KV head, chunk of up to
// kQueryHeads query heads of that KV head): every matrix element read from
// L2 serves all heads of the chunk.  Thread (half, i) owns output columns
// i + 128 c (c < D / 128) and sums rows j of its half (the matrices are stored
// transposed, so a row step reads 512 contiguous bytes per wavefront); the two
// halves meet in LDS.  The queries sit in LDS as [row][head], one 16-byte read
// per row.
constexpr int kQueryHeads = 4;

template <int D>
__global__ __launch_bounds__(256) void tq_query_kernel(TqPool t, const float* __restrict__ q,
                                                       float* __restrict__ qv, int n_q_heads,
                                                       int gqa_mode) {
    constexpr int NC = D / 128;                  // output columns per thread
    __shared__ float4 s_x[D];                    // query (pass 1) or R.q (pass 2), [row][head]
    __shared__ float s_part[2][kQueryHeads][D];  // per-half partial sums
    const int n_kv = t.g.n_kv_heads;
    // heads of KV head kvh: kvh + j * n_kv below n_q_heads (modulo map), or a block of `group`
    const int group = gqa_mode == 0 ? (n_q_heads + n_kv - 1) / n_kv : n_q_heads / n_kv;
    const int n_chunks = (group + kQueryHeads - 1) / kQueryHeads;
    const int kvh = blockIdx.x / n_chunks, c0 = (blockIdx.x % n_chunks) * kQueryHeads;
    const int b = blockIdx.y, tid = threadIdx.x, half = tid >> 7, i = tid & 127;
    auto head_of = [&](int k) { return gqa_mode == 0 ? kvh + (c0 + k) * n_kv : kvh * group + c0 + k; };
    int nh = 0;  // heads of this chunk that exist
    while (nh < kQueryHeads && c0 + nh < group && head_of(nh) < n_q_heads) ++nh;

    // stage the chunk's queries: thread (half, i) loads heads 2*half, 2*half + 1 of rows i + 128 c
    float* sx = reinterpret_cast<float*>(s_x);
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int k = 2 * half + kk, row = i + 128 * c;
            sx[row * kQueryHeads + k] = k < nh ? q[((size_t)b * n_q_heads + head_of(k)) * D + row] : 0.f;
        }
    __syncthreads();

    const float inv = 1.0f / t.scale;
    float r_own[NC][2];  // R.q of (head 2*half + kk, column i + 128 c), kept for the output
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        const float* mt = (pass == 0 ? t.rt : t.gt) + (size_t)kvh * D * D + (size_t)half * (D / 2) * D + i;
        const float4* xs = s_x + half * (D / 2);
        float acc[NC][kQueryHeads];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int k = 0; k < kQueryHeads; ++k) acc[c][k] = 0.f;
#pragma unroll 8
        for (int j = 0; j < D / 2; ++j) {
            const float4 x = xs[j];
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float m = mt[(size_t)j * D + 128 * c];
                acc[c][0] = fmaf(m, x.x, acc[c][0]);
                acc[c][1] = fmaf(m, x.y, acc[c][1]);
                acc[c][2] = fmaf(m, x.z, acc[c][2]);
                acc[c][3] = fmaf(m, x.w, acc[c][3]);
            }
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int k = 0; k < kQueryHeads; ++k) s_part[half][k][i + 128 * c] = acc[c][k];
        __syncthreads();
        // thread (half, i) finishes heads 2*half, 2*half + 1 of its columns
        float out[NC][2];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int k = 2 * half + kk, col = i + 128 * c;
                out[c][kk] = s_part[0][k][col] + s_part[1][k][col];
            }
        if (pass == 0) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    r_own[c][kk] = out[c][kk];
                    // every read of pass 0 ended at the barrier above
                    sx[(i + 128 * c) * kQueryHeads + 2 * half + kk] = out[c][kk];
                }
            __syncthreads();
        } else {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int k = 2 * half + kk, col = i + 128 * c;
                    if (k >= nh) continue;
                    float* row = qv + ((size_t)b * n_q_heads + head_of(k)) * 2 * D;
                    row[col] = r_own[c][kk] * inv;
                    row[D + col] = t.corr * (out[c][kk] * inv);
                }
        }
    }
}

// One-pass form of the same product: with GR = G.R precomputed per KV head
// (TqPool::grt, transposed), the virtual query is [R; GR].q, so its 2 d rows
// split over workgroups with no dependency between them.  A workgroup owns 64
// of those rows for every query head of one (sequence, KV head); lane l of
// each wavefront owns row 64 blockIdx.x + l and wavefront w sums the quarter
// j = w d / 4 .. of the columns (one coalesced 256-byte read of the transposed
// matrix per column), for up to kQuery2Heads heads whose query values are LDS
// broadcasts; the quarters meet in LDS.  NH (4, 8 or 16) bounds the heads per
// KV head; missing heads are zero queries, so the loops have no branches.
constexpr int kQuery2Heads = 16;

template <int D, int NH>
__global__ __launch_bounds__(256) void tq_query2_kernel(TqPool t, const float* __restrict__ q,
                                                        float* __restrict__ qv, int n_q_heads,
                                                        int gqa_mode) {
    __shared__ __attribute__((aligned(16))) float s_q[NH][D];
    __shared__ float s_part[4][NH][64];
    const int n_kv = t.g.n_kv_heads;
    const int group = gqa_mode == 0 ? (n_q_heads + n_kv - 1) / n_kv : n_q_heads / n_kv;
    const int kvh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    auto head_of = [&](int k) { return gqa_mode == 0 ? kvh + k * n_kv : kvh * group + k; };
    int nh = 0;  // heads of this KV head that exist (group <= NH, checked by the launcher)
    while (nh < group && head_of(nh) < n_q_heads) ++nh;
    const int row = 64 * blockIdx.x + lane;  // of the 2 D outputs; a block never straddles D
    const float* mt = (row < D ? t.rt + (size_t)kvh * D * D + row : t.grt + (size_t)kvh * D * D + (row - D));
    // the wavefront's D / 4 matrix values are all requested first, beside the
    // query loads: one memory round trip (the matrices are rarely still in the
    // caches after the decode kernel has streamed the pool)
    const int j0 = wave * (D / 4);
    float m[D / 4];
#pragma unroll
    for (int e = 0; e < D / 4; ++e) m[e] = mt[(size_t)(j0 + e) * D];
    constexpr int QL = NH * D / 256;  // query values per thread
    float qx[QL];
#pragma unroll
    for (int i = 0; i < QL; ++i) {
        const int idx = tid + 256 * i, k = idx / D, j = idx - k * D;
        qx[i] = k < nh ? q[((size_t)b * n_q_heads + head_of(k)) * D + j] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < QL; ++i) {
        const int idx = tid + 256 * i;
        s_q[idx / D][idx % D] = qx[i];
    }
    __syncthreads();
    float acc[NH];
#pragma unroll
    for (int k = 0; k < NH; ++k) acc[k] = 0.f;
#pragma unroll
    for (int e = 0; e < D / 4; e += 4) {
#pragma unroll
        for (int k = 0; k < NH; ++k) {
            const float4 x = *reinterpret_cast<const float4*>(&s_q[k][j0 + e]);
            acc[k] = fmaf(m[e], x.x, acc[k]);
            acc[k] = fmaf(m[e + 1], x.y, acc[k]);
            acc[k] = fmaf(m[e + 2], x.z, acc[k]);
            acc[k] = fmaf(m[e + 3], x.w, acc[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < NH; ++k) s_part[wave][k][lane] = acc[k];
    __syncthreads();
    const float inv = 1.0f / t.scale;
    for (int k = wave; k < nh; k += 4) {
        const float x = (s_part[0][k][lane] + s_part[1][k][lane]) + (s_part[2][k][lane] + s_part[3][k][lane]);
        float* dst = qv + ((size_t)b * n_q_heads + head_of(k)) * 2 * D;
        dst[row] = row < D ? x * inv : t.corr * (x * inv);
    }
}


// ---------------------------------------------------------------------------
// Any other head_dim (1..256 but 128 and 256).  The record is the reference's
// bit stream (pack_compressed, :591-617): the 3-bit codes of the D rotated
// coordinates, then the D QJL signs, LSB first, ceil(4 D / 8) bytes.  These
// kernels keep the reference's sequential f32 loops: tq_append_any_kernel is
// quantize_vector bit for bit as tq_append_kernel is, tq_query_any_kernel is
// precompute_query (:244-278), and tq_decode_any_kernel runs, for one
// (sequence, query head) per workgroup, attention_scores with
// dot_precomputed (:281-320, :489-516), the softmax, and weighted_value_sum,
// which skips weights below 1e-7 (:519-536).  The softmax's max and sum and
// the value sum's token slices reduce in parallel (the reference's sums are
// sequential), and expf is the device's.
// ---------------------------------------------------------------------------
template <int NJ>
__global__ __launch_bounds__(256) void tq_append_any_kernel(TqPool t, const float* __restrict__ k,
                                                            const float* __restrict__ v,
                                                            const int32_t* __restrict__ page_table,
                                                            int max_pages,
                                                            const int32_t* __restrict__ start_pos,
                                                            int n_seq, int n_tok) {
    __shared__ float s_x[4][kTqMaxDim];
    __shared__ uint32_t s_bits[4][kTqMaxDim / 8];  // 4 D bits
    const int D = t.g.head_dim, KB = tq_key_bytes(D);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n_kv = t.g.n_kv_heads;
    const long long item = (long long)blockIdx.x * 4 + w;
    const bool on = item < (long long)n_seq * n_tok * n_kv;
    const long long it = on ? item : 0;
    const int kvh = (int)(it % n_kv);
    const int tok = (int)((it / n_kv) % n_tok);
    const int seq = (int)(it / ((long long)n_kv * n_tok));
    const size_t row = (((size_t)seq * n_tok + tok) * n_kv + kvh) * D;

#pragma unroll
    for (int j = 0; j < NJ; ++j)
        if (lane + 64 * j < D) s_x[w][lane + 64 * j] = k[row + lane + 64 * j];
    if (lane < kTqMaxDim / 8) s_bits[w][lane] = 0u;
    __syncthreads();
    float ss = 0.f;
    for (int j = 0; j < D; ++j) ss = __fadd_rn(ss, __fmul_rn(s_x[w][j], s_x[w][j]));
    const float norm = sqrt_rn(ss);
    const float inv = norm > 1e-12f ? __fdiv_rn(1.0f, norm) : 0.0f;
    float x[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) x[j] = lane + 64 * j < D ? __fmul_rn(s_x[w][lane + 64 * j], inv) : 0.f;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NJ; ++j)
        if (lane + 64 * j < D) s_x[w][lane + 64 * j] = x[j];
    __syncthreads();

    // rotated coordinate c = lane + 64 j: sum over i of R[c][i] x_i, then the sqrt(d) scale
    const float* rt = t.rt + (size_t)kvh * D * D;
    float r[NJ];
    int c[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int col = lane + 64 * j;
        float acc = 0.f;
        if (col < D)
            for (int i = 0; i < D; ++i) acc = __fadd_rn(acc, __fmul_rn(rt[i * D + col], s_x[w][i]));
        r[j] = __fmul_rn(acc, t.scale);
        c[j] = nearest_centroid(r[j]);
    }
    __syncthreads();
    // residual and codes: coordinate i occupies bits 3i .. 3i+2
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int i = lane + 64 * j;
        if (i >= D) continue;
        s_x[w][i] = __fsub_rn(r[j], kCentroids3[c[j]]);
        const uint32_t cv = (uint32_t)c[j];
        const int bit = 3 * i, wd = bit >> 5, off = bit & 31;
        atomicOr(&s_bits[w][wd], cv << off);
        if (off > 29) atomicOr(&s_bits[w][wd + 1], cv >> (32 - off));
    }
    __syncthreads();
    // QJL sign of projection p at bit 3 D + p: G[p] . residual >= 0
    const float* gt = t.gt + (size_t)kvh * D * D;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int col = lane + 64 * j;
        if (col >= D) continue;
        float pr = 0.f;
        for (int i = 0; i < D; ++i) pr = __fadd_rn(pr, __fmul_rn(gt[i * D + col], s_x[w][i]));
        if (pr >= 0.0f) {
            const int bit = 3 * D + col;
            atomicOr(&s_bits[w][bit >> 5], 1u << (bit & 31));
        }
    }
    __syncthreads();
    if (!on) return;

    const int pos = start_pos[seq] + tok;
    if (pos < 0 || pos / kPageTokens >= max_pages) return;  // outside the sequence's table
    const int page = page_table[(size_t)seq * max_pages + pos / kPageTokens];
    if (page < 0 || page >= t.g.n_pages) return;
    const int slot = pos % kPageTokens;
    const size_t blk = (size_t)page * n_kv + kvh;
    uint8_t* kb = reinterpret_cast<uint8_t*>(t.g.k) + blk * (kPageTokens * (KB + 4));
    for (int b = lane; b < KB; b += 64) kb[slot * KB + b] = (uint8_t)(s_bits[w][b >> 2] >> (8 * (b & 3)));
    if (lane == 0) reinterpret_cast<float*>(kb + kPageTokens * KB)[slot] = norm;
    f16* vb = reinterpret_cast<f16*>(t.g.v) + blk * ((size_t)kPageTokens * D);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
        if (lane + 64 * j < D) vb[(lane + 64 * j) * kPageTokens + slot] = to_f16(v[row + lane + 64 * j]);
}

// precompute_query (:244-278) of (sequence b, query head h): qv row [q_rot | qjl_proj], each
// times 1 / sqrt(d), in the reference's order (qjl_proj from the unscaled q_rot).
__global__ __launch_bounds__(256) void tq_query_any_kernel(TqPool t, const float* __restrict__ q,
                                                           float* __restrict__ qv, int n_q_heads,
                                                           int gqa_mode) {
    __shared__ float s_q[kTqMaxDim], s_r[kTqMaxDim];
    const int D = t.g.head_dim, n_kv = t.g.n_kv_heads;
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const int kvh = gqa_mode == 0 ? h % n_kv : h / (n_q_heads / n_kv);
    const size_t row = (size_t)b * n_q_heads + h;
    if (i < D) s_q[i] = q[row * D + i];
    __syncthreads();
    const float* rt = t.rt + (size_t)kvh * D * D;
    const float* gt = t.gt + (size_t)kvh * D * D;
    float sum = 0.f;
    if (i < D)
        for (int j = 0; j < D; ++j) sum = __fadd_rn(sum, __fmul_rn(rt[j * D + i], s_q[j]));
    if (i < D) s_r[i] = sum;
    __syncthreads();
    if (i >= D) return;
    const float inv = __fdiv_rn(1.0f, t.scale);
    float proj = 0.f;
    for (int j = 0; j < D; ++j) proj = __fadd_rn(proj, __fmul_rn(gt[j * D + i], s_r[j]));
    qv[row * 2 * D + i] = __fmul_rn(sum, inv);
    qv[row * 2 * D + D + i] = __fmul_rn(proj, inv);
}

__device__ __forceinline__ float block_reduce(float x, float* red, bool is_max) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float y = __shfl_xor(x, o);
        x = is_max ? fmaxf(x, y) : x + y;
    }
    __syncthreads();  // red is reused
    if (lane == 0) red[w] = x;
    __syncthreads();
    x = red[0];
    for (int k = 1; k < (int)(blockDim.x >> 6); ++k) x = is_max ? fmaxf(x, red[k]) : x + red[k];
    return x;
}

// One workgroup per (query head h, sequence b): scores of the sequence's T keys into
// sc[(b * Hq + h) * t_cap ..], the softmax, and the value sum without the weights below
// 1e-7.  Keys on a page id outside [0, n_pages) are absent (no score, no weight); with
// none present the output is zero.
__global__ __launch_bounds__(256) void tq_decode_any_kernel(TqPool t, const float* __restrict__ qv,
                                                            const int32_t* __restrict__ page_table,
                                                            int max_pages,
                                                            const int32_t* __restrict__ ctx_len,
                                                            int n_q_heads, int gqa_mode,
                                                            const float* __restrict__ gate,
                                                            float* __restrict__ out,
                                                            float* __restrict__ sc, int t_cap) {
    __shared__ float s_qr[kTqMaxDim], s_qp[kTqMaxDim];
    __shared__ float red[4];
    __shared__ float s_part[256];
    const int D = t.g.head_dim, KB = tq_key_bytes(D), n_kv = t.g.n_kv_heads;
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int kvh = gqa_mode == 0 ? h % n_kv : h / (n_q_heads / n_kv);
    const size_t row = (size_t)b * n_q_heads + h;
    const int T = min(max(ctx_len[b], 0), max_pages * kPageTokens);
    const int32_t* pt = page_table + (size_t)b * max_pages;
    float* s = sc + row * (size_t)t_cap;
    if (tid < D) {
        s_qr[tid] = qv[row * 2 * D + tid];
        s_qp[tid] = qv[row * 2 * D + D + tid];
    }
    __syncthreads();
    const float scale = __fdiv_rn(1.0f, t.scale);  // 1 / sqrt(d) (:490)
    const uint8_t* kpool = reinterpret_cast<const uint8_t*>(t.g.k);
    const f16* vpool = reinterpret_cast<const f16*>(t.g.v);
    float m = -INFINITY;
    for (int tk = tid; tk < T; tk += 256) {
        const int page = pt[tk / kPageTokens], slot = tk % kPageTokens;
        float score = -INFINITY;
        if (page >= 0 && page < t.g.n_pages) {
            const uint8_t* kb = kpool + ((size_t)page * n_kv + kvh) * (kPageTokens * (KB + 4));
            const uint8_t* rec = kb + slot * KB;
            const float kn = reinterpret_cast<const float*>(kb + kPageTokens * KB)[slot];
            float mse = 0.f, qjl = 0.f;
            for (int i = 0; i < D; ++i) {
                const int bit = 3 * i;
                const uint32_t two = (uint32_t)rec[bit >> 3] | ((bit >> 3) + 1 < KB ? (uint32_t)rec[(bit >> 3) + 1] << 8 : 0u);
                const int code = (int)((two >> (bit & 7)) & 7u);
                mse = __fadd_rn(mse, __fmul_rn(s_qr[i], kCentroids3[code]));
            }
            for (int i = 0; i < D; ++i) {
                const int bit = 3 * D + i;
                const float sg = ((rec[bit >> 3] >> (bit & 7)) & 1) ? 1.0f : -1.0f;
                qjl = __fadd_rn(qjl, __fmul_rn(s_qp[i], sg));
            }
            const float res = __fadd_rn(mse, __fmul_rn(t.corr, qjl));
            score = __fmul_rn(__fmul_rn(kn, res), scale);
        }
        s[tk] = score;
        m = fmaxf(m, score);
    }
    m = block_reduce(m, red, true);
    float l = 0.f;
    if (m > -INFINITY) {
        for (int tk = tid; tk < T; tk += 256) {
            const float e = expf(s[tk] - m);
            s[tk] = e;
            l += e;
        }
    }
    l = block_reduce(l, red, false);  // every thread's own writes of s are read back below
    __syncthreads();
    // value sum: thread (slice, d), slices of nsl interleaved tokens, then slice order
    const int nsl = 256 / D, sl = tid / D, d = tid - sl * D;
    float acc = 0.f;
    if (m > -INFINITY && sl < nsl) {
        const float inv = __fdiv_rn(1.0f, l);
        for (int tk = sl; tk < T; tk += nsl) {
            const float wgt = s[tk] * inv;
            if (wgt < 1e-7f) continue;
            const int page = pt[tk / kPageTokens], slot = tk % kPageTokens;
            const f16* vb = vpool + ((size_t)page * n_kv + kvh) * ((size_t)kPageTokens * D);
            acc = __fadd_rn(acc, __fmul_rn(wgt, (float)vb[d * kPageTokens + slot]));
        }
    }
    s_part[tid] = acc;
    __syncthreads();
    if (tid < D) {
        float o = 0.f;
        for (int k2 = 0; k2 < nsl; ++k2) o += s_part[k2 * D + tid];
        if (gate) o *= 1.0f / (1.0f + expf(-gate[row * D + tid]));
        out[row * D + tid] = o;
    }
}
}  // namespace

hipError_t launch_tq_append(const TqPool& t, const float* k, const float* v,
                            const int32_t* page_table, int32_t max_pages, const int32_t* start_pos,
                            int32_t n_seq, int32_t n_tok, hipStream_t s) {
    const long long items = (long long)n_seq * n_tok * t.g.n_kv_heads;
    if (items <= 0) return hipSuccess;
    if ((items + 3) / 4 > 0x7fffffffLL) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((items + 3) / 4));
    if (t.g.head_dim == 128)
        hipLaunchKernelGGL(tq_append_kernel<128>, grid, dim3(256), 0, s, t, k, v, page_table, max_pages,
                           start_pos, n_seq, n_tok);
    else if (t.g.head_dim == 256)
        hipLaunchKernelGGL(tq_append_kernel<256>, grid, dim3(256), 0, s, t, k, v, page_table, max_pages,
                           start_pos, n_seq, n_tok);
    else if (t.g.head_dim < 1 || t.g.head_dim > kTqMaxDim)
        return hipErrorInvalidValue;
    else {
#define PI_TQ_ANY(NJ)                                                                              \
    hipLaunchKernelGGL(tq_append_any_kernel<NJ>, grid, dim3(256), 0, s, t, k, v, page_table, max_pages, \
                       start_pos, n_seq, n_tok)
        const int nj = (t.g.head_dim + 63) / 64;
        if (nj == 1) PI_TQ_ANY(1);
        else if (nj == 2) PI_TQ_ANY(2);
        else if (nj == 3) PI_TQ_ANY(3);
        else PI_TQ_ANY(4);
#undef PI_TQ_ANY
    }
    return hipGetLastError();
}

hipError_t launch_tq_read(const TqPool& t, const int32_t* page_table, int32_t max_pages,
                          int32_t seq, int32_t start, int32_t n_tok, uint8_t* keys_out,
                          float* norms_out, uint16_t* v_out, hipStream_t s) {
    const long long total = (long long)n_tok * t.g.n_kv_heads * t.g.head_dim;
    if (total <= 0) return hipSuccess;
    long long blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (t.g.head_dim < 1 || t.g.head_dim > kTqMaxDim) return hipErrorInvalidValue;
    hipLaunchKernelGGL(tq_read_kernel, dim3((unsigned)blocks), dim3(256), 0, s, t, page_table, max_pages,
                       seq, start, n_tok, keys_out, norms_out, v_out);
    return hipGetLastError();
}

hipError_t launch_tq_query(const TqPool& t, const float* q, float* qv, int32_t batch,
                           int32_t n_q_heads, int32_t gqa_mode, hipStream_t s) {
    if (batch <= 0) return hipSuccess;
    if (!tq_mfma_dim(t.g.head_dim)) {
        if (t.g.head_dim < 1 || t.g.head_dim > kTqMaxDim) return hipErrorInvalidValue;
        hipLaunchKernelGGL(tq_query_any_kernel, dim3((unsigned)n_q_heads, (unsigned)batch), dim3(256), 0, s,
                           t, q, qv, n_q_heads, gqa_mode);
        return hipGetLastError();
    }
    const int n_kv = t.g.n_kv_heads;
    const int group = gqa_mode == 0 ? (n_q_heads + n_kv - 1) / n_kv : n_q_heads / n_kv;
    if (t.grt && group <= kQuery2Heads && group > 0) {
        const dim3 grid2((unsigned)(2 * t.g.head_dim / 64), (unsigned)n_kv, (unsigned)batch);
#define PI_TQ_Q2(DD, NN) \
    hipLaunchKernelGGL((tq_query2_kernel<DD, NN>), grid2, dim3(256), 0, s, t, q, qv, n_q_heads, gqa_mode)
        const int nh = group <= 4 ? 4 : group <= 8 ? 8 : 16;
        if (t.g.head_dim == 128) {
            if (nh == 4) PI_TQ_Q2(128, 4);
            else if (nh == 8) PI_TQ_Q2(128, 8);
            else PI_TQ_Q2(128, 16);
        } else if (t.g.head_dim == 256) {
            if (nh == 4) PI_TQ_Q2(256, 4);
            else if (nh == 8) PI_TQ_Q2(256, 8);
            else PI_TQ_Q2(256, 16);
        } else {
            return hipErrorInvalidValue;
        }
#undef PI_TQ_Q2
        return hipGetLastError();
    }
    const int n_chunks = (group + kQueryHeads - 1) / kQueryHeads;
    const dim3 grid(t.g.n_kv_heads * n_chunks, batch);
    if (t.g.head_dim == 128)
        hipLaunchKernelGGL(tq_query_kernel<128>, grid, dim3(256), 0, s, t, q, qv, n_q_heads, gqa_mode);
    else if (t.g.head_dim == 256)
        hipLaunchKernelGGL(tq_query_kernel<256>, grid, dim3(256), 0, s, t, q, qv, n_q_heads, gqa_mode);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_tq_decode_any(const TqPool& t, const float* qv, const int32_t* page_table,
                                int32_t max_pages, const int32_t* ctx_len, int32_t batch,
                                int32_t n_q_heads, int32_t gqa_mode, const float* gate, float* out,
                                float* scores, hipStream_t s) {
    if (batch <= 0) return hipSuccess;
    if (tq_mfma_dim(t.g.head_dim) || t.g.head_dim < 1 || t.g.head_dim > kTqMaxDim) return hipErrorInvalidValue;
    hipLaunchKernelGGL(tq_decode_any_kernel, dim3((unsigned)n_q_heads, (unsigned)batch), dim3(256), 0, s, t,
                       qv, page_table, max_pages, ctx_len, n_q_heads, gqa_mode, gate, out, scores,
                       max_pages * kPageTokens);
    return hipGetLastError();
}

}  // namespace pi

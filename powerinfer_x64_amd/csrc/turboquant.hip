// turboquant.hip -- TurboQuant compressed KV cache on gfx950: key
// quantization on append, the per-query precompute, and a read-back of the
// stored records.  The decode itself is decode_kernel with the TurboQuant
// tile (decode.hip).
//
// Replaces CompressedKVCache (src/turboquant/mod.rs:408-566) with head_dim
// 128: keys are L2-normalised, rotated by the head's orthogonal matrix R,
// scaled by sqrt(128), coded with the 3-bit Lloyd-Max codebook, and the
// residual's projections on the QJL matrix G keep their signs
// (quantize_vector, :128-187); values are stored as f16 (:481-483).
//
// tq_append_kernel reproduces quantize_vector bit for bit: every sum is the
// reference's sequential f32 loop with a separate multiply and add (this
// file is built with -ffp-contract=off), sqrt and divide are correctly
// rounded, the nearest
// centroid takes the first strict minimum, and a QJL bit is set for a
// projection >= 0.  One wavefront per (sequence, token, KV
// head); lane i owns rotated coordinates i and i + 64.
#include "pi_device.hpp"
#include "pi_launch.hpp"

namespace pi {
namespace {

constexpr int TD = 128;  // head_dim of the TurboQuant pool

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

__global__ __launch_bounds__(256) void tq_append_kernel(TqPool t, const float* __restrict__ k,
                                                        const float* __restrict__ v,
                                                        const int32_t* __restrict__ page_table,
                                                        int max_pages,
                                                        const int32_t* __restrict__ start_pos,
                                                        int n_seq, int n_tok) {
    __shared__ float s_x[4][TD];
    __shared__ uint32_t s_bits[4][12];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n_kv = t.g.n_kv_heads;
    const long long item = (long long)blockIdx.x * 4 + w;
    const bool on = item < (long long)n_seq * n_tok * n_kv;
    const long long it = on ? item : 0;
    const int kvh = (int)(it % n_kv);
    const int tok = (int)((it / n_kv) % n_tok);
    const int seq = (int)(it / ((long long)n_kv * n_tok));
    const size_t row = (((size_t)seq * n_tok + tok) * n_kv + kvh) * TD;

    // L2 norm: sequential f32 sum of squares (:466-468)
    s_x[w][lane] = k[row + lane];
    s_x[w][lane + 64] = k[row + lane + 64];
    if (lane < 12) s_bits[w][lane] = 0u;
    __syncthreads();
    float ss = 0.f;
    for (int j = 0; j < TD; ++j) ss = __fadd_rn(ss, __fmul_rn(s_x[w][j], s_x[w][j]));
    const float norm = sqrt_rn(ss);
    const float inv = norm > 1e-12f ? __fdiv_rn(1.0f, norm) : 0.0f;
    const float x0 = __fmul_rn(s_x[w][lane], inv), x1 = __fmul_rn(s_x[w][lane + 64], inv);
    __syncthreads();
    s_x[w][lane] = x0;
    s_x[w][lane + 64] = x1;
    __syncthreads();

    // rotation rows lane, lane + 64, then the sqrt(d) scale (:131-146)
    const float* rt = t.rt + (size_t)kvh * TD * TD;
    float r0 = 0.f, r1 = 0.f;
    for (int j = 0; j < TD; ++j) {
        const float xj = s_x[w][j];
        r0 = __fadd_rn(r0, __fmul_rn(rt[j * TD + lane], xj));
        r1 = __fadd_rn(r1, __fmul_rn(rt[j * TD + lane + 64], xj));
    }
    r0 = __fmul_rn(r0, t.scale);
    r1 = __fmul_rn(r1, t.scale);
    const int c0 = nearest_centroid(r0), c1 = nearest_centroid(r1);
    __syncthreads();
    s_x[w][lane] = __fsub_rn(r0, kCentroids3[c0]);  // residual (:170-173)
    s_x[w][lane + 64] = __fsub_rn(r1, kCentroids3[c1]);
    // codes: coordinate i occupies bits 3i .. 3i+2 of the record
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = lane + 64 * h;
        const uint32_t c = (uint32_t)(h ? c1 : c0);
        const int bit = 3 * i, wd = bit >> 5, off = bit & 31;
        atomicOr(&s_bits[w][wd], c << off);
        if (off > 29) atomicOr(&s_bits[w][wd + 1], c >> (32 - off));
    }
    __syncthreads();

    // QJL signs of G . residual (:176-184)
    const float* gt = t.gt + (size_t)kvh * TD * TD;
    float p0 = 0.f, p1 = 0.f;
    for (int j = 0; j < TD; ++j) {
        const float rj = s_x[w][j];
        p0 = __fadd_rn(p0, __fmul_rn(gt[j * TD + lane], rj));
        p1 = __fadd_rn(p1, __fmul_rn(gt[j * TD + lane + 64], rj));
    }
    const uint64_t m0 = __ballot(p0 >= 0.0f), m1 = __ballot(p1 >= 0.0f);
    if (!on) return;

    const int pos = start_pos[seq] + tok;
    if (pos < 0 || pos / kPageTokens >= max_pages) return;  // outside the sequence's table
    const int page = page_table[(size_t)seq * max_pages + pos / kPageTokens];
    if (page < 0 || page >= t.g.n_pages) return;
    const int slot = pos % kPageTokens;
    const size_t blk = (size_t)page * n_kv + kvh;
    char* kb = reinterpret_cast<char*>(t.g.k) + blk * (kPageTokens * (kTqKeyBytes + 4));
    uint32_t* rec = reinterpret_cast<uint32_t*>(kb + slot * kTqKeyBytes);
    if (lane < 12) rec[lane] = s_bits[w][lane];
    if (lane == 12) rec[12] = (uint32_t)m0;
    if (lane == 13) rec[13] = (uint32_t)(m0 >> 32);
    if (lane == 14) rec[14] = (uint32_t)m1;
    if (lane == 15) rec[15] = (uint32_t)(m1 >> 32);
    if (lane == 16) reinterpret_cast<float*>(kb + kPageTokens * kTqKeyBytes)[slot] = norm;
    // values as f16 (round to nearest even), V block [dim][16 tokens]
    f16* vb = reinterpret_cast<f16*>(t.g.v) + blk * (kPageTokens * TD);
    vb[lane * kPageTokens + slot] = to_f16(v[row + lane]);
    vb[(lane + 64) * kPageTokens + slot] = to_f16(v[row + lane + 64]);
}

// Stored records of tokens start .. start+n_tok-1 of one sequence: keys
// [n_tok][Hkv][64] bytes, norms [n_tok][Hkv], values [n_tok][Hkv][128] f16.
__global__ __launch_bounds__(256) void tq_read_kernel(TqPool t, const int32_t* __restrict__ page_table,
                                                      int max_pages, int seq, int start, int n_tok,
                                                      uint8_t* __restrict__ keys_out,
                                                      float* __restrict__ norms_out,
                                                      uint16_t* __restrict__ v_out) {
    const int n_kv = t.g.n_kv_heads;
    const long long total = (long long)n_tok * n_kv * TD;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const int d = (int)(e % TD);
        const int kvh = (int)((e / TD) % n_kv);
        const int i = (int)(e / ((long long)TD * n_kv));
        const int pos = start + i;
        if (pos / kPageTokens >= max_pages) continue;
        const int page = page_table[(size_t)seq * max_pages + pos / kPageTokens];
        if (page < 0 || page >= t.g.n_pages) continue;
        const int slot = pos % kPageTokens;
        const size_t blk = (size_t)page * n_kv + kvh;
        const char* kb = reinterpret_cast<const char*>(t.g.k) + blk * (kPageTokens * (kTqKeyBytes + 4));
        const uint16_t* vb = reinterpret_cast<const uint16_t*>(t.g.v) + blk * (kPageTokens * TD);
        const size_t o = (size_t)i * n_kv + kvh;
        v_out[o * TD + d] = vb[d * kPageTokens + slot];
        if (d < kTqKeyBytes) keys_out[o * kTqKeyBytes + d] = (uint8_t)kb[slot * kTqKeyBytes + d];
        if (d == 0) norms_out[o] = reinterpret_cast<const float*>(kb + kPageTokens * kTqKeyBytes)[slot];
    }
}

// Virtual query of (sequence b, query head h) (precompute_query,
// :244-278): [R.q / sqrt(d) | corr * G.(R.q) / sqrt(d)], corr =
// residual_norm * qjl_scale of the 3-bit estimator (:297-316).
//
// One workgroup of 256 threads per (sequence, KV head, chunk of up to
// kQueryHeads query heads of that KV head): every matrix element read from
// L2 serves all heads of the chunk.  Thread (half, i) owns output column i
// and sums rows j of its half (the matrices are stored transposed, so a row
// step reads 512 contiguous bytes per wavefront); the two halves meet in
// LDS.  The queries sit in LDS as [row][head], one 16-byte read per row.
constexpr int kQueryHeads = 4;

__global__ __launch_bounds__(256) void tq_query_kernel(TqPool t, const float* __restrict__ q,
                                                       float* __restrict__ qv, int n_q_heads,
                                                       int gqa_mode) {
    __shared__ float4 s_x[TD];                    // query (pass 1) or R.q (pass 2), [row][head]
    __shared__ float s_part[2][kQueryHeads][TD];  // per-half partial sums
    const int n_kv = t.g.n_kv_heads;
    const int group = n_q_heads / n_kv;
    const int n_chunks = (group + kQueryHeads - 1) / kQueryHeads;
    const int kvh = blockIdx.x / n_chunks, c0 = (blockIdx.x % n_chunks) * kQueryHeads;
    const int nh = min(kQueryHeads, group - c0);
    const int b = blockIdx.y, tid = threadIdx.x, half = tid >> 7, i = tid & (TD - 1);
    auto head_of = [&](int k) { return gqa_mode == 0 ? kvh + (c0 + k) * n_kv : kvh * group + c0 + k; };

    // stage the chunk's queries: thread (half, i) loads heads 2*half, 2*half + 1 of row i
    float* sx = reinterpret_cast<float*>(s_x);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        const int k = 2 * half + kk;
        sx[i * kQueryHeads + k] = k < nh ? q[((size_t)b * n_q_heads + head_of(k)) * TD + i] : 0.f;
    }
    __syncthreads();

    const float inv = 1.0f / t.scale;
    float r_own[2] = {0.f, 0.f};  // R.q of (head 2*half + kk, column i), kept for the output
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        const float* mt = (pass == 0 ? t.rt : t.gt) + (size_t)kvh * TD * TD + (size_t)half * (TD / 2) * TD + i;
        const float4* xs = s_x + half * (TD / 2);
        float acc[kQueryHeads] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 16
        for (int j = 0; j < TD / 2; ++j) {
            const float m = mt[(size_t)j * TD];
            const float4 x = xs[j];
            acc[0] = fmaf(m, x.x, acc[0]);
            acc[1] = fmaf(m, x.y, acc[1]);
            acc[2] = fmaf(m, x.z, acc[2]);
            acc[3] = fmaf(m, x.w, acc[3]);
        }
#pragma unroll
        for (int k = 0; k < kQueryHeads; ++k) s_part[half][k][i] = acc[k];
        __syncthreads();
        // thread (half, i) finishes heads 2*half, 2*half + 1 of column i
        float out[2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int k = 2 * half + kk;
            out[kk] = s_part[0][k][i] + s_part[1][k][i];
        }
        if (pass == 0) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                r_own[kk] = out[kk];
                sx[i * kQueryHeads + 2 * half + kk] = out[kk];  // every read of pass 0 ended at the barrier
            }
            __syncthreads();
        } else {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int k = 2 * half + kk;
                if (k >= nh) continue;
                float* row = qv + ((size_t)b * n_q_heads + head_of(k)) * 2 * TD;
                row[i] = r_own[kk] * inv;
                row[TD + i] = t.corr * (out[kk] * inv);
            }
        }
    }
}

}  // namespace

hipError_t launch_tq_append(const TqPool& t, const float* k, const float* v,
                            const int32_t* page_table, int32_t max_pages, const int32_t* start_pos,
                            int32_t n_seq, int32_t n_tok, hipStream_t s) {
    const long long items = (long long)n_seq * n_tok * t.g.n_kv_heads;
    if (items <= 0) return hipSuccess;
    if ((items + 3) / 4 > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(tq_append_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, t, k,
                       v, page_table, max_pages, start_pos, n_seq, n_tok);
    return hipGetLastError();
}

hipError_t launch_tq_read(const TqPool& t, const int32_t* page_table, int32_t max_pages,
                          int32_t seq, int32_t start, int32_t n_tok, uint8_t* keys_out,
                          float* norms_out, uint16_t* v_out, hipStream_t s) {
    const long long total = (long long)n_tok * t.g.n_kv_heads * TD;
    if (total <= 0) return hipSuccess;
    long long blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(tq_read_kernel, dim3((unsigned)blocks), dim3(256), 0, s, t, page_table,
                       max_pages, seq, start, n_tok, keys_out, norms_out, v_out);
    return hipGetLastError();
}

hipError_t launch_tq_query(const TqPool& t, const float* q, float* qv, int32_t batch,
                           int32_t n_q_heads, int32_t gqa_mode, hipStream_t s) {
    if (batch <= 0) return hipSuccess;
    const int group = n_q_heads / t.g.n_kv_heads;
    const int n_chunks = (group + kQueryHeads - 1) / kQueryHeads;
    hipLaunchKernelGGL(tq_query_kernel, dim3(t.g.n_kv_heads * n_chunks, batch), dim3(256), 0, s, t,
                       q, qv, n_q_heads, gqa_mode);
    return hipGetLastError();
}

}  // namespace pi

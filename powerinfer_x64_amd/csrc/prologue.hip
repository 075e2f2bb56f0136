// prologue.hip -- the steps in front of attention: paged KV append/read,
// rotary embedding and per-head RMSNorm (gfx950).
//
//   kv_append   : LayerCache append (src/model/mod.rs:1140-1146) into the paged pool
//   kv_read     : pool -> reference layout [T][n_kv][D] f32
//   rope        : ops::apply_rope / apply_rope_with_freqs (src/ops.rs:35-67,130-157)
//                 as driven by src/model/mod.rs:1072-1138
//   head_rmsnorm: ops::rms_norm per head (src/ops.rs:13-27; src/model/mod.rs:1035-1070)
//   softmax     : ops::softmax on one row (src/ops.rs:160-180)
//   attn_prologue: the three above fused for a whole layer step
//                 (src/model/mod.rs:1035-1146): norm, RoPE, append
#include <cstdlib>

#include "pi_device.hpp"
#include "pi_launch.hpp"

namespace pi {
namespace {

template <typename PT>
__device__ __forceinline__ size_t k_index(int tok, int d) {
    constexpr int E = 16 / (int)sizeof(PT);
    return ((size_t)(d / E) * kPageTokens + tok) * E + (d % E);
}
__device__ __forceinline__ size_t v_index(int tok, int d) { return (size_t)d * kPageTokens + tok; }

template <typename ST, typename PT>
__global__ __launch_bounds__(256) void kv_append_kernel(KvGeom g, const ST* __restrict__ k,
                                                        const ST* __restrict__ v,
                                                        const int32_t* __restrict__ pt,
                                                        int max_pages,
                                                        const int32_t* __restrict__ start_pos,
                                                        int n_seq, int n_tok) {
    const int D = g.head_dim, H = g.n_kv_heads;
    const size_t total = (size_t)n_seq * n_tok * H * D;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int d = (int)(idx % D);
        const int h = (int)((idx / D) % H);
        const int t = (int)((idx / ((size_t)D * H)) % n_tok);
        const int s = (int)(idx / ((size_t)D * H * n_tok));
        const int pos = start_pos[s] + t;
        const int lp = pos / kPageTokens;
        if (pos < 0 || lp >= max_pages) continue;  // outside the sequence's table: dropped
        const int page = pt[(size_t)s * max_pages + lp];
        if (page < 0 || page >= g.n_pages) continue;
        const int tok = pos % kPageTokens;
        const size_t blk = (size_t)page * H + h;
        PT* kp = reinterpret_cast<PT*>(static_cast<char*>(g.k) + blk * g.kstride);
        PT* vp = reinterpret_cast<PT*>(static_cast<char*>(g.v) + blk * g.vstride);
        kp[k_index<PT>(tok, d)] = from_f32<PT>(to_f32(k[idx]));
        vp[v_index(tok, d)] = from_f32<PT>(to_f32(v[idx]));
    }
}

// Append by page block: workgroup (x, h) writes the slots that sequence x / ppn
// appends into its (x % ppn)-th page touched (ppn = pages one call can touch:
// ceil(n_tok / 16) + 1), K head h, as whole 16-byte chunks of the block where the
// chunk's tokens all belong to the call, so each block is written by one
// workgroup in full lines (the element-per-thread form spread a page's 2-byte
// writes over every XCD's L2, and HBM took twice the bytes).  Slots outside the
// call, positions past the table, and page ids outside the pool are left alone.
template <typename ST, typename PT>
__global__ __launch_bounds__(256) void kv_append_page_kernel(KvGeom g, const ST* __restrict__ k,
                                                             const ST* __restrict__ v,
                                                             const int32_t* __restrict__ pt,
                                                             int max_pages,
                                                             const int32_t* __restrict__ start_pos,
                                                             int n_tok, int ppn) {
    constexpr int E = 16 / (int)sizeof(PT);  // pool values per 16-byte chunk
    typedef PT pv __attribute__((ext_vector_type(E)));
    const int D = g.head_dim, H = g.n_kv_heads;
    const int sq = blockIdx.x / ppn, j = blockIdx.x % ppn, h = blockIdx.y;
    const long long start = start_pos[sq];
    const long long first = start > 0 ? start : 0;        // positions below 0 are dropped
    const long long lpl = first / kPageTokens + j;         // page of the sequence's table
    if (lpl >= max_pages) return;
    const int lp = (int)lpl;
    const long long t0 = first > lpl * kPageTokens ? first : lpl * kPageTokens;
    const long long t1 = start + n_tok < (lpl + 1) * kPageTokens ? start + n_tok : (lpl + 1) * kPageTokens;
    if (t0 >= t1) return;
    const int page = pt[(size_t)sq * max_pages + lp];
    if (page < 0 || page >= g.n_pages) return;
    const size_t blk = (size_t)page * H + h;
    PT* kp = reinterpret_cast<PT*>(static_cast<char*>(g.k) + blk * g.kstride);
    PT* vp = reinterpret_cast<PT*>(static_cast<char*>(g.v) + blk * g.vstride);
    const int s0 = (int)(t0 - lpl * kPageTokens), s1 = (int)(t1 - lpl * kPageTokens);  // slots [s0, s1)
    auto src = [&](const ST* base, int slot, int d) {  // the call's value of slot, dim d
        const int t = (int)(lpl * kPageTokens + slot - start);
        return to_f32(base[(((size_t)sq * n_tok + t) * H + h) * D + d]);
    };
    // K block [D / E][16][E]: chunk c = (dims E (c / 16) .., slot c % 16)
    for (int c = threadIdx.x; c < D / E * kPageTokens; c += 256) {
        const int slot = c % kPageTokens, d0 = E * (c / kPageTokens);
        if (slot < s0 || slot >= s1) continue;
        pv x;
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = from_f32<PT>(src(k, slot, d0 + e));
        *reinterpret_cast<pv*>(kp + (size_t)E * c) = x;
    }
    // V block [D][16]: chunk c = (dim c / (16 / E), slots E (c % (16 / E)) ..)
    constexpr int CPR = kPageTokens / E;  // chunks per dim row
    for (int c = threadIdx.x; c < D * CPR; c += 256) {
        const int d = c / CPR, sl0 = E * (c % CPR);
        if (sl0 + E <= s0 || sl0 >= s1) continue;
        if (sl0 >= s0 && sl0 + E <= s1) {
            pv x;
#pragma unroll
            for (int e = 0; e < E; ++e) x[e] = from_f32<PT>(src(v, sl0 + e, d));
            *reinterpret_cast<pv*>(vp + (size_t)E * c) = x;
        } else {  // a chunk the call covers in part: its own slots only
            for (int e = 0; e < E; ++e)
                if (sl0 + e >= s0 && sl0 + e < s1) vp[(size_t)E * c + e] = from_f32<PT>(src(v, sl0 + e, d));
        }
    }
}

template <typename PT>
__global__ __launch_bounds__(256) void kv_read_kernel(KvGeom g, const int32_t* __restrict__ pt,
                                                      int max_pages, int seq, int start,
                                                      int n_tok, float* __restrict__ ko,
                                                      float* __restrict__ vo) {
    const int D = g.head_dim, H = g.n_kv_heads;
    const size_t total = (size_t)n_tok * H * D;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int d = (int)(idx % D);
        const int h = (int)((idx / D) % H);
        const int t = (int)(idx / ((size_t)D * H));
        const int pos = start + t;
        const int lp = pos / kPageTokens;
        float kv = 0.f, vv = 0.f;
        if (pos >= 0 && lp < max_pages) {
            const int page = pt[(size_t)seq * max_pages + lp];
            if (page >= 0 && page < g.n_pages) {
                const int tok = pos % kPageTokens;
                const size_t blk = (size_t)page * H + h;
                kv = to_f32(reinterpret_cast<const PT*>(static_cast<const char*>(g.k) + blk * g.kstride)[k_index<PT>(tok, d)]);
                vv = to_f32(reinterpret_cast<const PT*>(static_cast<const char*>(g.v) + blk * g.vstride)[v_index(tok, d)]);
            }
        }
        ko[idx] = kv;
        vo[idx] = vv;
    }
}

// One thread per (token, head, rotated pair).  theta = (f32)position * freq,
// freq from the host-built table (the reference's own f32 formula), so only
// cos/sin are evaluated on the device.
__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ q, float* __restrict__ k,
                                                   const int32_t* __restrict__ pos, int n_tok,
                                                   int hq, int hkv, int D, int n_pairs, int neox,
                                                   RopeFreqs f) {
    const int heads = hq + (k ? hkv : 0);
    const size_t total = (size_t)n_tok * heads * n_pairs;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int i = (int)(idx % n_pairs);
        const int hh = (int)((idx / n_pairs) % heads);
        const int t = (int)(idx / ((size_t)n_pairs * heads));
        float* x = hh < hq ? q + ((size_t)t * hq + hh) * D : k + ((size_t)t * hkv + (hh - hq)) * D;
        const int a = neox ? i : 2 * i;
        const int b = neox ? i + n_pairs : 2 * i + 1;
        if (b >= D) continue;
        const float theta = (float)pos[t] * f.f[i];
        const float c = cosf(theta), s = sinf(theta);
        const float x0 = x[a], x1 = x[b];
        x[a] = x0 * c - x1 * s;
        x[b] = x0 * s + x1 * c;
    }
}

// One wavefront per row (any dim): sum of squares, then x * (1/rms) * w.
__global__ __launch_bounds__(256) void head_rmsnorm_kernel(float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           int n_rows, int dim, int row_stride,
                                                           float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n_rows) return;
    float* xr = x + (size_t)row * row_stride;
    float ss = 0.f;
    for (int d = lane; d < dim; d += 64) ss += xr[d] * xr[d];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss = wave_sum_xor(ss, m);
    const float rms = sqrtf(ss / (float)dim + eps);
    const float inv = 1.0f / rms;
    for (int d = lane; d < dim; d += 64) xr[d] = (xr[d] * inv) * w[d];
}

// ops::softmax (src/ops.rs:160-180) on one row of n values, in place: max,
// exp(x - max), sum, x * (1 / sum).  One workgroup.
__global__ __launch_bounds__(1024) void softmax_row_kernel(float* __restrict__ x, int n) {
    __shared__ float red[16];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float m = -INFINITY;
    for (int i = tid; i < n; i += 1024) m = fmaxf(m, x[i]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = wave_max_xor(m, o);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = red[0];
    for (int i = 1; i < 16; ++i) m = fmaxf(m, red[i]);
    __syncthreads();
    float sum = 0.f;
    for (int i = tid; i < n; i += 1024) {
        const float e = expf(x[i] - m);
        x[i] = e;
        sum += e;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum = wave_sum_xor(sum, o);
    if (lane == 0) red[wv] = sum;
    __syncthreads();
    sum = 0.f;
    for (int i = 0; i < 16; ++i) sum += red[i];
    const float inv = 1.0f / sum;
    for (int i = tid; i < n; i += 1024) x[i] *= inv;
}

// Start positions of a prologue launch: one per sequence on the device, or (dev null) the
// scalar first position of a one-sequence launch.  A launch may also write the context
// lengths of the decode rows that follow it, ctx_out[i] = scalar + 1 + i for i < n_ctx
// (row i attends the keys up to its own position), so the layer step needs no launch of
// its own for them.
struct PrologueStart {
    const int32_t* dev;
    int32_t scalar;
    int32_t* ctx_out;
    int32_t n_ctx;
    int32_t wg0;  // the workgroup (x) that writes ctx_out: the first token workgroup
    __device__ __forceinline__ int of(int sq) const { return dev ? dev[sq] : scalar; }
    __device__ __forceinline__ void write_ctx() const {
        if (ctx_out && (int)blockIdx.x == wg0 && blockIdx.y == 0)
            for (int i = threadIdx.x; i < n_ctx; i += blockDim.x) ctx_out[i] = scalar + 1 + i;
    }
};

// Fused decode / prefill prologue of a full-attention layer
// (src/model/mod.rs:1035-1146): for token t of sequence s at position
// start_pos[s] + t, every q head and k head is RMS-normed (optional weights)
// and rotated (NORM adjacent pairs or NeoX pairs with the host-built
// frequency table), q in place, k in place and appended with v to the paged
// pool.  Workgroup (x, y) = (sequence and token, y-th group of the token's
// head rows): the token's cos / sin table is computed once into LDS (the angle
// depends only on the position and the pair), then the 4 wavefronts take the
// group's head rows in turn, each row staged in LDS.  Prompts use one group
// per token (the table is shared by all heads); a launch of few tokens splits
// the heads four to a group, so the rows still spread over the chip, and
// computes each angle where it is used (no table, no barrier).
template <typename PT>
__global__ __launch_bounds__(256) void attn_prologue_kernel(
    float* __restrict__ q, float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ qn, const float* __restrict__ kn, float eps, RopeFreqs f,
    int n_pairs, int neox, KvGeom g, const int32_t* __restrict__ pt, int max_pages,
    PrologueStart start_pos, int n_seq, int n_tok, int hq, int norm_d) {
    __shared__ float row_s[4][256];
    __shared__ float cs_s[2][128];  // cos, sin of pair i at this token's position
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int D = g.head_dim, hkv = g.n_kv_heads, heads = hq + hkv;
    const int t = blockIdx.x % n_tok, sq = blockIdx.x / n_tok;
    const int pos = start_pos.of(sq) + t;
    start_pos.write_ctx();
    const bool table = gridDim.y == 1;  // uniform per launch
    if (table) {
        for (int i = threadIdx.x; i < n_pairs; i += 256) {
            const float theta = (float)pos * f.f[i];
            cs_s[0][i] = cosf(theta);
            cs_s[1][i] = sinf(theta);
        }
        __syncthreads();
    }
    float* r = row_s[wv];
    const int per = (heads + gridDim.y - 1) / gridDim.y;
    const int h1 = min(heads, (int)(blockIdx.y + 1) * per);
    for (int head = blockIdx.y * per + wv; head < h1; head += 4) {
        const bool is_q = head < hq;
        const int kvh = head - hq;
        float* x = is_q ? q + (((size_t)sq * n_tok + t) * hq + head) * D
                        : k + (((size_t)sq * n_tok + t) * hkv + kvh) * D;
        const float* nw = is_q ? qn : kn;
        float ss = 0.f;
        for (int d = lane; d < D; d += 64) {
            const float xv = x[d];
            r[d] = xv;
            ss += xv * xv;
        }
        if (nw) {  // ops::rms_norm (src/ops.rs:13-27) per head
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) ss = wave_sum_xor(ss, m);
            const float inv = 1.0f / sqrtf(ss / (float)norm_d + eps);
            for (int d = lane; d < D; d += 64) r[d] = (r[d] * inv) * nw[d];
        }
        __builtin_amdgcn_wave_barrier();
        for (int i = lane; i < n_pairs; i += 64) {  // ops::apply_rope / apply_rope_with_freqs
            const int a = neox ? i : 2 * i;
            const int b = neox ? i + n_pairs : 2 * i + 1;
            if (b >= D) continue;
            float c, sn;
            if (table) {
                c = cs_s[0][i];
                sn = cs_s[1][i];
            } else {
                const float theta = (float)pos * f.f[i];
                c = cosf(theta);
                sn = sinf(theta);
            }
            const float x0 = r[a], x1 = r[b];
            r[a] = x0 * c - x1 * sn;
            r[b] = x0 * sn + x1 * c;
        }
        __builtin_amdgcn_wave_barrier();
        for (int d = lane; d < D; d += 64) x[d] = r[d];
        // append-then-attend (src/model/mod.rs:1140-1146): K (normed, rotated) and V at pos
        const int lp = pos / kPageTokens;
        if (!is_q && pos >= 0 && lp < max_pages) {
            const int page = pt[(size_t)sq * max_pages + lp];
            if (page >= 0 && page < g.n_pages) {
                const int tok = pos % kPageTokens;
                const size_t blk = (size_t)page * hkv + kvh;
                PT* kp = reinterpret_cast<PT*>(static_cast<char*>(g.k) + blk * g.kstride);
                PT* vp = reinterpret_cast<PT*>(static_cast<char*>(g.v) + blk * g.vstride);
                const float* vr = v + (((size_t)sq * n_tok + t) * hkv + kvh) * D;
                for (int d = lane; d < D; d += 64) {
                    kp[k_index<PT>(tok, d)] = from_f32<PT>(r[d]);
                    vp[v_index(tok, d)] = from_f32<PT>(vr[d]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // the next row reuses r
    }
}

// The same prologue with each head row in registers: lane l holds the EPL =
// D / 64 consecutive values EPL l .. +EPL-1, loaded and stored as one vector,
// so a row needs no LDS staging and no wave barriers.  The RMS norm reduces
// across the wavefront; NORM pairs (2i, 2i+1) lie in one lane (EPL >= 2) or
// in lanes l, l ^ 1 (EPL = 1); NeoX pairs (i, i + n_pairs) in lanes l and
// l +- n_pairs / EPL, which needs n_pairs to be a multiple of EPL (the launch
// falls back to attn_prologue_kernel otherwise).
template <int N>
__device__ __forceinline__ void load_vec(float* d, const float* s) {
    if constexpr (N == 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(s);
        d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
    } else if constexpr (N == 2) {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        const f32x2 v = *reinterpret_cast<const f32x2*>(s);
        d[0] = v[0]; d[1] = v[1];
    } else {
        d[0] = s[0];
    }
}
template <int N>
__device__ __forceinline__ void store_vec(float* d, const float* s) {
    if constexpr (N == 4) {
        *reinterpret_cast<f32x4*>(d) = f32x4{s[0], s[1], s[2], s[3]};
    } else if constexpr (N == 2) {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<f32x2*>(d) = f32x2{s[0], s[1]};
    } else {
        d[0] = s[0];
    }
}

// One head row held EPL values a lane (element e0 + j of lane l, e0 = EPL l): RMS-normed
// with the weights w (none: no norm) and rotated; cos_sin(i, &c, &s) gives pair i's angle.
template <int EPL, typename CS>
__device__ __forceinline__ void norm_rope_row(float* xv, bool has_w, const float* w, float eps,
                                              int norm_d, int n_pairs, int neox, int lane,
                                              CS cos_sin) {
    const int e0 = EPL * lane;
    if (has_w) {  // ops::rms_norm (src/ops.rs:13-27) per head
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < EPL; ++j) ss += xv[j] * xv[j];
#pragma unroll
        for (int sh = 32; sh >= 1; sh >>= 1) ss = wave_sum_xor(ss, sh);
        const float inv = 1.0f / sqrtf(ss / (float)norm_d + eps);
#pragma unroll
        for (int j = 0; j < EPL; ++j) xv[j] = (xv[j] * inv) * w[j];
    }
    // ops::apply_rope / apply_rope_with_freqs: pair i is (x0, x1) -> (x0 c - x1 s, x0 s + x1 c)
    if (neox) {
        const int off = n_pairs / EPL;  // lanes between the two elements of a pair
        const int src = lane < off ? lane + off : lane - off;
        float pv[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) pv[j] = __shfl(xv[j], src < 64 ? src : lane, 64);
        if (lane < 2 * off) {
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const bool first = lane < off;
                const int i = first ? e0 + j : e0 + j - n_pairs;
                float c, sn;
                cos_sin(i, &c, &sn);
                xv[j] = first ? xv[j] * c - pv[j] * sn : pv[j] * sn + xv[j] * c;
            }
        }
    } else if constexpr (EPL >= 2) {
#pragma unroll
        for (int j = 0; j < EPL; j += 2) {
            const int i = (e0 + j) >> 1;
            if (i < n_pairs) {
                float c, sn;
                cos_sin(i, &c, &sn);
                const float x0 = xv[j], x1 = xv[j + 1];
                xv[j] = x0 * c - x1 * sn;
                xv[j + 1] = x0 * sn + x1 * c;
            }
        }
    } else {
        const float pv0 = __shfl_xor(xv[0], 1, 64);
        const int i = e0 >> 1;
        if (i < n_pairs) {
            float c, sn;
            cos_sin(i, &c, &sn);
            xv[0] = (lane & 1) ? pv0 * sn + xv[0] * c : xv[0] * c - pv0 * sn;
        }
    }
}

// The K / V side of a prompt launch, one workgroup per (16-position page, K head): the
// K head's rows of the launch's tokens on page lp = floor(start / 16) + j (the launch's
// first and last pages may also hold positions outside it, left alone) are RMS-normed,
// rotated at their positions and written back in f32, and their K and V values go to
// the page's blocks through LDS as whole 16-byte chunks.  Per token, K's values lie in
// 16-byte chunks 256 bytes apart and V's are single elements 32 bytes apart, which as
// per-token writes cost a prompt a quarter of its prologue.  pw = workgroup index
// among the page workgroups, ppn = pages a sequence's launch can touch.  The blocks and
// the cos / sin table live in the launch's dynamic LDS (prologue_page_lds bytes).
extern __shared__ __attribute__((aligned(16))) unsigned char pi_prologue_dyn[];
template <typename PT, int EPL>
__device__ __forceinline__ void prologue_page(float* __restrict__ k, const float* __restrict__ v,
                                              const float* __restrict__ kn, float eps,
                                              const RopeFreqs& f, int n_pairs, int neox,
                                              const KvGeom& g, const int32_t* __restrict__ pt,
                                              int max_pages, const PrologueStart& start_pos,
                                              int n_tok, int norm_d, int pw, int ppn) {
    constexpr int D = 64 * EPL;
    constexpr int E = 16 / (int)sizeof(PT);  // pool values per 16-byte chunk
    typedef PT pv __attribute__((ext_vector_type(E)));
    // K and V rows staged by slot, [16][KP] with a 16-byte pad a row: a row's values are
    // written contiguously, and the block writes below read a K chunk (E dims of one slot)
    // as one 16-byte read and a V chunk (E slots of one dim) as E reads, 16 rows spread
    // over the banks by the pad.  (Staging in the pool's block layouts made each 2-byte
    // write land on one or two banks across the wavefront.)
    constexpr int KP = D + E;
    PT* kb_s = reinterpret_cast<PT*>(pi_prologue_dyn);
    PT* vb_s = kb_s + kPageTokens * KP;
    float* cs_c = reinterpret_cast<float*>(vb_s + kPageTokens * KP);  // cos [slot][pair]
    float* cs_n = cs_c + kPageTokens * n_pairs;                       // sin
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int hkv = g.n_kv_heads;
    const int sq = pw / (ppn * hkv), rem = pw % (ppn * hkv);
    const int j = rem / hkv, h = rem % hkv;
    const int start = start_pos.of(sq);
    const int p0 = start >= 0 ? start / kPageTokens : -((kPageTokens - 1 - start) / kPageTokens);
    const int lp = p0 + j, pa = lp * kPageTokens;
    const int t0 = max(start, pa), t1 = min(start + n_tok, pa + kPageTokens);
    if (t0 >= t1) return;  // uniform: no position of the launch on this page
    const int s0 = t0 - pa, s1 = t1 - pa;  // the launch's slots [s0, s1)
    const int page = lp >= 0 && lp < max_pages ? pt[(size_t)sq * max_pages + lp] : -1;
    const bool app = page >= 0 && page < g.n_pages;  // uniform
    const int e0 = EPL * lane;
    // this wavefront's slots s0 + wv + 4 m: the rows and the norm weights first
    float xs[4][EPL], vs[4][EPL], kw[EPL];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int sl = s0 + wv + 4 * m;
        if (sl < s1) {
            const size_t row = (((size_t)sq * n_tok + (pa + sl - start)) * hkv + h) * D + e0;
            load_vec<EPL>(xs[m], k + row);
            load_vec<EPL>(vs[m], v + row);
        }
    }
    if (kn) load_vec<EPL>(kw, kn + e0);
    for (int i = threadIdx.x; i < (s1 - s0) * n_pairs; i += 256) {
        const int sl = s0 + i / n_pairs, pr = i % n_pairs;
        const float theta = (float)(pa + sl) * f.f[pr];
        cs_c[sl * n_pairs + pr] = cosf(theta);
        cs_n[sl * n_pairs + pr] = sinf(theta);
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int sl = s0 + wv + 4 * m;
        if (sl >= s1) break;
        float* xv = xs[m];
        norm_rope_row<EPL>(xv, kn != nullptr, kw, eps, norm_d, n_pairs, neox, lane,
                           [&](int i, float* c, float* sn) {
                               *c = cs_c[sl * n_pairs + i];
                               *sn = cs_n[sl * n_pairs + i];
                           });
        store_vec<EPL>(k + (((size_t)sq * n_tok + (pa + sl - start)) * hkv + h) * D + e0, xv);
        if (app) {
#pragma unroll
            for (int jj = 0; jj < EPL; ++jj) {
                kb_s[sl * KP + e0 + jj] = from_f32<PT>(xv[jj]);
                vb_s[sl * KP + e0 + jj] = from_f32<PT>(vs[m][jj]);
            }
        }
    }
    if (!app) return;  // uniform
    __syncthreads();
    const size_t blk = (size_t)page * hkv + h;
    PT* kp = reinterpret_cast<PT*>(static_cast<char*>(g.k) + blk * g.kstride);
    PT* vp = reinterpret_cast<PT*>(static_cast<char*>(g.v) + blk * g.vstride);
    // K block [D / E][16][E]: chunk c = (dims E (c / 16) .., slot c % 16)
    for (int c = threadIdx.x; c < D / E * kPageTokens; c += 256) {
        const int slot = c % kPageTokens;
        if (slot >= s0 && slot < s1)
            *reinterpret_cast<pv*>(kp + (size_t)E * c) = *reinterpret_cast<const pv*>(kb_s + slot * KP + E * (c / kPageTokens));
    }
    // V block [D][16]: chunk c = (dim c / (16 / E), slots E (c % (16 / E)) ..)
    constexpr int CPR = kPageTokens / E;  // chunks per dim row
    for (int c = threadIdx.x; c < D * CPR; c += 256) {
        const int sl0 = E * (c % CPR), dim = c / CPR;
        if (sl0 + E <= s0 || sl0 >= s1) continue;
        if (sl0 >= s0 && sl0 + E <= s1) {
            pv t;
#pragma unroll
            for (int e = 0; e < E; ++e) t[e] = vb_s[(sl0 + e) * KP + dim];
            *reinterpret_cast<pv*>(vp + (size_t)E * c) = t;
        } else {  // a chunk the launch covers in part: its own slots only
            for (int e = 0; e < E; ++e)
                if (sl0 + e >= s0 && sl0 + e < s1) vp[(size_t)E * c + e] = vb_s[(sl0 + e) * KP + dim];
        }
    }
}

template <typename PT, int EPL>
__global__ __launch_bounds__(256) void attn_prologue_vec_kernel(
    float* __restrict__ q, float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ qn, const float* __restrict__ kn, float eps, RopeFreqs f,
    int n_pairs, int neox, KvGeom g, const int32_t* __restrict__ pt, int max_pages,
    PrologueStart start_pos, int n_seq, int n_tok, int hq, int norm_d, int ppn) {
    constexpr int D = 64 * EPL;
    __shared__ float cs_s[2][128];  // cos, sin of pair i at this token's position
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    // ppn > 0: the first n_seq * ppn * n_kv_heads workgroups take the K / V side by page
    // (dispatched first, so they run beside the token workgroups), and the token workgroups
    // after them only the q heads
    const int toks = n_seq * n_tok;
    const int n_pg = ppn > 0 ? n_seq * ppn * g.n_kv_heads : 0;
    if ((int)blockIdx.x < n_pg) {
        if (blockIdx.y == 0)  // launches that split the token's heads over y: one copy
            prologue_page<PT, EPL>(k, v, kn, eps, f, n_pairs, neox, g, pt, max_pages, start_pos,
                                   n_tok, norm_d, (int)blockIdx.x, ppn);
        return;
    }
    const int hkv = g.n_kv_heads, heads = ppn > 0 ? hq : hq + hkv;
    const bool table = gridDim.y == 1;  // uniform per launch: the token remap below
    // A prompt launch keeps each run of 16 consecutive tokens (a page of K and V when
    // the prompt starts on a page) on one XCD: workgroups are dispatched round-robin
    // over the 8 XCDs, and workgroup 8 (16 g + i) + x takes token 128 g + 16 x + i, so
    // the partial-line writes of the page's 2-byte K / V values merge in that XCD's L2
    // instead of reaching HBM from eight caches.
    int u = (int)blockIdx.x - n_pg;
    if (table && u < toks / 128 * 128) {
        const int x = u & 7, m = u >> 3;
        u = (m >> 4) * 128 + x * 16 + (m & 15);
    }
    const int t = u % n_tok, sq = u / n_tok;
    const int pos = start_pos.of(sq) + t;
    start_pos.write_ctx();
    // cos / sin of the workgroup's token position, once per pair (every thread of the
    // workgroup works on that token)
    for (int i = threadIdx.x; i < n_pairs; i += 256) {
        const float theta = (float)pos * f.f[i];
        cs_s[0][i] = cosf(theta);
        cs_s[1][i] = sinf(theta);
    }
    __syncthreads();
    auto cos_sin = [&](int i, float* c, float* sn) {
        *c = cs_s[0][i];
        *sn = cs_s[1][i];
    };
    const int e0 = EPL * lane;  // this lane's first element of a row
    const int per = (heads + gridDim.y - 1) / gridDim.y;
    const int h1 = min(heads, (int)(blockIdx.y + 1) * per);
    auto row_of = [&](int head) {
        return head < hq ? q + (((size_t)sq * n_tok + t) * hq + head) * D
                         : k + (((size_t)sq * n_tok + t) * hkv + (head - hq)) * D;
    };
    // A wavefront's heads are head0, head0 + 4, ...: the rows of up to MH of them (and the V
    // rows of its K heads) are loaded before any is processed, so their loads overlap.
    constexpr int MH = 6;
    // the norm weights (the same for every row of a kind) are read once, beside the rows
    float qw[EPL], kw[EPL];
    bool wl = false;
    for (int head0 = blockIdx.y * per + wv; head0 < h1; head0 += 4 * MH) {
        float xs[MH][EPL], vs[MH][EPL];
#pragma unroll
        for (int m = 0; m < MH; ++m) {
            const int head = head0 + 4 * m;
            if (head < h1) {
                load_vec<EPL>(xs[m], row_of(head) + e0);
                if (head >= hq) load_vec<EPL>(vs[m], v + (((size_t)sq * n_tok + t) * hkv + (head - hq)) * D + e0);
            }
        }
        if (!wl) {
            if (qn) load_vec<EPL>(qw, qn + e0);
            if (kn) load_vec<EPL>(kw, kn + e0);
            wl = true;
        }
#pragma unroll
        for (int m = 0; m < MH; ++m) {
            const int head = head0 + 4 * m;
            if (head >= h1) break;
            const bool is_q = head < hq;
            const int kvh = head - hq;
            float* x = row_of(head);
            float* xv = xs[m];
            norm_rope_row<EPL>(xv, is_q ? qn != nullptr : kn != nullptr, is_q ? qw : kw, eps, norm_d,
                               n_pairs, neox, lane, cos_sin);
            store_vec<EPL>(x + e0, xv);
            // append-then-attend (src/model/mod.rs:1140-1146): K (normed, rotated) and V at pos
            const int lp = pos / kPageTokens;
            if (!is_q && pos >= 0 && lp < max_pages) {
                const int page = pt[(size_t)sq * max_pages + lp];
                if (page >= 0 && page < g.n_pages) {
                    const int tok = pos % kPageTokens;
                    const size_t blk = (size_t)page * hkv + kvh;
                    PT* kp = reinterpret_cast<PT*>(static_cast<char*>(g.k) + blk * g.kstride);
                    PT* vp = reinterpret_cast<PT*>(static_cast<char*>(g.v) + blk * g.vstride);
                    const float* vr = vs[m];
#pragma unroll
                    for (int j = 0; j < EPL; ++j) {
                        kp[k_index<PT>(tok, e0 + j)] = from_f32<PT>(xv[j]);
                        vp[v_index(tok, e0 + j)] = from_f32<PT>(vr[j]);
                    }
                }
            }
        }
    }
}

int grid_for(size_t total) {
    size_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) blocks = 1;
    return (int)blocks;
}

template <typename ST>
hipError_t append_src(const KvGeom& g, const void* k, const void* v, const int32_t* pt,
                      int32_t max_pages, const int32_t* sp, int32_t n_seq, int32_t n_tok,
                      hipStream_t s) {
    const size_t total = (size_t)n_seq * n_tok * g.n_kv_heads * g.head_dim;
    const ST* ks = reinterpret_cast<const ST*>(k);
    const ST* vs = reinterpret_cast<const ST*>(v);
    const long long ppn = (n_tok + kPageTokens - 1) / kPageTokens + 1;  // pages one sequence can touch
    if ((long long)n_seq * ppn <= 0x7fffffffLL && g.n_kv_heads <= 65535) {
        const dim3 grid((unsigned)(n_seq * ppn), (unsigned)g.n_kv_heads);
        if (g.dtype == 1)
            hipLaunchKernelGGL((kv_append_page_kernel<ST, f16>), grid, dim3(256), 0, s, g, ks, vs, pt,
                               max_pages, sp, n_tok, (int)ppn);
        else
            hipLaunchKernelGGL((kv_append_page_kernel<ST, float>), grid, dim3(256), 0, s, g, ks, vs, pt,
                               max_pages, sp, n_tok, (int)ppn);
        return hipGetLastError();
    }
    if (g.dtype == 1)
        hipLaunchKernelGGL((kv_append_kernel<ST, f16>), dim3(grid_for(total)), dim3(256), 0, s, g,
                           ks, vs, pt, max_pages, sp, n_seq, n_tok);
    else
        hipLaunchKernelGGL((kv_append_kernel<ST, float>), dim3(grid_for(total)), dim3(256), 0, s,
                           g, ks, vs, pt, max_pages, sp, n_seq, n_tok);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_kv_append(const KvGeom& g, const void* k, const void* v, int32_t src_dtype,
                            const int32_t* page_table, int32_t max_pages,
                            const int32_t* start_pos, int32_t n_seq, int32_t n_tok,
                            hipStream_t s) {
    switch (src_dtype) {
        case 0: return append_src<float>(g, k, v, page_table, max_pages, start_pos, n_seq, n_tok, s);
        case 1: return append_src<f16>(g, k, v, page_table, max_pages, start_pos, n_seq, n_tok, s);
        case 2: return append_src<bf16>(g, k, v, page_table, max_pages, start_pos, n_seq, n_tok, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_kv_read(const KvGeom& g, const int32_t* page_table, int32_t max_pages,
                          int32_t seq, int32_t start, int32_t n_tok, float* k_out, float* v_out,
                          hipStream_t s) {
    const size_t total = (size_t)n_tok * g.n_kv_heads * g.head_dim;
    if (g.dtype == 1)
        hipLaunchKernelGGL((kv_read_kernel<f16>), dim3(grid_for(total)), dim3(256), 0, s, g,
                           page_table, max_pages, seq, start, n_tok, k_out, v_out);
    else
        hipLaunchKernelGGL((kv_read_kernel<float>), dim3(grid_for(total)), dim3(256), 0, s, g,
                           page_table, max_pages, seq, start, n_tok, k_out, v_out);
    return hipGetLastError();
}

namespace {
// PI_PROLOGUE_VEC=0 keeps every launch on the LDS-staged attn_prologue_kernel (read per call).
bool use_vec_prologue() {
    const char* e = std::getenv("PI_PROLOGUE_VEC");
    return !(e && e[0] == '0');
}
}  // namespace

hipError_t launch_attn_prologue(float* q, float* k, const float* v, const float* q_norm_w,
                                const float* k_norm_w, float eps, const RopeFreqs& freqs,
                                int32_t n_pairs, int32_t neox, const KvGeom& g,
                                const int32_t* page_table, int32_t max_pages,
                                const int32_t* start_pos, int32_t n_seq, int32_t n_tok,
                                int32_t n_q_heads, hipStream_t s, int32_t start_scalar,
                                int32_t* ctx_out, int32_t n_ctx, int32_t norm_dim) {
    if (!start_pos && n_seq != 1) return hipErrorInvalidValue;
    const int norm_d = norm_dim > 0 ? norm_dim : g.head_dim;
    if (norm_d > g.head_dim) return hipErrorInvalidValue;
    const PrologueStart sp{start_pos, start_scalar, ctx_out, ctx_out ? n_ctx : 0, 0};
    const long long toks = (long long)n_seq * n_tok;
    if (toks <= 0) return hipSuccess;
    if (toks > 0x7fffffffLL || n_pairs > 128) return hipErrorInvalidValue;
    const int heads = n_q_heads + g.n_kv_heads;
    const dim3 grid((unsigned)toks, toks >= 1024 ? 1u : (unsigned)((heads + 3) / 4));
    const int epl = g.head_dim / 64;
    // vector accesses of EPL floats need rows aligned to EPL * 4 bytes
    const uintptr_t amask = (uintptr_t)(4 * (epl > 0 ? epl : 1) - 1);
    const bool aligned = (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)q_norm_w |
                           (uintptr_t)k_norm_w) & amask) == 0;
    if ((g.head_dim == 64 || g.head_dim == 128 || g.head_dim == 256) && (!neox || n_pairs % epl == 0) &&
        2 * n_pairs <= g.head_dim && aligned && use_vec_prologue()) {
        // A launch of 16+ tokens a sequence takes the K / V side by page: one more workgroup
        // per (page a sequence's launch can touch, K head), the token workgroups keeping the
        // q heads.
        const bool by_page = n_tok >= kPageTokens;
        const int ppn = by_page ? (n_tok + kPageTokens - 1) / kPageTokens + 1 : 0;
        const long long n_pg = by_page ? (long long)n_seq * ppn * g.n_kv_heads : 0;
        if (toks + n_pg > 0x7fffffffLL) return hipErrorInvalidValue;
        const dim3 grid_v((unsigned)(toks + n_pg), grid.y);
        PrologueStart spv = sp;
        spv.wg0 = (int32_t)n_pg;
        // the page workgroups' staged K and V rows and cos / sin table
        const size_t lds = by_page ? (size_t)2 * kPageTokens * (g.head_dim * (g.dtype == 1 ? 2 : 4) + 16) +
                                         (size_t)2 * kPageTokens * n_pairs * sizeof(float)
                                   : 0;
#define PI_PROLOGUE_VEC(PT, E)                                                                       \
    hipLaunchKernelGGL((attn_prologue_vec_kernel<PT, E>), grid_v, dim3(256), lds, s, q, k, v,       \
                       q_norm_w, k_norm_w, eps, freqs, n_pairs, neox, g, page_table, max_pages, spv, \
                       n_seq, n_tok, n_q_heads, norm_d, ppn)
        const bool hp = g.dtype == 1;
        switch (epl) {
            case 1: if (hp) PI_PROLOGUE_VEC(f16, 1); else PI_PROLOGUE_VEC(float, 1); break;
            case 2: if (hp) PI_PROLOGUE_VEC(f16, 2); else PI_PROLOGUE_VEC(float, 2); break;
            default: if (hp) PI_PROLOGUE_VEC(f16, 4); else PI_PROLOGUE_VEC(float, 4); break;
        }
#undef PI_PROLOGUE_VEC
        return hipGetLastError();
    }
    if (g.dtype == 1)
        hipLaunchKernelGGL(attn_prologue_kernel<f16>, grid, dim3(256), 0, s, q, k, v, q_norm_w,
                           k_norm_w, eps, freqs, n_pairs, neox, g, page_table, max_pages,
                           sp, n_seq, n_tok, n_q_heads, norm_d);
    else
        hipLaunchKernelGGL(attn_prologue_kernel<float>, grid, dim3(256), 0, s, q, k, v, q_norm_w,
                           k_norm_w, eps, freqs, n_pairs, neox, g, page_table, max_pages,
                           sp, n_seq, n_tok, n_q_heads, norm_d);
    return hipGetLastError();
}

hipError_t launch_rope(float* q, float* k, const int32_t* pos, int32_t n_tok, int32_t n_q_heads,
                       int32_t n_kv_heads, int32_t head_dim, int32_t n_pairs, int32_t neox,
                       const RopeFreqs& freqs, hipStream_t s) {
    const size_t total = (size_t)n_tok * (n_q_heads + (k ? n_kv_heads : 0)) * n_pairs;
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(total)), dim3(256), 0, s, q, k, pos, n_tok,
                       n_q_heads, n_kv_heads, head_dim, n_pairs, neox, freqs);
    return hipGetLastError();
}

// Zeros written by a kernel (a memset node must not sit in a captured graph).
__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        dst[i] = 0.f;
}

// Row (t, r) of an n_tok x n_rows grid: `width` floats from src + t * s_tok + r * s_row
// to dst + t * d_tok + r * d_row, then zeros out to `pad` floats.  One wave per row.
template <typename E>
__global__ __launch_bounds__(256) void pack_rows_kernel(E* __restrict__ dst,
                                                        const E* __restrict__ src, long long n,
                                                        int n_rows, int width, int pad,
                                                        long long s_tok, long long s_row,
                                                        long long d_tok, long long d_row) {
    const int lane = threadIdx.x & 63;
    for (long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6); row < n;
         row += (long long)gridDim.x * 4) {
        const long long t = row / n_rows;
        const long long r = row - t * n_rows;
        const E* sp = src + t * s_tok + r * s_row;
        E* dp = dst + t * d_tok + r * d_row;
        for (int c = lane; c < pad; c += 64) dp[c] = c < width ? sp[c] : E(0);
    }
}

// dst[i] = first + i for i < n (device-side positions and context lengths, so a
// layer step issues no host copies).
__global__ __launch_bounds__(256) void fill_iota_kernel(int32_t* __restrict__ dst, int n,
                                                        int first) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = first + i;
}

// out *= sigmoid(gate) (src/model/mod.rs:1192-1196)
__global__ __launch_bounds__(256) void apply_gate_kernel(float* __restrict__ out,
                                                         const float* __restrict__ gate, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] *= 1.0f / (1.0f + expf(-gate[i]));
}

static unsigned grid_1d(size_t n) {
    const size_t b = (n + 255) / 256;
    return (unsigned)(b > 65536 ? 65536 : (b == 0 ? 1 : b));
}

hipError_t launch_fill_zero(float* dst, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_1d(n)), dim3(256), 0, s, dst, n);
    return hipGetLastError();
}

template <typename E>
static hipError_t pack_rows(E* dst, const E* src, int32_t n_tok, int32_t n_rows, int32_t width,
                            int32_t pad, size_t s_tok, size_t s_row, size_t d_tok, size_t d_row,
                            hipStream_t s) {
    const long long n = (long long)n_tok * n_rows;
    if (n <= 0 || pad <= 0) return hipSuccess;
    if (width < 0 || width > pad) return hipErrorInvalidValue;
    const long long blocks = (n + 3) / 4;
    hipLaunchKernelGGL(pack_rows_kernel<E>, dim3((unsigned)(blocks > 65536 ? 65536 : blocks)), dim3(256), 0,
                       s, dst, src, n, n_rows, width, pad, (long long)s_tok, (long long)s_row,
                       (long long)d_tok, (long long)d_row);
    return hipGetLastError();
}

hipError_t launch_pack_rows(float* dst, const float* src, int32_t n_tok, int32_t n_rows,
                           int32_t width, int32_t pad, size_t s_tok, size_t s_row, size_t d_tok,
                           size_t d_row, hipStream_t s) {
    return pack_rows(dst, src, n_tok, n_rows, width, pad, s_tok, s_row, d_tok, d_row, s);
}

hipError_t launch_pack_rows16(uint16_t* dst, const uint16_t* src, int32_t n_tok, int32_t n_rows,
                             int32_t width, int32_t pad, size_t s_tok, size_t s_row, size_t d_tok,
                             size_t d_row, hipStream_t s) {
    return pack_rows(dst, src, n_tok, n_rows, width, pad, s_tok, s_row, d_tok, d_row, s);
}

hipError_t launch_fill_iota(int32_t* dst, int32_t n, int32_t first, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_iota_kernel, dim3((n + 255) / 256), dim3(256), 0, s, dst, n, first);
    return hipGetLastError();
}

hipError_t launch_apply_gate(float* out, const float* gate, size_t n, hipStream_t s) {
    hipLaunchKernelGGL(apply_gate_kernel, dim3(grid_1d(n)), dim3(256), 0, s, out, gate, n);
    return hipGetLastError();
}

hipError_t launch_softmax(float* x, int32_t n, hipStream_t s) {
    hipLaunchKernelGGL(softmax_row_kernel, dim3(1), dim3(1024), 0, s, x, n);
    return hipGetLastError();
}

hipError_t launch_head_rmsnorm(float* x, const float* w, int32_t n_rows, int32_t dim,
                               int32_t row_stride, float eps, hipStream_t s) {
    hipLaunchKernelGGL(head_rmsnorm_kernel, dim3((n_rows + 3) / 4), dim3(256), 0, s, x, w, n_rows,
                       dim, row_stride, eps);
    return hipGetLastError();
}

}  // namespace pi

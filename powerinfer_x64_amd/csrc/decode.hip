// decode.hip -- split-K flash-decoding attention over the paged KV pool (gfx950).
//
// Replaces the decode attention core of PowerInfer_x64
// (src/model/mod.rs:1148-1190): for every query head, softmax(q.K^T * scale)
// over the sequence's cached keys, weighted sum of V, then the optional
// sigmoid gate (:1192-1196).
//
// Work decomposition: one workgroup (4 wavefronts) per (sequence, KV head,
// split of `pps` pages).  All query heads that share the KV head (up to 16)
// ride in the N dimension of the MFMA tiles, so every K/V byte is read from
// HBM exactly once.  Per 16-token page a wavefront computes
//   S^T[16 tok x 16 heads] = K[16 x D] . Q^T[D x 16]      (QK^T)
//   O^T[D x 16]           += V^T[D x 16 tok] . P^T[16 x 16] (PV)
// with f16 MFMA (f16 pool) or f32 MFMA (f32 pool); softmax statistics stay in
// f32.  The page layouts (pi_launch.hpp) make each MFMA operand one linear
// load per lane.  The 4 wavefronts interleave pages, merge their (max, sum, O)
// in LDS, and the last workgroup of a (sequence, KV head) to finish merges the
// splits from the workspace, so a decode step is a single launch.
#include "pi_device.hpp"
#include "pi_launch.hpp"

#include <algorithm>
#include <cstdlib>

namespace pi {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxGD = 2048;  // G * D limit of the LDS merge buffer

template <typename KT, int D>
struct Tile;

// f16 pool: K chunk = 8 halfs (16 B), QK^T with 16x16x32 f16, PV with 16x16x16 f16.
template <int D>
struct Tile<f16, D> {
    static constexpr int NK = D / 32;  // K loads (16 B) per lane per page
    static constexpr int NV = D / 16;  // V loads (8 B) per lane per page
    f16x8 k[NK];
    f16x4 v[NV];
    struct Q {
        f16x8 r[NK];
    };

    __device__ __forceinline__ void load(const f16* kb, const f16* vb, int lane) {
        const f16x8* k8 = reinterpret_cast<const f16x8*>(kb);
#pragma unroll
        for (int j = 0; j < NK; ++j) k[j] = k8[j * 64 + lane];
        const int col = lane & 15, grp = lane >> 4;
#pragma unroll
        for (int t = 0; t < NV; ++t)
            v[t] = *reinterpret_cast<const f16x4*>(vb + (16 * t + col) * 16 + 4 * grp);
    }
    static __device__ __forceinline__ void load_q(Q& q, const float* qrow, float qs, bool on,
                                                  int grp) {
#pragma unroll
        for (int j = 0; j < NK; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                q.r[j][i] = on ? to_f16(qrow[32 * j + 8 * grp + i] * qs) : (f16)0.0f;
    }
    __device__ __forceinline__ f32x4 scores(const Q& q) const {
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NK; ++j) s = __builtin_amdgcn_mfma_f32_16x16x32_f16(k[j], q.r[j], s, 0, 0, 0);
        return s;
    }
    __device__ __forceinline__ void mask_v(int valid_from_grp) {
        // zero V rows of tokens >= valid (their weight is 0, but pool slack may hold NaN)
#pragma unroll
        for (int t = 0; t < NV; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i >= valid_from_grp) v[t][i] = (f16)0.0f;
    }
    __device__ __forceinline__ void pv(f32x4* o, const float p[4]) const {
        f16x4 pb = {to_f16(p[0]), to_f16(p[1]), to_f16(p[2]), to_f16(p[3])};
#pragma unroll
        for (int t = 0; t < NV; ++t) o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(v[t], pb, o[t], 0, 0, 0);
    }
};

// f32 pool: K chunk = 4 floats (16 B), QK^T and PV with 16x16x4 f32.
template <int D>
struct Tile<float, D> {
    static constexpr int NK = D / 16;
    static constexpr int NV = D / 16;
    f32x4 k[NK];
    f32x4 v[NV];
    struct Q {
        float r[D / 4];
    };

    __device__ __forceinline__ void load(const float* kb, const float* vb, int lane) {
        const f32x4* k4 = reinterpret_cast<const f32x4*>(kb);
#pragma unroll
        for (int j = 0; j < NK; ++j) k[j] = k4[j * 64 + lane];
        const int col = lane & 15, grp = lane >> 4;
#pragma unroll
        for (int t = 0; t < NV; ++t)
            v[t] = *reinterpret_cast<const f32x4*>(vb + (16 * t + col) * 16 + 4 * grp);
    }
    static __device__ __forceinline__ void load_q(Q& q, const float* qrow, float qs, bool on,
                                                  int grp) {
#pragma unroll
        for (int j = 0; j < NK; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) q.r[4 * j + e] = on ? qrow[16 * j + 4 * grp + e] * qs : 0.f;
    }
    __device__ __forceinline__ f32x4 scores(const Q& q) const {
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NK; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                s = __builtin_amdgcn_mfma_f32_16x16x4f32(k[j][e], q.r[4 * j + e], s, 0, 0, 0);
        return s;
    }
    __device__ __forceinline__ void mask_v(int valid_from_grp) {
#pragma unroll
        for (int t = 0; t < NV; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i >= valid_from_grp) v[t][i] = 0.f;
    }
    __device__ __forceinline__ void pv(f32x4* o, const float p[4]) const {
#pragma unroll
        for (int t = 0; t < NV; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[t][r], p[r], o[t], 0, 0, 0);
    }
};

__device__ __forceinline__ int head_of(int kvh, int col, int n_kv, int group, int mode) {
    return mode == 0 ? kvh + col * n_kv : kvh * group + col;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

template <typename KT, int D>
__global__ __launch_bounds__(kThreads) void decode_kernel(KvGeom g, DecodeParams p,
                                                          DecodeWorkspace ws, int pps,
                                                          int n_splits, int group) {
    using T = Tile<KT, D>;
    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int n_kv = g.n_kv_heads;
    const int tid = threadIdx.x;
    const int L = p.ctx_len[b];
    const int n_pages_b = (L + kPageTokens - 1) / kPageTokens;
    const int n_active = (n_pages_b + pps - 1) / pps;
    const int GD = group * D;

    if (n_active == 0) {  // empty context: softmax over nothing leaves zeros (src/ops.rs:161)
        if (split == 0)
            for (int idx = tid; idx < GD; idx += kThreads) {
                int c = idx / D, d = idx - c * D;
                int h = head_of(kvh, c, n_kv, group, p.gqa_mode);
                p.out[((size_t)b * p.n_q_heads + h) * D + d] = 0.f;
            }
        return;
    }
    if (split >= n_active) return;

    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const bool col_on = col < group;
    const int head = head_of(kvh, col_on ? col : 0, n_kv, group, p.gqa_mode);

    typename T::Q q;
    T::load_q(q, p.q + ((size_t)b * p.n_q_heads + head) * D, p.scale * kLog2e, col_on, grp);

    f32x4 o[D / 16];
#pragma unroll
    for (int t = 0; t < D / 16; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -1e30f, l_run = 0.f;

    const int page_begin = split * pps;
    const int page_end = min(page_begin + pps, n_pages_b);
    const int32_t* pt = p.page_table + (size_t)b * p.max_pages;
    const size_t blk = (size_t)kPageTokens * D;
    const KT* kpool = reinterpret_cast<const KT*>(g.k);
    const KT* vpool = reinterpret_cast<const KT*>(g.v);

    T cur, nxt;
    int pg = page_begin + wave;
    if (pg < page_end) {
        size_t off = ((size_t)pt[pg] * n_kv + kvh) * blk;
        cur.load(kpool + off, vpool + off, lane);
    }
    for (; pg < page_end; pg += kWaves) {
        const int pn = pg + kWaves;
        if (pn < page_end) {
            size_t off = ((size_t)pt[pn] * n_kv + kvh) * blk;
            nxt.load(kpool + off, vpool + off, lane);
        }
        f32x4 s = cur.scores(q);
        const int valid = L - pg * kPageTokens;  // tokens of this page inside the context
        if (valid < kPageTokens) {
            const int vg = valid - 4 * grp;  // valid tokens among this lane's 4
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (r >= vg) s[r] = -INFINITY;
            cur.mask_v(vg);
        }
        float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        mx = wave_max_xor(mx, 16);
        mx = wave_max_xor(mx, 32);
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - m_new);
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(s[r] - m_new);
        l_run = l_run * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
        m_run = m_new;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) o[t] *= alpha;
        cur.pv(o, pr);
        if (pn < page_end) cur = nxt;
    }
    l_run = wave_sum_xor(l_run, 16);
    l_run = wave_sum_xor(l_run, 32);

    // ---- merge the 4 wavefronts in LDS ----
    __shared__ float s_m[kWaves][16];
    __shared__ float s_l[kWaves][16];
    __shared__ __attribute__((aligned(16))) float s_o[kWaves][kMaxGD];
    if (col_on) {
#pragma unroll
        for (int t = 0; t < D / 16; ++t)
            *reinterpret_cast<f32x4*>(&s_o[wave][col * D + 16 * t + 4 * grp]) = o[t];
        if (grp == 0) {
            s_m[wave][col] = m_run;
            s_l[wave][col] = l_run;
        }
    }
    __syncthreads();

    const size_t bk = (size_t)b * n_kv + kvh;
    if (n_active == 1) {
        for (int idx = tid; idx < GD; idx += kThreads) {
            const int c = idx / D, d = idx - c * D;
            float M = s_m[0][c];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][c]);
            float acc = 0.f, lsum = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float f = fast_exp2(s_m[w][c] - M);
                acc += f * s_o[w][idx];
                lsum += f * s_l[w][c];
            }
            const int h = head_of(kvh, c, n_kv, group, p.gqa_mode);
            const size_t oi = ((size_t)b * p.n_q_heads + h) * D + d;
            float r = acc / lsum;
            if (p.gate) r *= sigmoidf_(p.gate[oi]);
            p.out[oi] = r;
        }
        return;
    }

    float* po = ws.partial_o + (bk * n_splits + split) * GD;
    float* pml = ws.partial_ml + (bk * n_splits + split) * group * 2;
    for (int idx = tid; idx < GD; idx += kThreads) {
        const int c = idx / D, d = idx - c * D;
        float M = s_m[0][c];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][c]);
        float acc = 0.f, lsum = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float f = fast_exp2(s_m[w][c] - M);
            acc += f * s_o[w][idx];
            lsum += f * s_l[w][c];
        }
        po[idx] = acc;
        if (d == 0) {
            pml[2 * c] = M;
            pml[2 * c + 1] = lsum;
        }
    }

    // ---- last workgroup of this (sequence, KV head) merges the splits ----
    __shared__ int s_last;
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned prev = __hip_atomic_fetch_add(ws.counters + bk, 1u, __ATOMIC_ACQ_REL,
                                               __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (unsigned)(n_active - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    const float* po0 = ws.partial_o + bk * n_splits * GD;
    const float* pml0 = ws.partial_ml + bk * n_splits * group * 2;
    for (int idx = tid; idx < GD; idx += kThreads) {
        const int c = idx / D, d = idx - c * D;
        float M = -1e30f;
        for (int s = 0; s < n_active; ++s) M = fmaxf(M, __builtin_nontemporal_load(&pml0[(s * group + c) * 2]));
        float acc = 0.f, lsum = 0.f;
        for (int s = 0; s < n_active; ++s) {
            const float ms = __builtin_nontemporal_load(&pml0[(s * group + c) * 2]);
            const float ls = __builtin_nontemporal_load(&pml0[(s * group + c) * 2 + 1]);
            const float f = fast_exp2(ms - M);
            acc += f * __builtin_nontemporal_load(&po0[(size_t)s * GD + idx]);
            lsum += f * ls;
        }
        const int h = head_of(kvh, c, n_kv, group, p.gqa_mode);
        const size_t oi = ((size_t)b * p.n_q_heads + h) * D + d;
        float r = acc / lsum;
        if (p.gate) r *= sigmoidf_(p.gate[oi]);
        p.out[oi] = r;
    }
    if (tid == 0) __hip_atomic_store(ws.counters + bk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename KT, int D>
hipError_t launch_t(const KvGeom& g, const DecodeParams& p, const DecodeWorkspace& ws, int pps,
                    int n_splits, hipStream_t s) {
    const int group = p.n_q_heads / g.n_kv_heads;
    dim3 grid(n_splits, g.n_kv_heads, p.batch);
    hipLaunchKernelGGL((decode_kernel<KT, D>), grid, dim3(kThreads), 0, s, g, p, ws, pps, n_splits,
                       group);
    return hipGetLastError();
}

}  // namespace

void decode_plan(const KvGeom& g, int32_t batch, int32_t max_pages, int32_t* pages_per_split,
                 int32_t* n_splits) {
    // Aim for ~8k workgroups over the table's upper bound so that ragged
    // batches still leave many active workgroups per CU (256 CUs).
    long long total = (long long)batch * g.n_kv_heads * max_pages;
    int pps = 4;
    while (pps < 256 && total / pps > 8192) pps *= 2;
    if (const char* e = std::getenv("PI_DECODE_PPS")) {
        int v = std::atoi(e);
        if (v >= 4 && v <= 4096 && (v & (v - 1)) == 0) pps = v;
    }
    *pages_per_split = pps;
    *n_splits = (max_pages + pps - 1) / pps;
}

size_t decode_ws_floats_o(const KvGeom& g, int32_t batch, int32_t n_q_heads, int32_t n_splits) {
    return (size_t)batch * g.n_kv_heads * n_splits * (n_q_heads / g.n_kv_heads) * g.head_dim;
}

hipError_t launch_decode(const KvGeom& g, const DecodeParams& p, const DecodeWorkspace& ws,
                         int32_t pps, int32_t n_splits, hipStream_t s) {
    const bool hp = g.dtype == 1;
    switch (g.head_dim) {
        case 64: return hp ? launch_t<f16, 64>(g, p, ws, pps, n_splits, s) : launch_t<float, 64>(g, p, ws, pps, n_splits, s);
        case 128: return hp ? launch_t<f16, 128>(g, p, ws, pps, n_splits, s) : launch_t<float, 128>(g, p, ws, pps, n_splits, s);
        case 256: return hp ? launch_t<f16, 256>(g, p, ws, pps, n_splits, s) : hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

}  // namespace pi

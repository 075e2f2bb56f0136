// decode.hip -- split-K flash-decoding attention over the paged KV pool (gfx950).
//
// Replaces the decode attention core of PowerInfer_x64
// (src/model/mod.rs:1148-1190): for every query head, softmax(q.K^T * scale)
// over the sequence's cached keys, weighted sum of V, then the optional
// sigmoid gate (:1192-1196).
//
// Work decomposition: a persistent grid of exactly as many workgroups (4
// wavefronts each) as the GPU holds at once.  The launch's work is the list of
// items (16 pages, fewer for small launches) of every (sequence, KV head)
// segment; each workgroup takes an
// equal contiguous range of items, found from a prefix scan of the context
// lengths, so ragged batches are balanced to within one item and no workgroup
// is left idle.  All query heads that share the KV head (up to 16) ride in the
// N dimension of the MFMA tiles, so every K/V byte is read from HBM once.
// Per 16-token page a wavefront computes
//   S^T[16 tok x 16 heads] = K[16 x D] . Q^T[D x 16]      (QK^T)
//   O^T[D x 16]           += V^T[D x 16 tok] . P^T[16 x 16] (PV)
// with f16 MFMA (f16 pool) or f32 MFMA (f32 pool); softmax statistics stay in
// f32.  The page layouts (pi_launch.hpp) make each MFMA operand one linear
// load per lane.
//
// Memory pipeline: within a run the 4 wavefronts interleave pages; a
// wavefront's page ids sit in one VGPR (lane j = j-th page) and are read with
// readlane, so no scalar load sits between two pages.  NP pages are processed
// per iteration while the next NP pages are in flight; the last iteration is
// peeled so the in-loop wait count is exact.  The running softmax max is
// raised lazily: it only moves when a score exceeds it by 2^8, so most pages
// skip the rescale of the accumulators.
//
// The 4 wavefronts merge (max, sum, O) in LDS.  A run that covers its whole
// segment writes the output; otherwise it writes a partial and
// decode_merge_kernel (same stream, next launch) combines the runs -- no
// cross-workgroup synchronisation inside a kernel.
#include "decode_sched.hpp"
#include "pi_device.hpp"
#include "pi_launch.hpp"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <type_traits>

// Fixed scratch of pi_attn_decode_noalloc: the run partials (o, then m and l)
// for callers that cannot allocate device memory.  Each GPU holds one copy
// until the process ends, and every no-alloc call on that GPU shares it.
// Nothing in it needs to start at zero: a slot is written before the merge
// kernel reads it.  Host code never passes this name to a kernel; it uses the
// device address that decode_scratch() looks up.
static __device__ __align__(256) float scratch[pi::kDecodeScratchFloats];

namespace pi {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxGD = 2048;            // G * D limit of the LDS merge buffer
constexpr float kLazyThreshold = 8.0f;  // log2 headroom before the running max moves
constexpr int kMaxRuns = 1024;          // runs of one segment the merge kernel stages
static_assert(kWaves == sched::kWaves && kPageTokens == sched::kPage, "schedule constants");

template <typename KT, int D>
struct Tile;

// f16 pool: K chunk = 8 halfs (16 B), QK^T with 16x16x32 f16, PV with 16x16x16 f16.
template <int D>
struct Tile<f16, D> {
    static constexpr int NK = D / 32;  // K loads (16 B) per lane per page
    static constexpr int NV = D / 16;  // V loads (8 B) per lane per page
    static constexpr int QD = D;  // floats per query row
    static __device__ __forceinline__ void prepare() {}
    f16x8 k[NK];
    f16x4 v[NV];
    struct Q {
        f16x8 r[NK];
    };

    __device__ __forceinline__ void load(const char* kbp, const char* vbp, int lane) {
        const f16* vb = reinterpret_cast<const f16*>(vbp);
        const f16x8* k8 = reinterpret_cast<const f16x8*>(kbp);
#pragma unroll
        for (int j = 0; j < NK; ++j) k[j] = k8[j * 64 + lane];
        const int col = lane & 15, grp = lane >> 4;
#pragma unroll
        for (int t = 0; t < NV; ++t)
            v[t] = *reinterpret_cast<const f16x4*>(vb + (16 * t + col) * 16 + 4 * grp);
    }
    // qrow is always a valid row; `qs` is 0 for padding columns.
    static __device__ __forceinline__ void load_q(Q& q, const float* qrow, float qs, int grp) {
#pragma unroll
        for (int j = 0; j < NK; ++j) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(qrow + 32 * j + 8 * grp);
            const f32x4 b = *reinterpret_cast<const f32x4*>(qrow + 32 * j + 8 * grp + 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                q.r[j][i] = to_f16(a[i] * qs);
                q.r[j][4 + i] = to_f16(b[i] * qs);
            }
        }
    }
    __device__ __forceinline__ f32x4 scores(const Q& q) const {
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NK; ++j) s = __builtin_amdgcn_mfma_f32_16x16x32_f16(k[j], q.r[j], s, 0, 0, 0);
        return s;
    }
    __device__ __forceinline__ void mask_v(int valid) {
        // zero V of tokens >= valid (their weight is 0, but slack slots may hold NaN)
#pragma unroll
        for (int t = 0; t < NV; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i >= valid) v[t][i] = (f16)0.0f;
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
    static constexpr int QD = D;
    static __device__ __forceinline__ void prepare() {}
    f32x4 k[NK];
    f32x4 v[NV];
    struct Q {
        float r[D / 4];
    };

    __device__ __forceinline__ void load(const char* kbp, const char* vbp, int lane) {
        const float* vb = reinterpret_cast<const float*>(vbp);
        const f32x4* k4 = reinterpret_cast<const f32x4*>(kbp);
#pragma unroll
        for (int j = 0; j < NK; ++j) k[j] = k4[j * 64 + lane];
        const int col = lane & 15, grp = lane >> 4;
#pragma unroll
        for (int t = 0; t < NV; ++t)
            v[t] = *reinterpret_cast<const f32x4*>(vb + (16 * t + col) * 16 + 4 * grp);
    }
    static __device__ __forceinline__ void load_q(Q& q, const float* qrow, float qs, int grp) {
#pragma unroll
        for (int j = 0; j < NK; ++j) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(qrow + 16 * j + 4 * grp);
#pragma unroll
            for (int e = 0; e < 4; ++e) q.r[4 * j + e] = a[e] * qs;
        }
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
    __device__ __forceinline__ void mask_v(int valid) {
#pragma unroll
        for (int t = 0; t < NV; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i >= valid) v[t][i] = 0.f;
    }
    __device__ __forceinline__ void pv(f32x4* o, const float p[4]) const {
#pragma unroll
        for (int t = 0; t < NV; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[t][r], p[r], o[t], 0, 0, 0);
    }
};

// TurboQuant pool (src/turboquant/mod.rs:408-566), head_dim D = 128 or 256:
// per (page, KV head) a K block of 16 packed keys (D/2 bytes each: 3-bit
// Lloyd-Max codes of the rotated, sqrt(D)-scaled unit key, LSB first, then D
// QJL sign bits) followed by the 16 f32 key norms, and a V block [D dims][16
// tokens] of f16 values.  The query row is the 2D-wide "virtual query"
// [R.q / sqrt(D) | c * G.R.q / sqrt(D)] (tq_query_kernel), so a key's score is
// norm * <virtual key, virtual query> with the virtual key [centroid(code_i) |
// +-1 sign_i].  The dot runs on v_mfma_f32_16x16x32_f16: the k index of MFMA
// block kb, lane group g, element e is dim (D/4) g + 8 kb + e (kb < D/32) or
// sign (D/4) g + 8 (kb - D/32) + e, so a lane decodes only the D/4 codes
// (3D/128 dwords) and D/4 signs (D/128 dwords) of its quarter of the key.  The
// centroid half of the query is split into f16 hi + lo parts; centroids are
// f16 (relative rounding <= 1.9e-4).
struct TqKey {};
constexpr uint64_t kTqMagF16 =       // f16 bits of 0.2451, 0.756, 1.344, 2.152
    0x33D8ull | (0x3A0Cull << 16) | (0x3D60ull << 32) | (0x404Eull << 48);

// f16 bits of Lloyd-Max centroid `c` (0..7): codes 4..7 are +M[c-4], codes
// 0..3 are -M[3-c] (the 3-bit codebook is symmetric).
__device__ __forceinline__ uint32_t tq_centroid_f16(uint32_t c) {
    const uint32_t k = (c ^ ((c >> 2) - 1u)) & 3u;
    return ((uint32_t)(kTqMagF16 >> (16 * k)) & 0xFFFFu) | ((c & 4u) ? 0u : 0x8000u);
}

// Decoding tables in LDS, built once per workgroup: a pair of 3-bit codes
// (6 bits, first code low) -> its two f16 centroids; a byte of QJL sign bits
// -> eight f16 +-1 values.
struct TqLut {
    uint32_t pair[64];
    f16x8 sign[256];
};
__device__ __forceinline__ TqLut& tq_lut() {
    __shared__ TqLut lut;
    return lut;
}
__device__ __forceinline__ void tq_lut_build() {
    TqLut& L = tq_lut();
    const int t = threadIdx.x;
    if (t < 64) L.pair[t] = tq_centroid_f16(t & 7) | (tq_centroid_f16(t >> 3) << 16);
    for (int b = t; b < 256; b += blockDim.x) {
        f16x8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = ((b >> e) & 1) ? (f16)1.0f : (f16)-1.0f;
        L.sign[b] = v;
    }
}

template <int D>
struct Tile<TqKey, D> {
    static constexpr int NV = D / 16;
    static constexpr int NQ = D / 32;        // MFMA k-blocks of each half (centroids, signs)
    static constexpr int CW = 3 * D / 128;   // code dwords of a lane's quarter
    static constexpr int SW = D / 128;       // sign dwords of a lane's quarter
    static constexpr int KB = tq_key_bytes(D);
    static constexpr int QD = 2 * D;
    uint32_t code[CW];  // 3-bit codes of dims (D/4) g .. +D/4 of token lane%16
    uint32_t sign[SW];  // QJL signs of the same dims
    f32x4 norm;         // norms of tokens 4g .. 4g+3 (the rows of this lane's scores)
    f16x4 v[NV];
    struct Q {
        f16x8 hi[2 * NQ];
        f16x8 lo[NQ];
    };

    __device__ __forceinline__ void load(const char* kbp, const char* vbp, int lane) {
        const int tok = lane & 15, grp = lane >> 4;
        const uint32_t* rec = reinterpret_cast<const uint32_t*>(kbp + tok * KB);
#pragma unroll
        for (int w = 0; w < CW; ++w) code[w] = rec[CW * grp + w];
#pragma unroll
        for (int w = 0; w < SW; ++w) sign[w] = rec[4 * CW + SW * grp + w];
        norm = *reinterpret_cast<const f32x4*>(kbp + kPageTokens * KB + 16 * grp);
        const f16* vb = reinterpret_cast<const f16*>(vbp);
#pragma unroll
        for (int t = 0; t < NV; ++t)
            v[t] = *reinterpret_cast<const f16x4*>(vb + (16 * t + tok) * 16 + 4 * grp);
    }
    static __device__ __forceinline__ void load_q(Q& q, const float* qrow, float qs, int grp) {
#pragma unroll
        for (int kb = 0; kb < 2 * NQ; ++kb) {
            const float* src = qrow + (kb < NQ ? (D / 4) * grp + 8 * kb : D + (D / 4) * grp + 8 * (kb - NQ));
            const f32x4 a = *reinterpret_cast<const f32x4*>(src);
            const f32x4 b = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float x = (i < 4 ? a[i] : b[i - 4]) * qs;
                const f16 h = to_f16(x);
                q.hi[kb][i] = h;
                if (kb < NQ) q.lo[kb][i] = to_f16(x - (float)h);
            }
        }
    }
    static __device__ __forceinline__ void prepare() { tq_lut_build(); }
    // the 6-bit code pair of elements 2p, 2p+1 of this lane's quarter
    __device__ __forceinline__ uint32_t pair_of(int p) const {
        const int bit = 6 * p, w = bit >> 5, off = bit & 31;
        const uint32_t x = off <= 26 ? code[w] >> off
                                     : __builtin_amdgcn_alignbit(code[w + 1], code[w], off);
        return x & 63u;
    }
    __device__ __forceinline__ f32x4 scores(const Q& q) const {
        const TqLut& L = tq_lut();
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < NQ; ++kb) {
            u32x4 w;
#pragma unroll
            for (int p = 0; p < 4; ++p) w[p] = L.pair[pair_of(4 * kb + p)];
            const f16x8 kf = __builtin_bit_cast(f16x8, w);
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, q.hi[kb], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, q.lo[kb], s, 0, 0, 0);
        }
#pragma unroll
        for (int kb = 0; kb < NQ; ++kb) {
            const f16x8 sf = L.sign[(sign[kb >> 2] >> (8 * (kb & 3))) & 255u];
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(sf, q.hi[NQ + kb], s, 0, 0, 0);
        }
        return s * norm;
    }
    __device__ __forceinline__ void mask_v(int valid) {
#pragma unroll
        for (int t = 0; t < NV; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i >= valid) v[t][i] = (f16)0.0f;
    }
    __device__ __forceinline__ void pv(f32x4* o, const float p[4]) const {
        f16x4 pb = {to_f16(p[0]), to_f16(p[1]), to_f16(p[2]), to_f16(p[3])};
#pragma unroll
        for (int t = 0; t < NV; ++t) o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(v[t], pb, o[t], 0, 0, 0);
    }
};

__device__ __forceinline__ int head_of(int kvh, int col, int n_kv, int group, int mode) {
    return mode == 0 ? kvh + col * n_kv : kvh * group + col;
}

// Query head of column c of segment `sidx` (KV head sidx / n_cb, column block
// sidx % n_cb), or -1 when the column holds no head.
__device__ __forceinline__ int seg_head(const DecodeParams& p, int sidx, int c, int n_kv) {
    const int kvh = sidx / p.n_cb, cg = (sidx % p.n_cb) * p.cols + c;
    if (c >= p.cols || cg >= p.group) return -1;
    const int h = head_of(kvh, cg, n_kv, p.group, p.gqa_mode);
    return h < p.n_q_heads ? h : -1;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// Softmax/PV state of one wavefront: O^T accumulators (lane = head column
// `col`, dims 16t + 4*grp + r), the lazily raised running max, and the
// per-lane partial sum (reduced over the 4 lane groups at the end).
template <int D>
struct Acc {
    f32x4 o[D / 16];
    float m, l;
};

template <typename KT, int D, int NP>
__device__ __forceinline__ void process(Acc<D>& acc, const Tile<KT, D>* tl, const int* valid,
                                        const typename Tile<KT, D>::Q& q, int grp) {
    f32x4 s[NP];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < NP; ++u) {
        s[u] = tl[u].scores(q);
        const int vg = valid[u] - 4 * grp;  // valid tokens among this lane's 4
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (r >= vg) s[u][r] = -INFINITY;
            mx = fmaxf(mx, s[u][r]);
        }
    }
    // Raise the running max only when some score exceeds it by the threshold;
    // all lanes of a head column then agree on the new max.
    if (__any(mx > acc.m + kLazyThreshold)) {
        mx = wave_max_xor(mx, 16);
        mx = wave_max_xor(mx, 32);
        const float m_new = fmaxf(acc.m, mx);
        const float alpha = fast_exp2(acc.m - m_new);
        acc.l *= alpha;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) acc.o[t] *= alpha;
        acc.m = m_new;
    }
#pragma unroll
    for (int u = 0; u < NP; ++u) {
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = fast_exp2(s[u][r] - acc.m);
        acc.l += (p[0] + p[1]) + (p[2] + p[3]);
        Tile<KT, D> t = tl[u];
        if (valid[u] < kPageTokens) t.mask_v(valid[u] - 4 * grp);
        t.pv(acc.o, p);
    }
}

// Prefix scan of per-sequence work items into LDS: s_cum[b] = items of
// sequences < b (per KV head); returns the total over all sequences.
__device__ __forceinline__ int scan_items(const DecodeParams& p, int* s_cum, int* s_red) {
    const int tid = threadIdx.x;
    const int batch = p.batch;
    int carry = 0;
    for (int base = 0; base < batch; base += kThreads) {
        const int b = base + tid;
        const int n = b < batch ? sched::items_of(sched::seq_tokens(p.ctx_len[b], p.max_pages), p.item_pages) : 0;
        // inclusive scan of n across the block
        int x = n;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o, 64);
            if ((tid & 63) >= o) x += y;
        }
        if ((tid & 63) == 63) s_red[tid >> 6] = x;
        __syncthreads();
        int wsum = 0;
        for (int w = 0; w < (tid >> 6); ++w) wsum += s_red[w];
        const int incl = carry + wsum + x;
        if (b < batch) s_cum[b] = incl - n;
        carry += s_red[0] + s_red[1] + s_red[2] + s_red[3];
        __syncthreads();
    }
    if (tid == 0) s_cum[batch] = carry;
    __syncthreads();
    return carry;
}

// Persistent, balanced decode.  The work of a launch is the list of "items"
// (p.item_pages pages of one (sequence, KV head) segment), ordered by sequence
// then KV head.  Workgroup w owns the contiguous item range
// [w*chunk, (w+1)*chunk), chunk = ceil(items / gridDim.x), so every
// workgroup streams the same number of pages and the launch has no tail.
// Consecutive items of one segment form a "run" that is accumulated without
// leaving registers; a run covering its whole segment writes the output,
// otherwise it writes a partial into the slot of its first item.
template <typename KT, int D, int NP>
__global__ __launch_bounds__(kThreads) void decode_kernel(KvGeom g, DecodeParams p,
                                                          DecodeWorkspace ws) {
    using T = Tile<KT, D>;
    __shared__ int s_cum[kMaxBatch + 1];
    __shared__ int s_red[4];
    __shared__ float s_m[kWaves][16];
    __shared__ float s_l[kWaves][16];
    __shared__ __attribute__((aligned(16))) float s_o[kWaves][kMaxGD];

    const int n_kv = g.n_kv_heads;
    const int n_seg = n_kv * p.n_cb;  // segments per sequence: (KV head, column block)
    const int tid = threadIdx.x;
    T::prepare();  // tile tables in LDS; the scan below has barriers
    const int per_kv = scan_items(p, s_cum, s_red);
    const int n_items = n_seg * per_kv;
    const int chunk = (n_items + gridDim.x - 1) / gridDim.x;
    int cur = blockIdx.x * chunk;
    const int end = min(n_items, cur + chunk);
    if (cur >= end) return;

    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const int GD = p.cols * D;
    const char* kpool = reinterpret_cast<const char*>(g.k);
    const char* vpool = reinterpret_cast<const char*>(g.v);

    int b = sched::find_seq(s_cum, p.batch, n_seg, cur);
    while (cur < end) {
        const sched::Run run = sched::run_at(s_cum, p.ctx_len, p.max_pages, n_seg, p.item_pages, b,
                                             cur, end);
        b = run.b;
        const int sidx = run.kvh, kvh = sidx / p.n_cb;  // segment within the sequence, its KV head
        const int seg0 = run.seg0, run_end = run.run_end, L = run.len;
        const int pg0 = run.pg0, pg1 = run.pg1;
        const bool whole = run.whole;
        if (cur == seg0 && tid == 0) {  // the segment's run table, for the merge kernel
            int wg1;
            const int n_runs = sched::merge_runs(s_cum, n_seg, chunk, b, sidx, &wg1);
            const size_t seg = (size_t)b * n_seg + sidx;
            ws.seg_runs[2 * seg] = wg1;
            ws.seg_runs[2 * seg + 1] = n_runs;
        }

        const int head = seg_head(p, sidx, col, n_kv);
        const bool col_on = head >= 0;
        typename T::Q q;
        T::load_q(q, p.q + ((size_t)b * p.n_q_heads + (col_on ? head : 0)) * T::QD,
                  col_on ? p.scale * kLog2e : 0.f, grp);
        Acc<D> acc;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) acc.o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc.m = -1e30f;
        acc.l = 0.f;
        const int32_t* pt = p.page_table + (size_t)b * p.max_pages;

        // sub-runs of up to 256 pages: a wavefront's page ids fit one VGPR
        for (int sub = pg0; sub < pg1; sub += sched::kSubPages) {
            int first, n_my;  // this wave's pages: first + 4j, j < n_my
            sched::sub_pages(sub, pg1, wave, &first, &n_my);
            // A page id outside [0, n_pages) holds no tokens: page 0 is read in
            // its place and every token of it is masked.
            const int pid_raw = lane < n_my ? pt[first + kWaves * lane] : 0;
            const bool bad = !sched::page_ok(pid_raw, g.n_pages);
            const int pid_v = bad ? 0 : pid_raw;
            const uint64_t bad_pages = __ballot(bad);
            const int first_pid = __builtin_amdgcn_readfirstlane(pid_v);
            auto load_group = [&](T* dst, int i) {
#pragma unroll
                for (int u = 0; u < NP; ++u) {
                    const int j = NP * i + u;
                    const int pid = j < n_my ? __builtin_amdgcn_readlane(pid_v, j) : first_pid;
                    const size_t blk = (size_t)pid * n_kv + kvh;
                    dst[u].load(kpool + blk * g.kstride, vpool + blk * g.vstride, lane);
                }
            };
            auto valid_of = [&](int* valid, int i) {
#pragma unroll
                for (int u = 0; u < NP; ++u) {
                    const int j = NP * i + u;
                    const int tok0 = (first + kWaves * j) * kPageTokens;
                    valid[u] = j < n_my && !((bad_pages >> j) & 1) ? min(L - tok0, kPageTokens) : 0;
                }
            };
            const int n_iter = (n_my + NP - 1) / NP;
            if (n_iter > 0) {
                T tcur[NP], tnxt[NP];
                int valid[NP];
                load_group(tcur, 0);
                for (int i = 0; i < n_iter - 1; ++i) {
                    load_group(tnxt, i + 1);
                    valid_of(valid, i);
                    process<KT, D, NP>(acc, tcur, valid, q, grp);
#pragma unroll
                    for (int u = 0; u < NP; ++u) tcur[u] = tnxt[u];
                }
                valid_of(valid, n_iter - 1);
                process<KT, D, NP>(acc, tcur, valid, q, grp);
            }
        }
        acc.l = wave_sum_xor(acc.l, 16);
        acc.l = wave_sum_xor(acc.l, 32);

        // ---- merge the 4 wavefronts in LDS ----
        // (a column with no head ran a zero query: finite values, never written out)
        if (col < p.cols) {
#pragma unroll
            for (int t = 0; t < D / 16; ++t)
                *reinterpret_cast<f32x4*>(&s_o[wave][col * D + 16 * t + 4 * grp]) = acc.o[t];
            if (grp == 0) {
                s_m[wave][col] = acc.m;
                s_l[wave][col] = acc.l;
            }
        }
        __syncthreads();
        const size_t slot = (size_t)sched::run_slot(cur == seg0, b, sidx, n_seg, p.batch, blockIdx.x);
        float* po = ws.partial_o + slot * GD;
        float* pml = ws.partial_ml + slot * p.cols * 2;
        for (int idx = tid; idx < GD; idx += kThreads) {
            const int c = idx / D, d = idx - c * D;
            float M = s_m[0][c];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][c]);
            float o = 0.f, lsum = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float f = fast_exp2(s_m[w][c] - M);
                o += f * s_o[w][idx];
                lsum += f * s_l[w][c];
            }
            if (whole) {
                const int h = seg_head(p, sidx, c, n_kv);
                if (h < 0) continue;
                const size_t oi = ((size_t)b * p.n_q_heads + h) * D + d;
                float r = lsum > 0.f ? o / lsum : 0.f;  // every key masked: zeros
                if (p.gate) r *= sigmoidf_(p.gate[oi]);
                p.out[oi] = r;
            } else {
                po[idx] = o;
                if (d == 0) {
                    pml[2 * c] = M;
                    pml[2 * c + 1] = lsum;
                }
            }
        }
        __syncthreads();  // LDS is reused by the next run
        cur = run_end;
    }
}

// Combines the run partials of every (sequence, KV head, column block) segment
// that spans more than one workgroup range; zero-length sequences get zeros.
// The segment's run table (workgroup of run 1, number of runs) was written by
// the decode workgroup that started it.  Grid (ceil(cols*D / 256), segments
// per sequence, batch):
// a workgroup owns 256 output values of one segment (64 16-byte groups); its
// 4 wavefronts first form the run weights of the block's columns, then sum
// every 4th run each and meet in LDS.
template <int V>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeParams p, DecodeWorkspace ws,
                                                           int n_kv, int D) {
    // V values per thread (4, or 1 for launches with few workgroups): 64 V per workgroup
    typedef typename std::conditional<V == 4, f32x4, float>::type VT;
    __shared__ float s_w[4][kMaxRuns];  // per column (<= 4 per 256 values) and run
    __shared__ int s_slot[kMaxRuns];
    __shared__ float s_inv[4];
    __shared__ __attribute__((aligned(16))) VT s_acc[4][64];
    const int sidx = blockIdx.y, b = blockIdx.z, n_seg = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cols = p.cols, GD = cols * D;
    const int e0 = blockIdx.x * 64 * V;
    const size_t seg = (size_t)b * n_seg + sidx;
    // The context length and the run table load together: a merge is a short chain of
    // dependent memory round trips, so every load that can is issued beside another.
    const int ctx = p.ctx_len[b];
    const int wg1 = ws.seg_runs[2 * seg], n_runs_raw = ws.seg_runs[2 * seg + 1];
    // the gate of wavefront 0's outputs too (it needs no merged value)
    const int e = e0 + V * lane;
    const bool on = e < GD;  // GD is a multiple of 4 (D >= 64)
    VT gt = VT{};
    if (p.gate && wave == 0 && on) {
        const int c = e / D, d = e - c * D;
        const int h = seg_head(p, sidx, c, n_kv);
        if (h >= 0) gt = *reinterpret_cast<const VT*>(p.gate + ((size_t)b * p.n_q_heads + h) * D + d);
    }
    if (sched::seq_tokens(ctx, p.max_pages) == 0) {
        // empty context: softmax over nothing leaves zeros (src/ops.rs:161)
        const int idx = e0 + tid;
        if (tid < 64 * V && idx < GD) {
            const int c = idx / D, d = idx - c * D;
            const int h = seg_head(p, sidx, c, n_kv);
            if (h >= 0) p.out[((size_t)b * p.n_q_heads + h) * D + d] = 0.f;
        }
        return;
    }
    const int n_runs = n_runs_raw;
    if (n_runs <= 1) return;  // one run: written directly by decode_kernel
    for (int r = tid; r < n_runs; r += 256)
        s_slot[r] = (int)sched::run_slot(r == 0, b, sidx, n_seg, p.batch, wg1 + r - 1);
    __syncthreads();
    const int c_lo = e0 / D, c_hi = min(cols - 1, (e0 + 64 * V - 1) / D);
    // thread (wave, lane): values e0 + 4 lane .. +3 of runs wave, wave + 4, ...; the first
    // kPre of those runs are loaded now, beside the (max, sum) pairs, before any weight is known
    constexpr int kPre = 4;
    const float* po = ws.partial_o + (on ? e : 0);
    auto part = [&](int r) { return *reinterpret_cast<const VT*>(po + (size_t)s_slot[r] * GD); };
    const VT zero = VT{};
    VT pre[kPre];
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
        const int r = wave + 4 * j;
        pre[j] = r < n_runs ? part(r) : zero;
    }
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2* pml = reinterpret_cast<const f2*>(ws.partial_ml);
    if (wave <= c_hi - c_lo) {  // one wavefront per column of this block
        const int c = c_lo + wave;
        // (running max, sum) of runs lane, lane + 64, ... : the first in registers
        const f2 ml0 = lane < n_runs ? pml[(size_t)s_slot[lane] * cols + c] : f2{-1e30f, 0.f};
        float M = ml0[0];
        for (int r = lane + 64; r < n_runs; r += 64) M = fmaxf(M, pml[(size_t)s_slot[r] * cols + c][0]);
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) M = wave_max_xor(M, m);
        float lsum = 0.f;
        if (lane < n_runs) {
            const float w = fast_exp2(ml0[0] - M);
            s_w[wave][lane] = w;
            lsum = w * ml0[1];
        }
        for (int r = lane + 64; r < n_runs; r += 64) {
            const f2 ml = pml[(size_t)s_slot[r] * cols + c];
            const float w = fast_exp2(ml[0] - M);
            s_w[wave][r] = w;
            lsum += w * ml[1];
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) lsum = wave_sum_xor(lsum, m);
        if (lane == 0) s_inv[wave] = lsum > 0.f ? 1.0f / lsum : 0.f;
    }
    __syncthreads();
    const int cw = (on ? e / D : c_lo) - c_lo;
    const float* w = s_w[cw];
    VT a[4];
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
        const int r = wave + 4 * j;
        a[j] = r < n_runs ? w[r] * pre[j] : zero;
    }
    int r = wave + 4 * kPre;
    for (; r + 12 < n_runs; r += 16) {  // four independent loads in flight
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] += w[r + 4 * j] * part(r + 4 * j);
    }
    for (; r < n_runs; r += 4) a[0] += w[r] * part(r);
    s_acc[wave][lane] = (a[0] + a[1]) + (a[2] + a[3]);
    __syncthreads();
    if (wave != 0 || !on) return;
    const VT acc = (s_acc[0][lane] + s_acc[1][lane]) + (s_acc[2][lane] + s_acc[3][lane]);
    const float inv = s_inv[cw];
    const int c = e / D, d = e - c * D;
    const int h = seg_head(p, sidx, c, n_kv);
    if (h < 0) return;
    const size_t oi = ((size_t)b * p.n_q_heads + h) * D + d;
    VT res = acc * inv;
    if (p.gate) {
        float* rp = reinterpret_cast<float*>(&res);
        const float* gp = reinterpret_cast<const float*>(&gt);
#pragma unroll
        for (int i = 0; i < V; ++i) rp[i] *= sigmoidf_(gp[i]);
    }
    *reinterpret_cast<VT*>(p.out + oi) = res;
}

template <typename KT, int D>
constexpr int np_of() {
    return std::is_same<KT, TqKey>::value ? 1 : sizeof(KT) == 2 ? 2 : 1;
}

template <typename KT, int D>
int wgs_per_cu() {
    static int n = -1;
    if (n < 0) {
        int v = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, decode_kernel<KT, D, np_of<KT, D>()>,
                                                         kThreads, 0) != hipSuccess || v <= 0)
            v = 1;
        n = v;
    }
    return n;
}

template <typename KT, int D>
hipError_t launch_t(const KvGeom& g, const DecodeParams& p, const DecodeWorkspace& ws,
                    const DecodePlan& plan, hipStream_t s) {
    hipLaunchKernelGGL((decode_kernel<KT, D, np_of<KT, D>()>), dim3(plan.grid), dim3(kThreads), 0,
                       s, g, p, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // 256 values per merge workgroup, or 64 when that leaves fewer than 128 workgroups
    // (one long sequence: each segment's many runs then spread over four times the CUs)
    const long long wg4 = (long long)((p.cols * D + 255) / 256) * g.n_kv_heads * p.n_cb * p.batch;
    if (wg4 >= 128)
        hipLaunchKernelGGL(decode_merge_kernel<4>, dim3((p.cols * D + 255) / 256, g.n_kv_heads * p.n_cb, p.batch),
                           dim3(256), 0, s, p, ws, g.n_kv_heads, D);
    else
        hipLaunchKernelGGL(decode_merge_kernel<1>, dim3((p.cols * D + 63) / 64, g.n_kv_heads * p.n_cb, p.batch),
                           dim3(256), 0, s, p, ws, g.n_kv_heads, D);
    return hipGetLastError();
}

}  // namespace

DecodePlan decode_plan(const KvGeom& g, int32_t batch, int32_t max_pages, int32_t n_q_heads,
                       int32_t gqa_mode, int device, int32_t max_tokens) {
    DecodePlan plan;
    // head blocking: the modulo map (h % Hkv) gives KV head k the heads k, k + Hkv, ... below
    // Hq, at most ceil(Hq / Hkv); a segment takes up to 16 of them and cols * D <= 2048 floats
    plan.group = gqa_mode == 0 ? (n_q_heads + g.n_kv_heads - 1) / g.n_kv_heads : n_q_heads / g.n_kv_heads;
    const int max_cols = std::min(16, kMaxGD / g.head_dim);
    plan.n_cb = (plan.group + max_cols - 1) / max_cols;
    plan.cols = (plan.group + plan.n_cb - 1) / plan.n_cb;  // even blocks
    const int n_seg = g.n_kv_heads * plan.n_cb;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        cus <= 0)
        cus = 256;
    int per_cu = 1;
    const bool hp = g.dtype == 1;
    if (g.dtype == kTqDtype) per_cu = g.head_dim == 256 ? wgs_per_cu<TqKey, 256>() : wgs_per_cu<TqKey, 128>();
    else switch (g.head_dim) {
        case 64: per_cu = hp ? wgs_per_cu<f16, 64>() : wgs_per_cu<float, 64>(); break;
        case 128: per_cu = hp ? wgs_per_cu<f16, 128>() : wgs_per_cu<float, 128>(); break;
        default: per_cu = hp ? wgs_per_cu<f16, 256>() : wgs_per_cu<float, 256>(); break;
    }
    // A segment splits into at most grid + 1 runs; the merge kernel stages
    // kMaxRuns of them in LDS, so the grid stays below that.
    plan.grid = std::min(cus * per_cu, kMaxRuns - 1);
    if (const char* e = std::getenv("PI_DECODE_GRID")) {
        const int v = std::atoi(e);
        if (v >= 1 && v < kMaxRuns) plan.grid = v;
    }
    // Item size: kItemPages pages, halved while the launch's upper bound of
    // items would not give every workgroup two items (small batches and short
    // contexts then still spread over the whole chip).  The bound is the caller's
    // max_tokens per sequence when it gives one, else the table row.
    const long long seq_pages =
        max_tokens > 0 ? std::min<long long>(max_pages, ((long long)max_tokens + kPageTokens - 1) / kPageTokens)
                       : max_pages;
    const long long max_seg_pages = (long long)batch * n_seg * seq_pages;
    int ip = kItemPages;
    while (ip > 1 && max_seg_pages / ip < 2LL * plan.grid) ip >>= 1;
    plan.item_pages = ip;
    // one partial slot per segment and one per workgroup (run_slot)
    plan.n_slots = (long long)batch * n_seg + plan.grid;
    plan.batch = batch;
    return plan;
}

namespace {
constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];
}  // namespace

hipError_t decode_scratch(int device, float** ptr) {
    *ptr = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    float* p = g_scratch[device].load(std::memory_order_acquire);
    if (!p) {
        // the device is current (pi_create sets it); each GPU has its own copy
        void* a = nullptr;
        const hipError_t e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        p = static_cast<float*>(a);
        g_scratch[device].store(p, std::memory_order_release);
    }
    *ptr = p;
    return hipSuccess;
}

size_t decode_ws_floats_o(const KvGeom& g, const DecodePlan& plan) {
    return (size_t)plan.n_slots * plan.cols * g.head_dim;
}

size_t decode_ws_ints_runs(const KvGeom& g, const DecodePlan& plan) {
    return (size_t)2 * plan.batch * g.n_kv_heads * plan.n_cb;
}

hipError_t launch_decode(const KvGeom& g, const DecodeParams& p, const DecodeWorkspace& ws,
                         const DecodePlan& plan, hipStream_t s) {
    if (g.dtype == kTqDtype) {
        if (g.head_dim == 128) return launch_t<TqKey, 128>(g, p, ws, plan, s);
        if (g.head_dim == 256) return launch_t<TqKey, 256>(g, p, ws, plan, s);
        return hipErrorInvalidValue;
    }
    const bool hp = g.dtype == 1;
    switch (g.head_dim) {
        case 64: return hp ? launch_t<f16, 64>(g, p, ws, plan, s) : launch_t<float, 64>(g, p, ws, plan, s);
        case 128: return hp ? launch_t<f16, 128>(g, p, ws, plan, s) : launch_t<float, 128>(g, p, ws, plan, s);
        case 256: return hp ? launch_t<f16, 256>(g, p, ws, plan, s) : launch_t<float, 256>(g, p, ws, plan, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace pi

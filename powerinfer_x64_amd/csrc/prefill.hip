// prefill.hip -- causal GQA flash attention for a whole prompt (gfx950 MFMA).
//
// Replaces the reference's prefill attention, which runs the decode loop once
// per prompt token (src/model/mod.rs:668 token loop, :1140-1190 append-then-
// attend), i.e. row i attends keys 0..i.
//
// Work decomposition: a workgroup of 4 wavefronts owns 32 query positions and
// 4 query heads that share one KV head (group % 4 == 0), or 128 positions of
// one head otherwise; each wavefront owns 32 query rows.  Per 64-key block the
// workgroup stages K [64 x D] and V^T [D x 64] (bf16/f16) in LDS, and each
// wavefront computes with v_mfma_f32_32x32x16:
//   S^T[64 key x 32 q] = K . Q^T          (16 MFMA)
//   O^T[D x 32 q]     += V^T . P^T        (16 MFMA)
// Softmax runs in f32 on S^T, where a lane owns one query column, so the row
// max/sum need one cross-lane step.  Causal blocks past the diagonal are
// skipped; workgroups are launched heaviest-first.
#include "pi_device.hpp"
#include "pi_launch.hpp"

namespace pi {
namespace {

constexpr int D = 128;
constexpr int BN = 64;         // keys per block
constexpr int ROWS = 32;       // query rows per wavefront
constexpr int KSTR = D + 8;    // LDS row stride of K (elements)
constexpr int VSTR = BN + 4;   // LDS row stride of V^T (elements)
constexpr float kLazy = 8.0f;  // log2 headroom before the running max moves

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16> {
    typedef bf16x8 v8;
    typedef bf16x4 v4;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mfma<f16> {
    typedef f16x8 v8;
    typedef f16x4 v4;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

struct PrefillArgs {
    const void* q;
    const void* k;
    const void* v;
    float* out;
    int S, hq, hkv, group, causal, gqa_mode, pack4;
    float qk_scale;  // scale * log2(e)
};

__device__ __forceinline__ int head_of(int kvh, int c, int hkv, int group, int mode) {
    return mode == 0 ? kvh + c * hkv : kvh * group + c;
}

template <typename T>
__global__ __launch_bounds__(256, 2) void prefill_kernel(PrefillArgs a) {
    typedef typename Mfma<T>::v8 v8;
    typedef typename Mfma<T>::v4 v4;
    // double-buffered K [64 x D] and V^T [D x 64] tiles
    __shared__ __attribute__((aligned(16))) T sk[2][BN * KSTR];
    __shared__ __attribute__((aligned(16))) T sv[2][D * VSTR];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.z;
    const int S = a.S;
    const int qb = gridDim.y - 1 - blockIdx.y;  // heaviest (latest) query blocks first

    int kvh, head, p0, p_last;
    if (a.pack4) {
        const int cg = blockIdx.x % (a.group / 4);
        kvh = blockIdx.x / (a.group / 4);
        head = head_of(kvh, 4 * cg + wave, a.hkv, a.group, a.gqa_mode);
        p0 = qb * ROWS;
        p_last = p0 + ROWS - 1;
    } else {
        head = blockIdx.x;
        kvh = a.gqa_mode == 0 ? head % a.hkv : head / a.group;
        p0 = qb * 4 * ROWS + wave * ROWS;
        p_last = qb * 4 * ROWS + 4 * ROWS - 1;
    }
    const int kv_end = a.causal ? min(S, p_last + 1) : S;
    const int n_blocks = (kv_end + BN - 1) / BN;

    const int r = lane & 31;   // query column of this lane
    const int hh = lane >> 5;  // which 8-wide k slice
    const int qpos = p0 + r;

    // Q^T operand: lane holds q[qpos][16*kk + 8*hh .. +7]
    const T* qg = reinterpret_cast<const T*>(a.q);
    v8 qr[D / 16];
    {
        const bool ok = qpos < S;
        const T* qrow = qg + (((size_t)b * S + (ok ? qpos : 0)) * a.hq + head) * D;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
            v8 t = *reinterpret_cast<const v8*>(qrow + 16 * kk + 8 * hh);
            if (!ok) t = v8{};
            qr[kk] = t;
        }
    }

    f32x16 o[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) o[i] = f32x16{};
    float m_run = -1e30f, l_run = 0.f;  // running max in scaled log2 units

    const T* kg = reinterpret_cast<const T*>(a.k);
    const T* vg = reinterpret_cast<const T*>(a.v);
    const size_t tok_stride = (size_t)a.hkv * D;
    const T* kbase = kg + ((size_t)b * S * a.hkv + kvh) * D;
    const T* vbase = vg + ((size_t)b * S * a.hkv + kvh) * D;
    const int tg = tid & 15, dc = tid >> 4;

    v8 kreg[4], vreg[4];
    auto load_tile = [&](int kb) {
        const int k0 = kb * BN;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int id = tid + 256 * i;
            const int tk = id >> 4, c = id & 15;
            v8 t = v8{};
            if (k0 + tk < S) t = *reinterpret_cast<const v8*>(kbase + (size_t)(k0 + tk) * tok_stride + 8 * c);
            kreg[i] = t;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tk = 4 * tg + i;
            v8 t = v8{};
            if (k0 + tk < S) t = *reinterpret_cast<const v8*>(vbase + (size_t)(k0 + tk) * tok_stride + 8 * dc);
            vreg[i] = t;
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int id = tid + 256 * i;
            const int tk = id >> 4, c = id & 15;
            *reinterpret_cast<v8*>(&sk[buf][tk * KSTR + 8 * c]) = kreg[i];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v4 t = {vreg[0][e], vreg[1][e], vreg[2][e], vreg[3][e]};
            *reinterpret_cast<v4*>(&sv[buf][(8 * dc + e) * VSTR + 4 * tg]) = t;
        }
    };

    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kb = 0; kb < n_blocks; ++kb) {
        const int k0 = kb * BN;
        const int buf = kb & 1;
        const bool more = kb + 1 < n_blocks;
        if (more) load_tile(kb + 1);  // in flight while this block computes

        // every key of this block in this wave's future: nothing to do
        if (!(a.causal && k0 > p0 + ROWS - 1)) {
            // ---- S^T = K . Q^T : two 32x32 tiles (keys 0-31, 32-63) ----
            f32x16 s[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                f32x16 acc = f32x16{};
#pragma unroll
                for (int kk = 0; kk < D / 16; ++kk) {
                    const v8 ka = *reinterpret_cast<const v8*>(&sk[buf][(32 * tt + r) * KSTR + 16 * kk + 8 * hh]);
                    acc = Mfma<T>::mma(ka, qr[kk], acc);
                }
                s[tt] = acc;
            }
            // mask; lane holds key rows 32*tt + 8*i + 4*hh + j for query qpos
            const bool need_mask = (a.causal && k0 + BN - 1 > p0) || (k0 + BN > S);
            float mx = -INFINITY;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        float x = s[tt][4 * i + j];
                        if (need_mask) {
                            const int key = k0 + 32 * tt + 8 * i + 4 * hh + j;
                            if (key >= S || (a.causal && key > qpos)) x = -INFINITY;
                        }
                        s[tt][4 * i + j] = x;
                        mx = fmaxf(mx, x);
                    }
            // lazily raised running max (scaled units); the scale is fused into exp2
            const float c = a.qk_scale;
            if (__any(mx * c > m_run + kLazy)) {
                mx = wave_max_xor(mx, 32);
                const float m_new = fmaxf(m_run, mx * c);
                const float alpha = fast_exp2(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int i = 0; i < D / 32; ++i) o[i] *= alpha;
                m_run = m_new;
            }
            float ls = 0.f;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float pe = fast_exp2(__builtin_fmaf(s[tt][e], c, -m_run));
                    s[tt][e] = pe;
                    ls += pe;
                }
            l_run += ls;

            // ---- O^T += V^T . P^T : 4 key steps of 16, 4 dim tiles of 32 ----
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int tt = ks >> 1, i0 = 2 * (ks & 1);
                v8 pb;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    pb[j] = (T)s[tt][4 * i0 + j];
                    pb[4 + j] = (T)s[tt][4 * (i0 + 1) + j];
                }
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt) {
                    const T* vrow = &sv[buf][(32 * dt + r) * VSTR + 16 * ks + 4 * hh];
                    const v4 lo = *reinterpret_cast<const v4*>(vrow);
                    const v4 hi = *reinterpret_cast<const v4*>(vrow + 8);
                    const v8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    o[dt] = Mfma<T>::mma(va, pb, o[dt]);
                }
            }
        }
        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }

    l_run = wave_sum_xor(l_run, 32);
    if (qpos >= S) return;
    const float inv = 1.0f / l_run;
    float* orow = a.out + (((size_t)b * S + qpos) * a.hq + head) * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f32x4 t = {o[dt][4 * i] * inv, o[dt][4 * i + 1] * inv, o[dt][4 * i + 2] * inv,
                       o[dt][4 * i + 3] * inv};
            *reinterpret_cast<f32x4*>(orow + 32 * dt + 8 * i + 4 * hh) = t;
        }
}

}  // namespace

hipError_t launch_prefill(const void* q, const void* k, const void* v, int32_t dtype,
                          int32_t batch, int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads,
                          int32_t head_dim, int32_t causal, int32_t gqa_mode, float scale,
                          float* out, hipStream_t s) {
    if (head_dim != D) return hipErrorInvalidValue;
    PrefillArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.S = seq_len;
    a.hq = n_q_heads;
    a.hkv = n_kv_heads;
    a.group = n_q_heads / n_kv_heads;
    a.causal = causal;
    a.gqa_mode = gqa_mode;
    a.pack4 = (a.group % 4) == 0;
    a.qk_scale = scale * kLog2e;
    dim3 grid;
    // x = head group (fastest), y = query block (reversed in the kernel), so the
    // heaviest query blocks of every head group are dispatched first.
    if (a.pack4)
        grid = dim3(n_kv_heads * (a.group / 4), (seq_len + ROWS - 1) / ROWS, batch);
    else
        grid = dim3(n_q_heads, (seq_len + 4 * ROWS - 1) / (4 * ROWS), batch);
    if (dtype == 2)
        hipLaunchKernelGGL(prefill_kernel<bf16>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(prefill_kernel<f16>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace pi

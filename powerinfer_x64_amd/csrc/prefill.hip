// prefill.hip -- causal GQA flash attention for a whole prompt (gfx950 MFMA).
//
// Replaces the reference's prefill attention, which runs the decode loop once
// per prompt token (src/model/mod.rs:668 token loop, :1140-1190 append-then-
// attend), i.e. row i attends keys 0..i.
//
// One kernel, prefill_fa_kernel (below): a workgroup of 8 wavefronts covers
// HPW query heads that share one KV head and 256/HPW query positions; each
// wavefront owns 32 query rows of one head and computes, per 64-key tile,
//   S^T[64 key x 32 q] = K . Q^T          (16 x v_mfma_f32_32x32x16)
//   O^T[D x 32 q]     += V^T . P^T        (16 x v_mfma_f32_32x32x16)
// with the softmax in f32 on S^T, where a lane owns one query column, so the
// row max / sum need one cross-lane step.  Tiles past the diagonal are
// skipped; workgroups are launched heaviest-first.
#include "pi_device.hpp"
#include "pi_launch.hpp"

namespace pi {
namespace {

constexpr int D = 128;
constexpr int BN = 64;         // keys per block
constexpr int ROWS = 32;       // query rows per wavefront
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
    // sum of the 8 packed values (f32 accumulation, v_dot2 against ones)
    static __device__ __forceinline__ float sum8(v8 p) {
        typedef bf16 v2 __attribute__((ext_vector_type(2)));
        const v2 one = {(bf16)1.0f, (bf16)1.0f};
        const float a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 0, 1), one,
                                                        0.f, false);
        const float b = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 4, 5), one,
                                                        0.f, false);
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 6, 7), one,
                                               __builtin_amdgcn_fdot2_f32_bf16(
                                                   __builtin_shufflevector(p, p, 2, 3), one, a, false),
                                               false) + b;
    }
};
template <>
struct Mfma<f16> {
    typedef f16x8 v8;
    typedef f16x4 v4;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ float sum8(v8 p) {
        typedef f16 v2 __attribute__((ext_vector_type(2)));
        const v2 one = {(f16)1.0f, (f16)1.0f};
        const float a = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 0, 1), one, 0.f, false);
        const float b = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 4, 5), one, 0.f, false);
        return __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 6, 7), one,
                                      __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 2, 3),
                                                             one, a, false),
                                      false) + b;
    }
};

struct PrefillArgs {
    const void* q;
    const void* k;
    const void* v;
    float* out;
    int S, hq, hkv, group, causal, gqa_mode;
    float qk_scale;  // scale * log2(e)
};

__device__ __forceinline__ int head_of(int kvh, int c, int hkv, int group, int mode) {
    return mode == 0 ? kvh + c * hkv : kvh * group + c;
}

// ---------------------------------------------------------------------------
// prefill_fa_kernel: 8 wavefronts per workgroup (2 per SIMD), one workgroup
// per CU.  Wave w owns 32 query rows of one query head: head slot w % HPW of
// the workgroup's HPW heads (they share one KV head) and row tile w / HPW, so
// a workgroup covers HPW heads x 256/HPW rows and every K/V byte it stages in
// LDS serves 8 wavefronts.
//
// K and V tiles (64 keys x D) are staged through registers into four LDS
// buffers (one barrier per tile): K in its [key][dim] order with 272-byte
// rows, V transposed to V^T [dim][key] with 136-byte rows, both bank-conflict
// free for the fragment reads, whose addresses are one base register plus an
// immediate.  K and V^T fragments are read PF ahead of their MFMAs.
// Only a wavefront's last tile can need the causal / prompt-end mask; the
// mask is one wave-uniform branch around a straight-line select block.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float max16(const f32x16& s) {
    const float a = fmaxf(fmaxf(s[0], s[1]), s[2]);
    const float b = fmaxf(fmaxf(s[3], s[4]), s[5]);
    const float c = fmaxf(fmaxf(s[6], s[7]), s[8]);
    const float d = fmaxf(fmaxf(s[9], s[10]), s[11]);
    const float e = fmaxf(fmaxf(s[12], s[13]), s[14]);
    return fmaxf(fmaxf(fmaxf(a, b), fmaxf(c, d)), fmaxf(e, s[15]));
}

template <typename T, int HPW>
__global__ __launch_bounds__(512, 1) void prefill_fa_kernel(PrefillArgs a) {
    typedef typename Mfma<T>::v8 v8;
    typedef typename Mfma<T>::v4 v4;
    constexpr int NW = 8;
    constexpr int RT = NW / HPW;      // row tiles per workgroup
    constexpr int WROWS = ROWS * RT;  // query rows per workgroup
    constexpr int NBUF = 4;
    constexpr int KS = D + 8;   // K [key][dim] row stride (elements): 272 B
    constexpr int VT = BN + 4;  // V^T [dim][key] row stride (elements): 136 B
    __shared__ __attribute__((aligned(16))) T sk[NBUF][BN * KS];
    __shared__ __attribute__((aligned(16))) T sv[NBUF][D * VT];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hs = wave % HPW, rt = wave / HPW;
    const int b = blockIdx.z;
    const int S = a.S;
    const int qb = gridDim.y - 1 - blockIdx.y;  // heaviest (latest) query blocks first
    const int per_kv = a.group / HPW;           // workgroups per KV head
    const int kvh = blockIdx.x / per_kv;
    const int head = head_of(kvh, (blockIdx.x % per_kv) * HPW + hs, a.hkv, a.group, a.gqa_mode);
    const int p0 = qb * WROWS + rt * ROWS;
    const int wg_keys = a.causal ? min(S, qb * WROWS + WROWS) : S;
    const int n_tiles = (wg_keys + BN - 1) / BN;
    const int w_keys = a.causal ? min(S, p0 + ROWS) : S;
    const int w_tiles = p0 < S ? (w_keys + BN - 1) / BN : 0;  // tiles this wavefront attends
    const bool last_masked = w_tiles > 0 && ((a.causal && (w_tiles - 1) * BN + BN - 1 > p0) ||
                                             w_tiles * BN > S);

    const int r = lane & 31;   // query column of this lane
    const int hh = lane >> 5;  // 8-wide k slice of the MFMA operands
    const int qpos = p0 + r;

    // Q^T operand: lane holds q[qpos][16*kk + 8*hh .. +7]
    v8 qr[D / 16];
    {
        const T* qg = reinterpret_cast<const T*>(a.q);
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
    float m_run = -1e30f, l_run = 0.f;  // running max (scaled log2 units), lane partial sum

    const size_t tok_stride = (size_t)a.hkv * D;
    const T* kbase = reinterpret_cast<const T*>(a.k) + ((size_t)b * S * a.hkv + kvh) * D;
    const T* vbase = reinterpret_cast<const T*>(a.v) + ((size_t)b * S * a.hkv + kvh) * D;

    // Tile t (64 keys) is staged through registers: thread i loads two
    // 16-byte K chunks (rows (i + 512j) / 16) and, for key pair i % 32, the
    // 8 dims 8*(i/32) .. +7 of both keys of V, which it writes transposed as
    // V^T.  Rows past the prompt read as zeros (their scores are masked).
    v8 kreg[2], vreg[2];
    const int kp = tid & 31, vdc = tid >> 5;
    auto load_tile = [&](int t) {
        const int k0 = t * BN;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int id = tid + 512 * i;
            const int row = id >> 4, ch = id & 15;
            v8 x = v8{};
            if (k0 + row < S) x = *reinterpret_cast<const v8*>(kbase + (size_t)(k0 + row) * tok_stride + 8 * ch);
            kreg[i] = x;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int key = k0 + 2 * kp + i;
            v8 x = v8{};
            if (key < S) x = *reinterpret_cast<const v8*>(vbase + (size_t)key * tok_stride + 8 * vdc);
            vreg[i] = x;
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int id = tid + 512 * i;
            const int row = id >> 4, ch = id & 15;
            *reinterpret_cast<v8*>(&sk[buf][row * KS + 8 * ch]) = kreg[i];
        }
        typedef T v2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const v2 x = {vreg[0][e], vreg[1][e]};
            *reinterpret_cast<v2*>(&sv[buf][(8 * vdc + e) * VT + 2 * kp]) = x;
        }
    };

    const float c = a.qk_scale;
    // Per-lane LDS bases in buffer 0: every fragment of a tile is base +
    // buffer offset + an immediate offset.
    typedef __attribute__((address_space(3))) const T* lds_ptr;
    const lds_ptr k_lane = (lds_ptr)&sk[0][r * KS + 8 * hh];
    const lds_ptr v_lane = (lds_ptr)&sv[0][r * VT + 4 * hh];
    auto kfrag = [&](lds_ptr kt, int i) {  // i = 2*kk + tt
        return *reinterpret_cast<__attribute__((address_space(3))) const v8*>(kt + (i & 1) * 32 * KS + (i >> 1) * 16);
    };
    // V^T operand: dims 32*dt + r, keys 16*ks + 4*hh + (0..3) and +8 -- the
    // key order of the P^T operand.
    auto vfrag = [&](lds_ptr vt, int i) {  // i = 4*ks + dt
        const lds_ptr p1 = vt + (i & 3) * 32 * VT + (i >> 2) * 16;
        const v4 lo = *reinterpret_cast<__attribute__((address_space(3))) const v4*>(p1);
        const v4 hi = *reinterpret_cast<__attribute__((address_space(3))) const v4*>(p1 + 8);
        return v8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    constexpr int PF = 4;  // fragments in flight

    // S^T = K . Q^T for tile t: two 32x32 tiles (keys 0-31, 32-63),
    // interleaved so consecutive MFMAs are independent; K fragments read PF
    // ahead
    auto tile_qk = [&](int t, f32x16* s) {
        const lds_ptr kt = k_lane + (t % NBUF) * (BN * KS);
        s[0] = f32x16{};
        s[1] = f32x16{};
        {
            v8 kf[PF];
#pragma unroll
            for (int i = 0; i < PF; ++i) kf[i] = kfrag(kt, i);
#pragma unroll
            for (int i = 0; i < 2 * (D / 16); ++i) {
                const v8 ka = kf[i % PF];
                if (i + PF < 2 * (D / 16)) kf[i % PF] = kfrag(kt, i + PF);
                s[i & 1] = Mfma<T>::mma(ka, qr[i >> 1], s[i & 1]);
            }
            // keep PF fragment reads in flight ahead of the MFMAs
            __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
            for (int i = 0; i < 2 * (D / 16) - PF; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);
        }
    };
    // The rest of tile t on its scores s: mask, running max, P = exp2, and
    // O^T += V^T . P^T.  Lane holds keys k0 + 32*tt + 8*i + 4*hh + j of query
    // qpos.
    auto tile_rest = [&](int t, f32x16* s, bool masked) {
        const lds_ptr vt = v_lane + (t % NBUF) * (D * VT);
        const int k0 = t * BN;
        if (masked) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int key = k0 + 32 * tt + 8 * (e >> 2) + 4 * hh + (e & 3);
                    if (key >= S || (a.causal && key > qpos)) s[tt][e] = -INFINITY;
                }
        }
        float mx = fmaxf(max16(s[0]), max16(s[1]));
        if (__any(mx * c > m_run + kLazy)) {
            mx = wave_max_xor(mx, 32);
            const float m_new = fmaxf(m_run, mx * c);
            const float alpha = fast_exp2(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < D / 32; ++i) o[i] *= alpha;
            m_run = m_new;
        }
        // O^T += V^T . P^T : 4 key steps of 16 x 4 dim tiles of 32; the exps of
        // key step ks+1 overlap the MFMAs of key step ks
        v8 vf[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i) vf[i] = vfrag(vt, i);
        float ls[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int tt = ks >> 1, i0 = 2 * (ks & 1);
            v8 pb;
            float p[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                p[j] = fast_exp2(__builtin_fmaf(s[tt][4 * i0 + j], c, -m_run));
                p[4 + j] = fast_exp2(__builtin_fmaf(s[tt][4 * (i0 + 1) + j], c, -m_run));
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) pb[j] = (T)p[j];
            // row sum of the rounded P that the PV product uses
            ls[ks] = Mfma<T>::sum8(pb);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                const int i = 4 * ks + dt;
                const v8 va = vf[i % PF];
                if (i + PF < 16) vf[i % PF] = vfrag(vt, i + PF);
                o[dt] = Mfma<T>::mma(va, pb, o[dt]);
            }
        }
        l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };

    load_tile(0);
    store_tile(0);
    if (n_tiles > 1) {
        load_tile(1);
        store_tile(1);
    }
    __syncthreads();
    // Two wave groups in opposite phases.  Between two barriers, waves 0-3
    // run QK of tile t and then the softmax + PV of tile t; waves 4-7 run the
    // softmax + PV of tile t-1 (scores kept in registers across the barrier)
    // and then QK of tile t.  Each SIMD holds one wave of each group, so one
    // wave's MFMAs overlap the other's softmax.  Tile t lives in buffer
    // t % 4; the store of tile t+2 goes to the buffer of tile t-2, last read
    // (V by waves 4-7) before the previous barrier.
    // The loop runs one step past the last tile for the lagging group.
    f32x16 s[2];
    const bool lag = wave >= NW / 2;
    for (int t = 0; t <= n_tiles; ++t) {
        const bool pre = t + 2 < n_tiles;
        if (pre) load_tile(t + 2);  // in flight while tile t computes
        if (!lag && t < w_tiles) tile_qk(t, s);
        const int tr = lag ? t - 1 : t;  // tile whose softmax + PV runs now
        if (tr >= 0 && tr < w_tiles) tile_rest(tr, s, tr == w_tiles - 1 && last_masked);
        if (lag && t < w_tiles) tile_qk(t, s);
        if (pre) store_tile((t + 2) % NBUF);
        if (t < n_tiles) __syncthreads();
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
    a.qk_scale = scale * kLog2e;
    // x = workgroup's head set (fastest), y = query block (reversed in the
    // kernel so the heaviest blocks go first); with x = KV head and
    // round-robin dispatch over the 8 XCDs, a KV head's K/V stays in one L2.
    const int hpw = a.group % 4 == 0 ? 4 : (a.group % 2 == 0 ? 2 : 1);
    const int rows = ROWS * 8 / hpw;
    const dim3 grid(n_kv_heads * (a.group / hpw), (seq_len + rows - 1) / rows, batch);
    const bool bf = dtype == 2;
    switch (hpw) {
        case 4:
            if (bf) hipLaunchKernelGGL((prefill_fa_kernel<bf16, 4>), grid, dim3(512), 0, s, a);
            else hipLaunchKernelGGL((prefill_fa_kernel<f16, 4>), grid, dim3(512), 0, s, a);
            break;
        case 2:
            if (bf) hipLaunchKernelGGL((prefill_fa_kernel<bf16, 2>), grid, dim3(512), 0, s, a);
            else hipLaunchKernelGGL((prefill_fa_kernel<f16, 2>), grid, dim3(512), 0, s, a);
            break;
        default:
            if (bf) hipLaunchKernelGGL((prefill_fa_kernel<bf16, 1>), grid, dim3(512), 0, s, a);
            else hipLaunchKernelGGL((prefill_fa_kernel<f16, 1>), grid, dim3(512), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace pi

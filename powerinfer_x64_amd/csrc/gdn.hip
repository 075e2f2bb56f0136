// gdn.hip -- gated-DeltaNet (Qwen3.5 linear attention) kernels for gfx950.
//
// Replaces src/model/mod.rs:796-916 of PowerInfer_x64: the beta/g gates, the
// K->V head tiling (V head vh reads K head vh % n_k_heads), L2 normalisation
// of q and k (q also scaled by 1/sqrt(k_hd)) and the delta-rule recurrence
//   S *= exp(g); kv = S^T k; delta = (v - kv) * beta; S += k delta^T; o = S^T q
// on a per-head fp32 state S[k_hd][v_hd] (row k, v contiguous).
//
// Decode: state columns evolve independently (delta[v] only reads column v),
// so a workgroup owns (sequence, V head, 32 state columns) and streams that
// tile of the state once in and once out (gdn_decode_kernel).
#include "pi_device.hpp"
#include "pi_launch.hpp"

namespace pi {
namespace {

constexpr int DK = 128;
constexpr int DV = 128;

__global__ __launch_bounds__(256) void gdn_gates_kernel(const float* __restrict__ beta_raw,
                                                        const float* __restrict__ a_raw,
                                                        const float* __restrict__ ssm_a,
                                                        const float* __restrict__ dt_bias,
                                                        float* __restrict__ beta,
                                                        float* __restrict__ g, int n_tok,
                                                        int hv) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_tok * hv) return;
    const int h = idx % hv;
    beta[idx] = 1.0f / (1.0f + expf(-beta_raw[idx]));
    const float sp_in = a_raw[idx] + dt_bias[h];
    const float sp = sp_in > 10.0f ? sp_in : logf(1.0f + expf(sp_in));
    g[idx] = ssm_a[h] * sp;
}

// Depthwise causal conv1d + SiLU over the QKV channels (src/model/mod.rs:750-776).
// For sequence s, token t and channel i the window is rows t .. t+d_conv-1 of
// X_ext = [state_s (d_conv-1 rows, oldest first); x_s (n_tok rows)], and
//   out[t][i] = silu(sum_k w[i*d_conv + k] * X_ext[t + k][i]).
// One thread per (s, t, i); channels are the fastest index, so loads coalesce.
__global__ __launch_bounds__(256) void gdn_conv1d_kernel(const float* __restrict__ x,
                                                         const float* __restrict__ state,
                                                         const float* __restrict__ w,
                                                         float* __restrict__ out, int n_seq,
                                                         int n_tok, int conv_dim, int d_conv) {
    const size_t total = (size_t)n_seq * n_tok * conv_dim;
    const int nh = d_conv - 1;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int i = (int)(idx % conv_dim);
        const int t = (int)((idx / conv_dim) % n_tok);
        const int sq = (int)(idx / ((size_t)conv_dim * n_tok));
        const float* xs = x + (size_t)sq * n_tok * conv_dim;
        const float* ss = state + (size_t)sq * nh * conv_dim;
        float val = 0.f;
        for (int k = 0; k < d_conv; ++k) {
            const int r = t + k;  // row of X_ext
            const float v = r < nh ? ss[(size_t)r * conv_dim + i] : xs[(size_t)(r - nh) * conv_dim + i];
            val += w[(size_t)i * d_conv + k] * v;
        }
        out[idx] = val / (1.0f + expf(-val));
    }
}

// The model's case, d_conv = 4 with 4 | conv_dim and 16-byte aligned rows: a
// thread owns channels 4 c4 .. 4 c4 + 3 of one sequence and walks kConvTok
// tokens with the three previous rows of X_ext in registers, so every input
// is read once (16 bytes) and its taps once per thread; the 3-D grid needs no
// index division.  Same arithmetic per element as gdn_conv1d_kernel.
constexpr int kConvTok = 32;
__global__ __launch_bounds__(256) void gdn_conv1d_k4_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ state,
                                                            const float* __restrict__ w,
                                                            float* __restrict__ out, int n_tok,
                                                            int conv_dim) {
    const int c4 = blockIdx.x * 256 + threadIdx.x;
    if (4 * c4 >= conv_dim) return;
    const int t0 = blockIdx.y * kConvTok, sq = blockIdx.z;
    const size_t q4 = (size_t)conv_dim / 4;  // 16-byte groups per row
    const f32x4* xs = reinterpret_cast<const f32x4*>(x + (size_t)sq * n_tok * conv_dim) + c4;
    const f32x4* ss = reinterpret_cast<const f32x4*>(state + (size_t)sq * 3 * conv_dim) + c4;
    f32x4* os = reinterpret_cast<f32x4*>(out + (size_t)sq * n_tok * conv_dim) + c4;
    f32x4 wk[4];  // wk[k][e] = tap k of channel 4 c4 + e
    {
        const f32x4* wr = reinterpret_cast<const f32x4*>(w) + 4 * c4;
        f32x4 wc[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) wc[e] = wr[e];
#pragma unroll
        for (int k = 0; k < 4; ++k) wk[k] = f32x4{wc[0][k], wc[1][k], wc[2][k], wc[3][k]};
    }
    auto ext = [&](int r) { return r < 3 ? ss[(size_t)r * q4] : xs[(size_t)(r - 3) * q4]; };
    f32x4 a = ext(t0), b = ext(t0 + 1), c = ext(t0 + 2);
    const int t1 = min(n_tok, t0 + kConvTok);
    for (int t = t0; t < t1; ++t) {
        const f32x4 d = xs[(size_t)t * q4];  // X_ext row t + 3
        f32x4 val = {0.f, 0.f, 0.f, 0.f};
        val += wk[0] * a;
        val += wk[1] * b;
        val += wk[2] * c;
        val += wk[3] * d;
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = val[e] / (1.0f + expf(-val[e]));
        os[(size_t)t * q4] = o;
        a = b;
        b = c;
        c = d;
    }
}

// New state = the last d_conv-1 rows of X_ext (after gdn_conv1d_kernel has
// read the old one; same stream, next launch).
__global__ __launch_bounds__(256) void gdn_conv_state_kernel(const float* __restrict__ x,
                                                             float* __restrict__ state, int n_seq,
                                                             int n_tok, int conv_dim, int d_conv) {
    const int nh = d_conv - 1;
    const size_t total = (size_t)n_seq * nh * conv_dim;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int i = (int)(idx % conv_dim);
        const int j = (int)((idx / conv_dim) % nh);
        const int sq = (int)(idx / ((size_t)conv_dim * nh));
        float* ss = state + (size_t)sq * nh * conv_dim;
        if (n_tok >= nh) {
            ss[(size_t)j * conv_dim + i] = x[((size_t)sq * n_tok + n_tok - nh + j) * conv_dim + i];
        }
    }
}

// Short prompts (n_tok < d_conv-1): shift the state by n_tok rows in one
// thread per (sequence, channel), so no row is overwritten before it is read.
__global__ __launch_bounds__(256) void gdn_conv_state_shift_kernel(const float* __restrict__ x,
                                                                   float* __restrict__ state,
                                                                   int n_seq, int n_tok,
                                                                   int conv_dim, int d_conv) {
    const int nh = d_conv - 1;
    const size_t total = (size_t)n_seq * conv_dim;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int i = (int)(idx % conv_dim);
        const int sq = (int)(idx / conv_dim);
        float* ss = state + (size_t)sq * nh * conv_dim;
        for (int j = 0; j < nh; ++j) {
            const int r = j + n_tok;  // X_ext row that becomes state row j
            ss[(size_t)j * conv_dim + i] =
                r < nh ? ss[(size_t)r * conv_dim + i] : x[((size_t)sq * n_tok + r - nh) * conv_dim + i];
        }
    }
}

// RMSNormGated (src/model/mod.rs:918-932) in place: for every (row, V head),
// o * (1/sqrt(mean(o^2) + eps)) * w * silu(z).  One wavefront per (row, head).
__global__ __launch_bounds__(256) void gdn_rmsnorm_gated_kernel(float* __restrict__ o,
                                                                const float* __restrict__ z,
                                                                const float* __restrict__ w,
                                                                int n_heads_total, int v_hd,
                                                                float eps) {
    const int lane = threadIdx.x & 63;
    const int hrow = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (hrow >= n_heads_total) return;
    float* oh = o + (size_t)hrow * v_hd;
    const float* zh = z + (size_t)hrow * v_hd;
    if ((v_hd == 128 || v_hd == 64) && (((uintptr_t)oh | (uintptr_t)zh) & 7) == 0) {  // 8-byte accesses (v_hd 128)
        typedef float f2 __attribute__((ext_vector_type(2)));
        const int npl = v_hd / 64;  // values per lane: 2 (one f2) or 1
        float ov[2] = {0.f, 0.f}, zv[2] = {0.f, 0.f};
        if (npl == 2) {
            const f2 a = reinterpret_cast<const f2*>(oh)[lane], b = reinterpret_cast<const f2*>(zh)[lane];
            ov[0] = a[0]; ov[1] = a[1]; zv[0] = b[0]; zv[1] = b[1];
        } else {
            ov[0] = oh[lane];
            zv[0] = zh[lane];
        }
        float sq = ov[0] * ov[0] + ov[1] * ov[1];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) sq = wave_sum_xor(sq, m);
        const float sc = 1.0f / sqrtf(sq / (float)v_hd + eps);
        float r[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int d = npl * lane + e;
            r[e] = e < npl ? (ov[e] * sc * w[d]) * (zv[e] / (1.0f + expf(-zv[e]))) : 0.f;
        }
        if (npl == 2) reinterpret_cast<f2*>(oh)[lane] = f2{r[0], r[1]};
        else oh[lane] = r[0];
        return;
    }
    float ss = 0.f;
    for (int d = lane; d < v_hd; d += 64) ss += oh[d] * oh[d];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss = wave_sum_xor(ss, m);
    const float scale = 1.0f / sqrtf(ss / (float)v_hd + eps);
    for (int d = lane; d < v_hd; d += 64) {
        const float zv = zh[d];
        oh[d] = (oh[d] * scale * w[d]) * (zv / (1.0f + expf(-zv)));
    }
}

// Decode step.  A workgroup owns (sequence, V head, 32 state columns): a
// 128 x 32 tile of the state, 16 KB, whose rows are 128-byte lines.  Thread t
// holds rows t/8 + 32 i (i < 4), columns 4 (t % 8) .. +3, as four 16-byte
// loads issued before anything else, so the step costs one memory round trip.
// Every wavefront computes the q / k norms and k.q itself with shuffles.  The
// readout after the update is o = S'^T q = (gamma S)^T q + delta (k.q), so both
// column sums ((gamma S)^T k and (gamma S)^T q) come from the state as loaded,
// in one reduction: over a wavefront's rows with shuffles and over the 4
// wavefronts in LDS, behind one barrier.
constexpr int DCOLS = 32;  // state columns per decode workgroup

__global__ __launch_bounds__(256) void gdn_decode_kernel(const float* __restrict__ q,
                                                         const float* __restrict__ k,
                                                         const float* __restrict__ v,
                                                         const float* __restrict__ beta,
                                                         const float* __restrict__ g,
                                                         float* __restrict__ state,
                                                         float* __restrict__ out, int hk,
                                                         int hv) {
    __shared__ __attribute__((aligned(16))) float s_part[4][2 * DCOLS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c0 = blockIdx.x * DCOLS;
    const int vh = blockIdx.y, b = blockIdx.z;
    const int kh = vh % hk;  // K head tiled onto this V head (src/model/mod.rs:845-853)
    const int cg = tid & 7, rr = tid >> 3;
    const size_t sh = (size_t)b * hv + vh;
    float* S = state + sh * DK * DV + c0 + 4 * cg;
    f32x4 s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = *reinterpret_cast<const f32x4*>(S + (size_t)(rr + 32 * i) * DV);

    // q / k of the K head, L2-normalised with max(|x|, 1e-12); q also / sqrt(Dk)
    // (src/model/mod.rs:855-875).  Lane l holds rows l and l + 64.
    const float* qr = q + ((size_t)b * hk + kh) * DK;
    const float* kr = k + ((size_t)b * hk + kh) * DK;
    const float q0 = qr[lane], q1 = qr[lane + 64], k0 = kr[lane], k1 = kr[lane + 64];
    const f32x4 vv = *reinterpret_cast<const f32x4*>(v + sh * DV + c0 + 4 * cg);
    const float decay = expf(g[sh]), bt = beta[sh];
    float sq = q0 * q0 + q1 * q1, sk = k0 * k0 + k1 * k1, skq = k0 * q0 + k1 * q1;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        sq = wave_sum_xor(sq, m);
        sk = wave_sum_xor(sk, m);
        skq = wave_sum_xor(skq, m);
    }
    const float inq = 1.0f / fmaxf(sqrtf(sq), 1e-12f) * (1.0f / sqrtf((float)DK));
    const float ink = 1.0f / fmaxf(sqrtf(sk), 1e-12f);
    const float kq = skq * ink * inq;  // (normalised k) . (normalised, scaled q)
    // this thread's rows rr, rr + 32 (first halves) and rr + 64, rr + 96 (second)
    float kn[4], qn[4];
    kn[0] = __shfl(k0, rr, 64) * ink;
    kn[1] = __shfl(k0, rr + 32, 64) * ink;
    kn[2] = __shfl(k1, rr, 64) * ink;
    kn[3] = __shfl(k1, rr + 32, 64) * ink;
    qn[0] = __shfl(q0, rr, 64) * inq;
    qn[1] = __shfl(q0, rr + 32, 64) * inq;
    qn[2] = __shfl(q1, rr, 64) * inq;
    qn[3] = __shfl(q1, rr + 32, 64) * inq;

    // S *= exp(g); kv_mem = S^T k and S^T q of the decayed state (src/model/mod.rs:883-898)
    f32x4 kv = {0.f, 0.f, 0.f, 0.f}, qv = kv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s[i] *= decay;
        kv += s[i] * kn[i];
        qv += s[i] * qn[i];
    }
#pragma unroll
    for (int m = 8; m <= 32; m <<= 1)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            kv[c] = wave_sum_xor(kv[c], m);
            qv[c] = wave_sum_xor(qv[c], m);
        }
    if (lane < 8) {
        *reinterpret_cast<f32x4*>(&s_part[wave][4 * lane]) = kv;
        *reinterpret_cast<f32x4*>(&s_part[wave][DCOLS + 4 * lane]) = qv;
    }
    __syncthreads();
    f32x4 kv_mem = *reinterpret_cast<const f32x4*>(&s_part[0][4 * cg]);
#pragma unroll
    for (int w = 1; w < 4; ++w) kv_mem += *reinterpret_cast<const f32x4*>(&s_part[w][4 * cg]);
    // delta = (v - kv_mem) beta; S += k delta^T (:899-916)
    const f32x4 delta = (vv - kv_mem) * bt;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s[i] += kn[i] * delta;
        *reinterpret_cast<f32x4*>(S + (size_t)(rr + 32 * i) * DV) = s[i];
    }
    // o = S'^T q = (decayed S)^T q + delta (k.q)
    if (tid < 8) {
        f32x4 acc = *reinterpret_cast<const f32x4*>(&s_part[0][DCOLS + 4 * tid]);
#pragma unroll
        for (int w = 1; w < 4; ++w) acc += *reinterpret_cast<const f32x4*>(&s_part[w][DCOLS + 4 * tid]);
        *reinterpret_cast<f32x4*>(out + sh * DV + c0 + 4 * tid) = acc + delta * kq;
    }
}

// One GDN layer step of a single token (src/model/mod.rs:750-932 at n = 1) in
// one launch: conv1d + SiLU (d_conv 4) with the rolling state, the gates, the
// q / k L2 norms, the delta rule and RMSNormGated x SiLU(z), which otherwise
// take five launches.  One workgroup of 512 threads per V head vh (K head
// kh = vh % hk):
//  - it convolves the 128 q and 128 k channels of kh and the 128 v channels
//    of vh itself (a K head's q / k channels are convolved once per V head
//    tiled onto it: 384 channels of 4 taps, a few cycles);
//  - the conv state is read from cs_in and its one-token shift written to
//    cs_out (the layer alternates two buffers), each workgroup copying a
//    1 / hv share of the channels, so no workgroup reads what another writes;
//  - thread t holds state rows t / 32 + 16 i (i < 8), columns 4 (t % 32) ..
//    + 3, loaded before anything else; both column sums ((g S)^T k and
//    (g S)^T q) reduce together over the rows (o = (g S)^T q + delta (k.q),
//    as in gdn_decode_kernel), then wavefront 0 applies RMSNormGated to the
//    head's 128 outputs.
// The arithmetic of each step follows gdn_conv1d_k4_kernel, gdn_gates_kernel,
// gdn_decode_kernel and gdn_rmsnorm_gated_kernel.
__global__ __launch_bounds__(512) void gdn_step_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ cs_in,
                                                       float* __restrict__ cs_out,
                                                       const float* __restrict__ w,
                                                       const float* __restrict__ z,
                                                       const float* __restrict__ beta_raw,
                                                       const float* __restrict__ a_raw,
                                                       const float* __restrict__ ssm_a,
                                                       const float* __restrict__ dt_bias,
                                                       const float* __restrict__ norm_w, float eps,
                                                       float* __restrict__ state,
                                                       float* __restrict__ out, int hk, int hv) {
    __shared__ float s_q[DK], s_k[DK], s_v[DV];
    __shared__ __attribute__((aligned(16))) float s_red[8][2 * DV];  // per wavefront: S^T k | S^T q
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int vh = blockIdx.x, kh = vh % hk;
    const int C = 2 * hk * DK + hv * DV;
    const int cg = tid & 31, rr = tid >> 5;
    float* S = state + (size_t)vh * DK * DV + 4 * cg;
    // The conv inputs of this thread's channel are requested first and the state
    // tile after them, so the conv (which everything else waits for) does not
    // queue behind the tile's 64 KB.  X_ext = [cs_in rows 0..2 (oldest first); x],
    // taps w[c][0..3]; thread t < 384 convolves q (t < 128) or k of kh, or v of vh.
    const int cc = tid < DK ? kh * DK + tid
                 : tid < 2 * DK ? hk * DK + kh * DK + tid - DK
                 : 2 * hk * DK + vh * DV + min(tid - 2 * DK, DV - 1);
    const f32x4 wc = *reinterpret_cast<const f32x4*>(w + (size_t)cc * 4);
    const float x0 = cs_in[cc], x1 = cs_in[C + cc], x2 = cs_in[2 * C + cc], x3 = x[cc];
    // the new conv state for this workgroup's share of the channels (C / hv <= 512 of
    // them at the model's shapes; larger shares loop below) and the gate inputs
    const int c_lo = (int)((long long)vh * C / hv), c_hi = (int)((long long)(vh + 1) * C / hv);
    const int c1 = c_lo + tid;
    float n0 = 0.f, n1 = 0.f, n2 = 0.f;
    if (c1 < c_hi) {
        n0 = cs_in[C + c1];
        n1 = cs_in[2 * C + c1];
        n2 = x[c1];
    }
    const float braw = beta_raw[vh], araw = a_raw[vh], dtb = dt_bias[vh], sa = ssm_a[vh];
    // z and the norm weights of the RMSNormGated (wavefront 0 applies it) load here too
    f32x4 zv = {0.f, 0.f, 0.f, 0.f}, nw = zv;
    if (wave == 0 && lane < 32) {
        zv = *reinterpret_cast<const f32x4*>(z + (size_t)vh * DV + 4 * cg);
        nw = *reinterpret_cast<const f32x4*>(norm_w + 4 * cg);
    }
    f32x4 s[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = *reinterpret_cast<const f32x4*>(S + (size_t)(rr + 16 * i) * DV);
    {
        float val = 0.f;
        val += wc[0] * x0;
        val += wc[1] * x1;
        val += wc[2] * x2;
        val += wc[3] * x3;
        const float act = val / (1.0f + expf(-val));
        if (tid < DK) s_q[tid] = act;
        else if (tid < 2 * DK) s_k[tid - DK] = act;
        else if (tid < 2 * DK + DV) s_v[tid - 2 * DK] = act;
    }
    // the new conv state: rows 1, 2 of the old one and this token
    if (c1 < c_hi) {
        cs_out[c1] = n0;
        cs_out[C + c1] = n1;
        cs_out[2 * C + c1] = n2;
    }
    for (int c = c1 + 512; c < c_hi; c += 512) {
        cs_out[c] = cs_in[C + c];
        cs_out[C + c] = cs_in[2 * C + c];
        cs_out[2 * C + c] = x[c];
    }
    // gates (src/model/mod.rs:806-839)
    const float bt = 1.0f / (1.0f + expf(-braw));
    const float sp_in = araw + dtb;
    const float sp = sp_in > 10.0f ? sp_in : logf(1.0f + expf(sp_in));
    const float decay = expf(sa * sp);
    __syncthreads();

    // L2 norms (max(|x|, 1e-12); q also / sqrt(Dk)) and k.q, in every wavefront
    const float q0 = s_q[lane], q1 = s_q[lane + 64], k0 = s_k[lane], k1 = s_k[lane + 64];
    float sq = q0 * q0 + q1 * q1, sk = k0 * k0 + k1 * k1, skq = k0 * q0 + k1 * q1;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        sq = wave_sum_xor(sq, m);
        sk = wave_sum_xor(sk, m);
        skq = wave_sum_xor(skq, m);
    }
    const float inq = 1.0f / fmaxf(sqrtf(sq), 1e-12f) * (1.0f / sqrtf((float)DK));
    const float ink = 1.0f / fmaxf(sqrtf(sk), 1e-12f);
    const float kq = skq * ink * inq;
    float kn[8];
    f32x4 kv = {0.f, 0.f, 0.f, 0.f}, qv = kv;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        kn[i] = s_k[rr + 16 * i] * ink;
        const float qn = s_q[rr + 16 * i] * inq;
        s[i] *= decay;
        kv += s[i] * kn[i];
        qv += s[i] * qn;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {  // rows rr and rr + 1 of a wavefront: lanes l, l + 32
        kv[c] += __shfl_xor(kv[c], 32, 64);
        qv[c] += __shfl_xor(qv[c], 32, 64);
    }
    if (lane < 32) {
        *reinterpret_cast<f32x4*>(&s_red[wave][4 * cg]) = kv;
        *reinterpret_cast<f32x4*>(&s_red[wave][DV + 4 * cg]) = qv;
    }
    __syncthreads();
    f32x4 kv_mem = *reinterpret_cast<const f32x4*>(&s_red[0][4 * cg]);
#pragma unroll
    for (int wv = 1; wv < 8; ++wv) kv_mem += *reinterpret_cast<const f32x4*>(&s_red[wv][4 * cg]);
    const f32x4 vv = *reinterpret_cast<const f32x4*>(&s_v[4 * cg]);
    const f32x4 delta = (vv - kv_mem) * bt;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        s[i] += kn[i] * delta;
        *reinterpret_cast<f32x4*>(S + (size_t)(rr + 16 * i) * DV) = s[i];
    }
    if (wave == 0 && lane < 32) {
        // o = (decayed S)^T q + delta (k.q); then RMSNormGated over the head's 128 values
        f32x4 o = *reinterpret_cast<const f32x4*>(&s_red[0][DV + 4 * cg]);
#pragma unroll
        for (int wv = 1; wv < 8; ++wv) o += *reinterpret_cast<const f32x4*>(&s_red[wv][DV + 4 * cg]);
        o += delta * kq;
        float ss = o[0] * o[0] + o[1] * o[1] + o[2] * o[2] + o[3] * o[3];
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
        const float sc = 1.0f / sqrtf(ss / (float)DV + eps);
        f32x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = (o[e] * sc * nw[e]) * (zv[e] / (1.0f + expf(-zv[e])));
        *reinterpret_cast<f32x4*>(out + (size_t)vh * DV + 4 * cg) = r;
    }
}

// ---------------------------------------------------------------------------
// Any head widths (k_hd <= 1024, any v_hd): the per-token recurrence of
// src/model/mod.rs:841-916 itself, token after token.  A wavefront owns CG
// state columns of one (sequence, V head): lane (r = lane / CG, c = lane % CG)
// holds rows r + (64 / CG) i (i < NR) of column c0 + c in registers, so every
// column sum (the norms, S^T k, S^T q) is a shuffle over the 64 / CG row groups
// and no wavefront waits for another (CG 8 up to k_hd 256, CG 2 above).  The next token's q, k, v, beta and g are
// loaded while the current one computes.  `stride` is the token pitch of the
// q / k / v / beta / g rows: n_tok consecutive tokens of one sequence
// (prefill), or one token of each of `batch` sequences (decode, n_tok = 1).
// ---------------------------------------------------------------------------
template <int NR, int CG>
__global__ __launch_bounds__(256) void gdn_recur_kernel(const float* __restrict__ q,
                                                        const float* __restrict__ k,
                                                        const float* __restrict__ v,
                                                        const float* __restrict__ beta,
                                                        const float* __restrict__ g,
                                                        float* __restrict__ state,
                                                        float* __restrict__ out, int n_tok,
                                                        int hk, int hv, int dk, int dv) {
    constexpr int RG = 64 / CG;  // row groups
    const int lane = threadIdx.x & 63;
    const int c0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * CG;
    if (c0 >= dv) return;  // a whole wavefront past the last column
    const int vh = blockIdx.y, b = blockIdx.z, kh = vh % hk;
    const int r = lane / CG, col = c0 + lane % CG;
    const bool con = col < dv;
    // token t of this (sequence, V head): rows of q / k at ((b + t) * hk + kh) * dk, ...
    const size_t sh = (size_t)b * hv + vh;
    float* S = state + sh * dk * dv + (con ? col : 0);
    float s[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int row = r + RG * i;
        s[i] = (con && row < dk) ? S[(size_t)row * dv] : 0.f;
    }
    const float qs = 1.0f / sqrtf((float)dk);
    float qn[NR], kn[NR], vx = 0.f, bt = 0.f, gx = 0.f;
    auto fetch = [&](int t) {
        const size_t tok = (size_t)b + t;  // sequence b's token t (one of the two is 0)
        const float* qr = q + (tok * hk + kh) * dk;
        const float* kr = k + (tok * hk + kh) * dk;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int row = r + RG * i;
            qn[i] = row < dk ? qr[row] : 0.f;
            kn[i] = row < dk ? kr[row] : 0.f;
        }
        vx = con ? v[(tok * hv + vh) * dv + col] : 0.f;
        bt = beta[tok * hv + vh];
        gx = g[tok * hv + vh];
    };
    fetch(0);
    for (int t = 0; t < n_tok; ++t) {
        float qc[NR], kc[NR];
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            qc[i] = qn[i];
            kc[i] = kn[i];
            sq += qc[i] * qc[i];
            sk += kc[i] * kc[i];
        }
        const float vc = vx, bc = bt, decay = expf(gx);
        if (t + 1 < n_tok) fetch(t + 1);
#pragma unroll
        for (int m = CG; m <= 32; m <<= 1) {
            sq = wave_sum_xor(sq, m);
            sk = wave_sum_xor(sk, m);
        }
        // L2 norms with max(|x|, 1e-12), q also / sqrt(k_hd) (src/model/mod.rs:855-875)
        const float nq = fmaxf(sqrtf(sq), 1e-12f), nk = fmaxf(sqrtf(sk), 1e-12f);
        // S *= exp(g); kv_mem = S^T k (:883-898)
        float kv = 0.f;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            kc[i] = kc[i] / nk;
            qc[i] = qc[i] / nq * qs;
            s[i] *= decay;
            kv += s[i] * kc[i];
        }
#pragma unroll
        for (int m = CG; m <= 32; m <<= 1) kv = wave_sum_xor(kv, m);
        // delta = (v - kv_mem) beta; S += k delta^T; o = S^T q (:899-916)
        const float delta = (vc - kv) * bc;
        float o = 0.f;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            s[i] += kc[i] * delta;
            o += s[i] * qc[i];
        }
#pragma unroll
        for (int m = CG; m <= 32; m <<= 1) o = wave_sum_xor(o, m);
        if (r == 0 && con) out[(((size_t)b + t) * hv + vh) * dv + col] = o;
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int row = r + RG * i;
        if (con && row < dk) S[(size_t)row * dv] = s[i];
    }
}

// ---------------------------------------------------------------------------
// ssm::ssm_forward (src/ssm/mod.rs:40-157): the Mamba-2-style selective scan of
// one token, which the reference keeps beside the gated-DeltaNet path.  Four
// launches: the conv taps (or the pass-through), one wavefront per row of the
// dt (alpha) and B (beta) projections, one thread per state column for the
// discretised update and its column sum, one wavefront per row of the output
// projection.  Which branches apply follows the reference's slice-length tests
// (has_conv, has_b, has_out), decided on the host.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ssm_conv_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ w, int has_conv,
                                                       float* __restrict__ conv_out, int d_inner,
                                                       int d_conv) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d_inner) return;
    if (has_conv) {  // :63-70, every tap on the current input
        float sum = 0.f;
        for (int t = 0; t < d_conv; ++t) sum += x[i] * w[(size_t)i * d_conv + t];
        conv_out[i] = sum;
    } else {  // :71-74
        conv_out[i] = x[i];
    }
}

// rows [0, d_inner): dt_i = softplus(dt_bias_i + alpha_i . conv_out) with the
// reference's +-20 cut-offs (:85-99); rows [d_inner, d_inner + d_state) when
// has_b: B_s = beta_s . conv_out (:102-110).
__global__ __launch_bounds__(256) void ssm_proj_kernel(const float* __restrict__ conv_out,
                                                       const float* __restrict__ alpha,
                                                       const float* __restrict__ dt_bias,
                                                       const float* __restrict__ beta,
                                                       float* __restrict__ dt, float* __restrict__ bv,
                                                       int n_rows, int d_inner) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n_rows) return;
    const float* wr = row < d_inner ? alpha + (size_t)row * d_inner : beta + (size_t)(row - d_inner) * d_inner;
    float sum = 0.f;
    for (int j = lane; j < d_inner; j += 64) sum += conv_out[j] * wr[j];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) sum = wave_sum_xor(sum, m);
    if (lane != 0) return;
    if (row < d_inner) {
        const float z = dt_bias[row] + sum;
        dt[row] = z > 20.0f ? z : z < -20.0f ? 0.0f : logf(1.0f + expf(z));
    } else {
        bv[row - d_inner] = sum;
    }
}

// state[s][i] = exp(-dt_i exp(A[s][i])) state[s][i] + (dt_i B) conv_out_i with
// B = B_s (has_b) or conv_out_i (:113-128); colsum_i = sum_s state[s][i].
__global__ __launch_bounds__(256) void ssm_scan_kernel(const float* __restrict__ conv_out,
                                                       const float* __restrict__ a,
                                                       const float* __restrict__ dt,
                                                       const float* __restrict__ bv, int has_b,
                                                       float* __restrict__ state,
                                                       float* __restrict__ colsum, int d_inner,
                                                       int d_state) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d_inner) return;
    const float dti = dt[i], ci = conv_out[i];
    float sum = 0.f;
    for (int st = 0; st < d_state; ++st) {
        const size_t idx = (size_t)st * d_inner + i;
        const float a_d = expf(-dti * expf(a[idx]));
        const float b_d = dti * (has_b ? bv[st] : ci);
        const float x = a_d * state[idx] + b_d * ci;
        state[idx] = x;
        sum += x;
    }
    colsum[i] = sum;
}

// has_out: y_j = sum_i colsum_i out[j][i] (:131-145); else y_i = colsum_i (:146-155).
__global__ __launch_bounds__(256) void ssm_out_kernel(const float* __restrict__ colsum,
                                                      const float* __restrict__ w, int has_out,
                                                      float* __restrict__ y, int d_inner) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= d_inner) return;
    if (!has_out) {
        if (lane == 0) y[row] = colsum[row];
        return;
    }
    const float* wr = w + (size_t)row * d_inner;
    float sum = 0.f;
    for (int i = lane; i < d_inner; i += 64) sum += colsum[i] * wr[i];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) sum = wave_sum_xor(sum, m);
    if (lane == 0) y[row] = sum;
}

// ---------------------------------------------------------------------------
// Chunked prefill.  For a chunk of C = 64 tokens of one V head, with q/k
// normalised, gamma_i = exp(lg_i), lg = inclusive cumsum of g over the chunk
// and S the state entering the chunk, the per-token recurrence above equals
//   (I + A) Delta = diag(beta) (V - diag(gamma) K S),
//       A_ij = beta_i exp(lg_i - lg_j) k_i.k_j  (j < i)
//   O = diag(gamma) Q S + M Delta,  M_ij = exp(lg_i - lg_j) q_i.k_j  (j <= i)
//   S' = exp(lg_C) S + K^T diag(exp(lg_C - lg_i)) Delta
// gdn_prep_kernel (parallel over chunks x K heads) builds T = (I + A)^-1, M,
// lg and the q/k inverse norms; gdn_scan_kernel walks the chunks in order for
// one (V head, 16 state columns) with the state tile in LDS.  The prep's
// K K^T and Q K^T tiles run on the f16 MFMA over hi + lo parts, its 16x16
// inverse blocks on the f32 MFMA (v_mfma_f32_16x16x4f32).
// ---------------------------------------------------------------------------
constexpr int GC = 64;          // chunk length
constexpr int KS_ = DK + 4;     // LDS row stride of [64][128] tiles
constexpr int TS_ = GC + 4;     // LDS row stride of [64][64] / [16][64] tiles
constexpr int SCOLS = 16;       // state columns per scan workgroup
// f16 row stride of [rows][128] f16 tiles (288 B): two rows apart differ by two 16-byte
// chunks of LDS banks, so the 16-row x 4-chunk MFMA operand reads are conflict-free
constexpr int KH_ = DK + 16;

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// C += X . Y for 16x16 f32 blocks in LDS (row-major, strides xs / ys).  Lane
// l: A operand X[l%16][k], B operand Y[k][l%16], k = 4s + l/16; returns the
// lane's C[4*(l/16) + r][l%16], r = 0..3.
__device__ __forceinline__ f32x4 mm16(const float* X, int xs, const float* Y, int ys, f32x4 acc) {
    const int l = threadIdx.x & 63, i = l & 15, g = l >> 4;
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = mfma4(X[i * xs + 4 * s + g], Y[(4 * s + g) * ys + i], acc);
    return acc;
}

struct GdnWs {
    f16* q16;   // [n_chunks][Hk][64][128] q / max(|q|,1e-12) / sqrt(Dk), f16
    f16* k16;   // [n_chunks][Hk][64][128] k / max(|k|,1e-12), f16
    float* tm;  // [n_chunks][Hv] (I + A)^-1 as f16 hi [64][64] then f16 lo [64][64]
    float* mm;  // [n_chunks][Hv] M, the same hi / lo form
    float* lg;  // [n_chunks][Hv][64] cumulative log decay
};

// One workgroup of 8 wavefronts per (chunk, K head).  Phase A stages the
// chunk's q and k rows of the K head, L2-normalises them, and forms the lower
// 16x16 tiles of K K^T and Q K^T once; phase B derives, for the V heads tiled
// onto this K head (vh = kh + r * hk, src/model/mod.rs:845-853), two at a time
// (waves 0-3 and 4-7), the decayed
//   A_ij = beta_i exp(lg_i - lg_j) k_i.k_j  (j < i),  M_ij = exp(lg_i - lg_j) q_i.k_j  (j <= i)
// and T = (I + A)^-1.  Phase B reuses the LDS of phase A's q / k rows.
constexpr int PREP_B = 3 * GC * TS_;  // floats of one half's A | T | scratch

__global__ __launch_bounds__(512) void gdn_prep_kernel(const float* __restrict__ q,
                                                       const float* __restrict__ k,
                                                       const float* __restrict__ beta,
                                                       const float* __restrict__ g, int n_tok,
                                                       int hk, int hv, GdnWs w) {
    constexpr int BIG = 2 * PREP_B > 2 * GC * KS_ ? 2 * PREP_B : 2 * GC * KS_;
    __shared__ __attribute__((aligned(16))) float s_big[BIG];   // sk | sq, then 2 x (sa | st | sx)
    __shared__ __attribute__((aligned(16))) float skk[GC * TS_];  // K K^T (lower tiles)
    __shared__ __attribute__((aligned(16))) float sqk[GC * TS_];  // Q K^T (lower tiles)
    __shared__ __attribute__((aligned(16))) float slg[2][GC], sb[2][GC];
    // phase A: the normalised k / q rows as f16 hi + lo parts (row stride KH_
    // halves, 288 bytes: conflict-free 16-byte reads down 16 rows)
    f16* skh = reinterpret_cast<f16*>(s_big);
    f16* skl = skh + GC * KH_;
    f16* sqh = skl + GC * KH_;
    f16* sql = sqh + GC * KH_;
    static_assert(4 * GC * KH_ * 2 <= BIG * 4, "phase A tiles fit s_big");
    const int kh = blockIdx.y;
    const int n_chunks = (n_tok + GC - 1) / GC;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int half = wave >> 2, wl = wave & 3, ht = tid & 255;

    // The workgroup walks chunks blockIdx.x, + gridDim.x, ... of its K head.
    // The next chunk's raw q / k rows (thread t: 16 values of row t / 8,
    // pieces (t % 8) + 8 j) and the g, beta of its first V-head pair (waves 0
    // and 4, lane = token) are loaded into registers while this chunk
    // computes, so their latency hides under the compute.
    const int row = tid >> 3, part = tid & 7;
    f32x4 a[4], b[4];
    float g_nx = 0.f, b_nx = 0.f;
    // part j of the rows: pieces part + 8 j (part 0 also brings g and beta)
    auto fetch = [&](int n, int j) {
        const int t0 = n * GC;
        const int vh = kh + half * hk, tg = min(t0 + lane, n_tok - 1);
        if (j == 0 && wl == 0 && vh < hv) {
            g_nx = g[(size_t)tg * hv + vh];
            b_nx = beta[(size_t)tg * hv + vh];
        }
        const size_t src = ((size_t)min(t0 + row, n_tok - 1) * hk + kh) * DK;
        a[j] = *reinterpret_cast<const f32x4*>(q + src + 4 * (part + 8 * j));
        b[j] = *reinterpret_cast<const f32x4*>(k + src + 4 * (part + 8 * j));
    };
#pragma unroll
    for (int j = 0; j < 4; ++j) fetch(blockIdx.x, j);
    for (int n = blockIdx.x; n < n_chunks; n += gridDim.x) {
    const int t0 = n * GC;
    float g_pre = g_nx, b_pre = b_nx;
    // raw rows of the K head, L2-normalised on the way in (src/model/mod.rs:
    // 860-875); the row sums reduce over 8 lanes.  Rows past the prompt are
    // zero (their inverse norm is then irrelevant).  The normalised rows go
    // to LDS in f32 and to the workspace in f16 for the scan.
    {
        const int t = t0 + row;
        const bool ok = t < n_tok;
        float ssq = 0.f, ssk = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ssq += a[j][e] * a[j][e];
                ssk += b[j][e] * b[j][e];
            }
#pragma unroll
        for (int m = 1; m < 8; m <<= 1) {
            ssq += __shfl_xor(ssq, m, 64);
            ssk += __shfl_xor(ssk, m, 64);
        }
        const float iq = ok ? 1.0f / fmaxf(sqrtf(ssq), 1e-12f) * (1.0f / sqrtf((float)DK)) : 0.f;
        const float ik = ok ? 1.0f / fmaxf(sqrtf(ssk), 1e-12f) : 0.f;
        const size_t base = ((size_t)n * hk + kh) * GC * DK + (size_t)row * DK;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = 4 * (part + 8 * j);
            const f32x4 x = a[j] * iq, y = b[j] * ik;
            f16x4 xh, xl, yh, yl;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                xh[e] = to_f16(x[e]);
                xl[e] = to_f16(x[e] - (float)xh[e]);
                yh[e] = to_f16(y[e]);
                yl[e] = to_f16(y[e] - (float)yh[e]);
            }
            *reinterpret_cast<f16x4*>(sqh + row * KH_ + c) = xh;
            *reinterpret_cast<f16x4*>(sql + row * KH_ + c) = xl;
            *reinterpret_cast<f16x4*>(skh + row * KH_ + c) = yh;
            *reinterpret_cast<f16x4*>(skl + row * KH_ + c) = yl;
            *reinterpret_cast<f16x4*>(w.q16 + base + c) =
                f16x4{to_f16(x[0]), to_f16(x[1]), to_f16(x[2]), to_f16(x[3])};
            *reinterpret_cast<f16x4*>(w.k16 + base + c) =
                f16x4{to_f16(y[0]), to_f16(y[1]), to_f16(y[2]), to_f16(y[3])};
        }
    }
    __syncthreads();
    // lower-triangular 16x16 tiles: 10 of K K^T, then 10 of Q K^T
    const int ln = lane & 15, lg4 = lane >> 4;
    for (int tix = wave; tix < 20; tix += 8) {
        const bool isq = tix >= 10;
        int ib = 0, jb = isq ? tix - 10 : tix;
        while (jb > ib) { jb -= ib + 1; ++ib; }  // enumerate (ib, jb), jb <= ib
        // C = X Y^T over the 128 dims with v_mfma_f32_16x16x32_f16 on hi / lo
        // parts (hi.hi + hi.lo + lo.hi; the lo.lo term is below f32 rounding)
        const f16* xh = (isq ? sqh : skh) + (16 * ib + ln) * KH_ + 8 * lg4;
        const f16* xl = (isq ? sql : skl) + (16 * ib + ln) * KH_ + 8 * lg4;
        const f16* yh = skh + (16 * jb + ln) * KH_ + 8 * lg4;
        const f16* yl = skl + (16 * jb + ln) * KH_ + 8 * lg4;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < DK / 32; ++kb) {
            const f16x8 ah = *reinterpret_cast<const f16x8*>(xh + 32 * kb);
            const f16x8 al = *reinterpret_cast<const f16x8*>(xl + 32 * kb);
            const f16x8 bh = *reinterpret_cast<const f16x8*>(yh + 32 * kb);
            const f16x8 bl = *reinterpret_cast<const f16x8*>(yl + 32 * kb);
            acc = mfma16(ah, bh, acc);
            acc = mfma16(ah, bl, acc);
            acc = mfma16(al, bh, acc);
        }
        float* dst = isq ? sqk : skk;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[(16 * ib + 4 * lg4 + r) * TS_ + 16 * jb + ln] = acc[r];
    }
    __syncthreads();  // q / k rows are dead: s_big now holds two halves of A, T, scratch
    // The next chunk's rows load in quarters, after the barriers that end the
    // cumulative sum, A / M, the diagonal blocks and the first block round:
    // the 64 KB a chunk keep the CU's address unit busy for thousands of
    // cycles, and issued at once (at the end of phase A, or all here) they
    // stalled the issuing wavefronts before the next barrier; ahead of the
    // cumulative sum (one wavefront per half) a quarter still cost ~1 700.
    const bool nxt = n + (int)gridDim.x < n_chunks;

    float* sa = s_big + half * PREP_B;  // A
    float* st = sa + GC * TS_;          // T = (I + A)^-1
    float* sx = st + GC * TS_;          // per-wave 16x16 scratch
    float* hlg = slg[half];
    float* hb = sb[half];
    for (int v0 = kh; v0 < hv; v0 += 2 * hk) {
        const int vh = v0 + half * hk;
        const bool on = vh < hv;  // uniform per half; barriers stay uniform per workgroup
        if (on && wl == 0) {      // inclusive cumsum of g, and beta (0 past the end)
            const int t = t0 + lane;
            if (v0 != kh) {
                const int tc = min(t, n_tok - 1);
                g_pre = g[(size_t)tc * hv + vh];
                b_pre = beta[(size_t)tc * hv + vh];
            }
            float x = t < n_tok ? g_pre : 0.f;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const float y = __shfl_up(x, o, 64);
                if (lane >= o) x += y;
            }
            hlg[lane] = x * kLog2e;  // log2 units for exp2
            hb[lane] = t < n_tok ? b_pre : 0.f;
            w.lg[((size_t)n * hv + vh) * GC + lane] = x;
        }
        __syncthreads();
        if (nxt && v0 == kh) fetch(n + gridDim.x, 0);
        if (on) {
            // thread: row i, columns 4 j4 .. 4 j4 + 3; entries above the
            // diagonal are 0 (and need no exp)
            f16* mm = reinterpret_cast<f16*>(w.mm + ((size_t)n * hv + vh) * GC * GC);
            for (int e = ht; e < GC * GC / 4; e += 256) {
                const int i = e / (GC / 4), j0 = 4 * (e % (GC / 4));
                // branch-free: 16-byte reads of lg and of the K K^T / Q K^T
                // rows, masked by selects (entries above the diagonal, whose
                // tiles were never written, are read and discarded)
                const float li = hlg[i], bi = hb[i];
                const f32x4 lj = *reinterpret_cast<const f32x4*>(hlg + j0);
                const f32x4 kk = *reinterpret_cast<const f32x4*>(skk + i * TS_ + j0);
                const f32x4 qk = *reinterpret_cast<const f32x4*>(sqk + i * TS_ + j0);
                f32x4 av, mv;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int j = j0 + r;
                    const float dec = fast_exp2(li - lj[r]);
                    av[r] = j < i ? bi * dec * kk[r] : 0.f;
                    mv[r] = j <= i ? dec * qk[r] : 0.f;
                }
                *reinterpret_cast<f32x4*>(sa + i * TS_ + j0) = av;
                *reinterpret_cast<f32x4*>(st + i * TS_ + j0) = f32x4{0.f, 0.f, 0.f, 0.f};
                f16x4 mh, ml;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    mh[r] = to_f16(mv[r]);
                    ml[r] = to_f16(mv[r] - (float)mh[r]);
                }
                *reinterpret_cast<f16x4*>(mm + i * GC + j0) = mh;
                *reinterpret_cast<f16x4*>(mm + GC * GC + i * GC + j0) = ml;
            }
        }
        __syncthreads();
        if (nxt && v0 == kh) fetch(n + gridDim.x, 1);
        // T = (I + A)^-1, A strictly lower triangular, by 16x16 blocks:
        //   T_ii = (I + A_ii)^-1                      (forward substitution, wave i)
        //   T_ij = -T_ii . sum_{j <= k < i} A_ik T_kj  (i > j, by block distance)
        if (on && lane < 16) {
            // lane m holds column m of T_ww: t[i] = d_im - sum_{j < i} A[i][j] t[j]
            const float* ab = sa + 16 * wl * TS_ + 16 * wl;
            float tv[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float acc = i == lane ? 1.f : 0.f;
#pragma unroll
                for (int j = 0; j < i; ++j) acc -= ab[i * TS_ + j] * tv[j];
                tv[i] = acc;
                st[(16 * wl + i) * TS_ + 16 * wl + lane] = acc;
            }
        }
        __syncthreads();
        if (nxt && v0 == kh) fetch(n + gridDim.x, 2);
        float* sxw = sx + wl * 16 * TS_;  // this wave's 16x16 scratch
        for (int d = 1; d < 4; ++d) {
            if (d == 2 && nxt && v0 == kh) fetch(n + gridDim.x, 3);
            if (on && wl < 4 - d) {
                const int j = wl, i = wl + d;
                f32x4 x = {0.f, 0.f, 0.f, 0.f};
                for (int kb = j; kb < i; ++kb)
                    x = mm16(sa + 16 * i * TS_ + 16 * kb, TS_, st + 16 * kb * TS_ + 16 * j, TS_, x);
#pragma unroll
                for (int r = 0; r < 4; ++r) sxw[(4 * lg4 + r) * TS_ + ln] = x[r];
                __builtin_amdgcn_wave_barrier();
                f32x4 y = {0.f, 0.f, 0.f, 0.f};
                y = mm16(st + 16 * i * TS_ + 16 * i, TS_, sxw, TS_, y);
#pragma unroll
                for (int r = 0; r < 4; ++r) st[(16 * i + 4 * lg4 + r) * TS_ + 16 * j + ln] = -y[r];
            }
            __syncthreads();
        }
        if (on) {
            f16* tm = reinterpret_cast<f16*>(w.tm + ((size_t)n * hv + vh) * GC * GC);
            for (int e = ht; e < GC * GC / 4; e += 256) {
                const int row = e / (GC / 4), c4 = e % (GC / 4);
                const f32x4 x = *reinterpret_cast<const f32x4*>(st + row * TS_ + 4 * c4);
                f16x4 h, l;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    h[r] = to_f16(x[r]);
                    l[r] = to_f16(x[r] - (float)h[r]);
                }
                *reinterpret_cast<f16x4*>(tm + row * GC + 4 * c4) = h;
                *reinterpret_cast<f16x4*>(tm + GC * GC + row * GC + 4 * c4) = l;
            }
        }
        __syncthreads();  // A, T and the scratch are rewritten for the next V heads
    }
    }  // chunks
}

// gdn_scan_kernel: 8 compute wavefronts walk the chunks in order for one (V
// head, 16 state columns), beside 4 loader wavefronts (data movement, below).
// Waves 0-3 own the K side (K.S, R, Delta) and waves 4-7 the Q side (Q.S, O)
// of chunk row block w % 4; the state update is split over all 8 (16 state
// rows each).  The Q side forms a chunk's O in the next chunk's first phase,
// off the chain from one state to the next.
//
// Precision: the state S stays in f32 in registers (wave w holds rows
// 16w..16w+15 of S^T in the MFMA C layout).  The K.S, Q.S and K^T.Dp
// products run on v_mfma_f32_16x16x32_f16 with q / k rounded once to f16 and
// S^T / Dp split into f16 hi + lo parts (two MFMAs per 32-wide block); with
// normalised q, k this keeps the products within ~1e-5 of f32.  Delta = T.R
// and M.Delta split both operands (three MFMAs per block).
//
// Data movement: chunk n+1's q, k, T and M tiles (64 KB) arrive in the other
// half of a double buffer by direct global -> LDS loads while chunk n
// computes.  Four more wavefronts (8-11) issue them, one tile each, spread
// over the chunk's phases, and wait for them before its last barrier: the 64
// load instructions a chunk takes keep the CU's address unit busy for about
// two thousand cycles, and a compute wave that issued them would stall behind
// that queue on the chunk's dependent chain.  K^T comes from transposing
// reads of the k tile.  The small per-chunk loads are unmasked (clamped), so
// no compiler-inserted wait lands inside a phase.
constexpr int KT_ = GC + 16;  // f16 row stride of the [16][64] R^T, Delta^T tiles (160 B, as KH_)

__global__ __launch_bounds__(768) void gdn_scan_kernel(const float* __restrict__ q,
                                                       const float* __restrict__ k,
                                                       const float* __restrict__ v,
                                                       const float* __restrict__ beta,
                                                       float* __restrict__ state,
                                                       float* __restrict__ out, int n_tok,
                                                       int hk, int hv, GdnWs w) {
    // Chunk tiles, double-buffered, filled by direct global -> LDS loads:
    // q, k [64][128] f16 (256-byte rows, 16-byte chunk c of row r at c ^ (r % 16)),
    // T, M hi + lo [64][64] f16 each (128-byte rows, chunk c of row r at c ^ (r/2 % 8)).
    __shared__ __attribute__((aligned(1024))) f16 sq_[2][GC * DK];
    __shared__ __attribute__((aligned(1024))) f16 sk_[2][GC * DK];
    __shared__ __attribute__((aligned(1024))) f16 st_[2][2 * GC * GC];  // T hi, then lo
    __shared__ __attribute__((aligned(1024))) f16 sm_[2][2 * GC * GC];  // M hi, then lo
    __shared__ __attribute__((aligned(16))) f16 ssh[SCOLS * KH_];   // S^T hi
    __shared__ __attribute__((aligned(16))) f16 ssl[SCOLS * KH_];   // S^T lo
    __shared__ __attribute__((aligned(16))) f16 srth[SCOLS * KT_];  // R^T hi
    __shared__ __attribute__((aligned(16))) f16 srtl[SCOLS * KT_];  // R^T lo
    __shared__ __attribute__((aligned(16))) f16 sdth[SCOLS * KT_];  // Delta^T hi
    __shared__ __attribute__((aligned(16))) f16 sdtl[SCOLS * KT_];  // Delta^T lo
    __shared__ __attribute__((aligned(16))) f16 sdph[SCOLS * KT_];  // (gamma_C/gamma) Delta, ^T, hi
    __shared__ __attribute__((aligned(16))) f16 sdpl[SCOLS * KT_];  // ... lo
    __shared__ float sgam[2][GC], sdec[2][GC], sb[2][GC];  // exp(lg_i), exp(lg_C - lg_i), beta
    // blockIdx.x = tile * hv + vh: with hv a multiple of 8 the tiles of one
    // head share an XCD (and its L2) under round-robin dispatch.
    const int vh = blockIdx.x % hv, tile = blockIdx.x / hv, kh = vh % hk;
    const int c0 = tile * SCOLS;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 15, g4 = lane >> 4;
    const int rb = wave & 3;          // chunk row block of this wave
    const bool kside = wave < 4;      // wave-uniform
    const int row0 = 16 * wave;       // state rows (dims) this wave updates
    const int n_chunks = (n_tok + GC - 1) / GC;
    float* S = state + (size_t)vh * DK * DV;

    // Direct loads (16 bytes per lane; lane i lands at base + 16 i), issued
    // from inline assembly so that the compiler adds no waits before LDS
    // reads; M0 (the LDS destination) is saved and restored.
    typedef __attribute__((address_space(3))) void lds_void;
    auto dma16s = [](const void* base, unsigned voff, lds_void* dst) {
        const unsigned lds = (unsigned)(uintptr_t)dst;
        unsigned saved;
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\t"
                     "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(voff), "s"(base), "s"(lds) : "memory");
    };
    if (wave >= 8) {
        // loader wave: tile lt (0 q, 1 k, 2 T pair, 3 M pair) of every chunk,
        // 16 loads of 1 KB: q / k rows 4 j + lane / 16, T / M rows 8 j +
        // lane / 8 of the [128][64] hi / lo pair
        const int lt = wave - 8;
        unsigned doff[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (lt < 2) {
                const int r = 4 * j + (lane >> 4), c = (lane & 15) ^ (r & 15);
                doff[j] = (unsigned)((r * DK + 8 * c) * 2);
            } else {
                const int r = 8 * j + (lane >> 3), rr = r & 63, c = (lane & 7) ^ ((rr >> 1) & 7);
                doff[j] = (unsigned)(((r >> 6) * GC * GC + rr * GC + 8 * c) * 2);
            }
        }
        auto issue = [&](int n, int j0, int j1) {
            const int b = n & 1;
            const size_t qb = ((size_t)n * hk + kh) * GC * DK;
            const size_t tb = ((size_t)n * hv + vh) * GC * GC * 2;  // f16 elements of a T / M pair
            const f16* tm = reinterpret_cast<const f16*>(w.tm);
            const f16* mm = reinterpret_cast<const f16*>(w.mm);
            const f16* src = lt == 0 ? w.q16 + qb : lt == 1 ? w.k16 + qb : lt == 2 ? tm + tb : mm + tb;
            f16* dst = lt == 0 ? sq_[b] : lt == 1 ? sk_[b] : lt == 2 ? st_[b] : sm_[b];
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (j >= j0 && j < j1) dma16s(src, doff[j], (lds_void*)&dst[512 * j]);
        };
        // The same barriers as the compute waves: one before the chunk loop,
        // three per chunk.  Chunk n+1's buffer held chunk n-1's tiles, last
        // read before chunk n-1's final barrier.  A wave's 16 loads take about
        // a third of a chunk to issue (the CU's address unit is shared by the
        // four loaders), so they are spread over the chunk's three phases
        // instead of holding the first barrier, most of them before the first
        // two so that few remain in flight at the chunk's last barrier.
        // The M tile's buffer holds chunk n-1's M until the Q side has formed
        // that chunk's O in phase 1 of chunk n, so M loads wait for the first
        // barrier.
        const int j1 = lt == 3 ? 0 : 9, j2 = lt == 3 ? 10 : 16;
        issue(0, 0, 16);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        for (int n = 0; n < n_chunks; ++n) {
            const bool more = n + 1 < n_chunks;
            if (more) issue(n + 1, 0, j1);
            __syncthreads();
            if (more) issue(n + 1, j1, j2);
            __syncthreads();
            if (more) issue(n + 1, j2, 16);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
        return;
    }

    // master state: sv[r] = S^T[c = 4 g4 + r][dim = row0 + ln] (MFMA C layout)
    f32x4 sv;
#pragma unroll
    for (int r = 0; r < 4; ++r) sv[r] = S[(size_t)(row0 + ln) * DV + c0 + 4 * g4 + r];
    auto put_state = [&]() {  // S^T hi / lo parts for the next K.S, Q.S
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const f16 h = to_f16(sv[r]);
            ssh[(4 * g4 + r) * KH_ + row0 + ln] = h;
            ssl[(4 * g4 + r) * KH_ + row0 + ln] = to_f16(sv[r] - (float)h);
        }
    };
    put_state();

    // V tile (K-side waves, MFMA C layout: rows 16 rb + 4 g4 + r, column ln), lg and beta
    float pv[4], plg = 0.f, plc = 0.f, pb = 0.f;
    bool pbm = false;
    // Rows past the prompt reload the last token (finite values; their beta
    // is 0, so R = 0 there); no lane is masked, so no load waits on another.
    auto fetch_small = [&](int n) {
        const int t0 = n * GC;
        if (kside) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = min(t0 + 16 * rb + 4 * g4 + r, n_tok - 1);
                pv[r] = v[((size_t)t * hv + vh) * DV + c0 + ln];
            }
        }
        if (wave == 0) {
            const int tl = min(lane, GC - 1);
            plg = w.lg[((size_t)n * hv + vh) * GC + tl];
            plc = w.lg[((size_t)n * hv + vh) * GC + GC - 1];
            const int t = t0 + tl;
            pb = beta[(size_t)min(t, n_tok - 1) * hv + vh];  // masked in stage_small
            pbm = t < n_tok;
        }
    };
    auto stage_small = [&](int n) {
        if (wave == 0) {
            sgam[n & 1][tid] = expf(plg);
            sdec[n & 1][tid] = expf(plc - plg);
            sb[n & 1][tid] = pbm ? pb : 0.f;
        }
    };
    // A-operand tile reads (row r, 8 elements at column 8 c)
    auto frag_qk = [&](const f16* t, int r, int c) {
        return *reinterpret_cast<const f16x8*>(t + r * DK + 8 * (c ^ (r & 15)));
    };
    auto frag_tm = [&](const f16* t, int r, int c) {
        return *reinterpret_cast<const f16x8*>(t + r * GC + 8 * (c ^ ((r >> 1) & 7)));
    };
    // C[16 x 16] = X[row0 .. +15][0 .. 32 nkb) . Y^T with X (swizzled [64][64]
    // hi, lo) and Y^T ([16][64] hi, lo, row stride KT_): hi.hi + hi.lo + lo.hi
    auto mm_split_sw = [&](const f16* xh, const f16* xl, const f16* yh, const f16* yl, int r0,
                           int nkb) {
        // two accumulation chains (hi.hi + lo.hi, hi.lo) halve the dependent MFMA run
        f32x4 c = {0.f, 0.f, 0.f, 0.f}, d = c;
        for (int kb = 0; kb < nkb; ++kb) {
            const f16x8 ah = frag_tm(xh, r0 + ln, 4 * kb + g4);
            const f16x8 al = frag_tm(xl, r0 + ln, 4 * kb + g4);
            const f16x8 bh = *reinterpret_cast<const f16x8*>(yh + ln * KT_ + 8 * g4 + 32 * kb);
            const f16x8 bl = *reinterpret_cast<const f16x8*>(yl + ln * KT_ + 8 * g4 + 32 * kb);
            c = mfma16(ah, bh, c);
            d = mfma16(ah, bl, d);
            c = mfma16(al, bh, c);
        }
        return c + d;
    };
    // K^T operand of the state update by two transposing reads: in each
    // 16-lane group, lane j points at token kb0 + j/4, dims row0 + 4 (j % 4)
    // .. +3; lane i then holds tokens kb0 .. kb0+3 of dim row0 + i.
    typedef short s4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s4* lds_s4;
    typedef f16 f16x4_ __attribute__((ext_vector_type(4)));
    auto frag_kt = [&](const f16* kt, int kb) {  // tokens 32 kb + 8 g4 .. +7, dim row0 + ln
        f16x8 res;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int tok = 32 * kb + 8 * g4 + 4 * h + (ln >> 2);
            const int dim = row0 + 4 * (ln & 3);
            const int c = (dim >> 3) ^ (tok & 15);
            const f16* p = kt + tok * DK + 8 * c + (dim & 7);
            const s4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(p));
            const f16x4_ y = __builtin_bit_cast(f16x4_, x);
#pragma unroll
            for (int e = 0; e < 4; ++e) res[4 * h + e] = y[e];
        }
        return res;
    };

    float vcur[4] = {0.f, 0.f, 0.f, 0.f};
    // O of a chunk (Q-side waves) is formed in phase 1 of the next chunk, off
    // the chain from one state to the next, and stored in that chunk's phase 2
    float opend[4] = {0.f, 0.f, 0.f, 0.f};
    f32x4 xprev = {0.f, 0.f, 0.f, 0.f};  // Q S of the previous chunk
    auto form_o = [&](int cp) {  // O = gamma Q S + M Delta of the chunk in buffer cp
        const f32x4 o = mm_split_sw(sm_[cp], sm_[cp] + GC * GC, sdth, sdtl, 16 * rb, (rb >> 1) + 1);
#pragma unroll
        for (int r = 0; r < 4; ++r) opend[r] = sgam[cp][16 * rb + 4 * g4 + r] * xprev[r] + o[r];
    };
    auto store_o = [&](int tp) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = tp + 16 * rb + 4 * g4 + r;
            if (t < n_tok) out[((size_t)t * hv + vh) * DV + c0 + ln] = opend[r];
        }
    };
    fetch_small(0);
    __builtin_amdgcn_s_waitcnt(0);
    stage_small(0);
#pragma unroll
    for (int r = 0; r < 4; ++r) vcur[r] = pv[r];
    __syncthreads();
    for (int n = 0; n < n_chunks; ++n) {
        const int t0 = n * GC, cb = n & 1;
        if (n + 1 < n_chunks) fetch_small(n + 1);
        const f16* tq = sq_[cb];
        const f16* tk = sk_[cb];
        const float gC = sgam[cb][GC - 1];
        // phase 1: O of chunk n-1 (waves 4-7, from Delta^T and M still in
        // place), then K.S (waves 0-3) or Q.S (waves 4-7), rows 16 rb ..
        if (!kside && n >= 1) form_o(cb ^ 1);
        f32x4 xs;
        {
            const f16* xt = kside ? tk : tq;
            const f16* sh = ssh + ln * KH_ + 8 * g4;
            const f16* sl = ssl + ln * KH_ + 8 * g4;
            f32x4 xa = {0.f, 0.f, 0.f, 0.f}, xb = xa;  // S^T hi / lo chains
#pragma unroll
            for (int kb = 0; kb < DK / 32; ++kb) {
                const f16x8 a = frag_qk(xt, 16 * rb + ln, 4 * kb + g4);
                xa = mfma16(a, *reinterpret_cast<const f16x8*>(sh + 32 * kb), xa);
                xb = mfma16(a, *reinterpret_cast<const f16x8*>(sl + 32 * kb), xb);
            }
            xs = xa + xb;
        }
        if (kside) {  // R = beta (V - gamma KS), written transposed as hi / lo
            f16x4 rh, rl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * rb + 4 * g4 + r;
                const float rv = sb[cb][i] * (vcur[r] - sgam[cb][i] * xs[r]);
                rh[r] = to_f16(rv);
                rl[r] = to_f16(rv - (float)rh[r]);
            }
            *reinterpret_cast<f16x4*>(srth + ln * KT_ + 16 * rb + 4 * g4) = rh;
            *reinterpret_cast<f16x4*>(srtl + ln * KT_ + 16 * rb + 4 * g4) = rl;
        }
        __syncthreads();
        if (!kside && n >= 1) store_o(t0 - GC);
        // phase 2: Delta = T R (T lower triangular: column blocks <= rb)
        if (kside) {
            const f32x4 dl = mm_split_sw(st_[cb], st_[cb] + GC * GC, srth, srtl, 16 * rb, (rb >> 1) + 1);
            f16x4 dh, dlo, ph, pl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * rb + 4 * g4 + r;
                dh[r] = to_f16(dl[r]);
                dlo[r] = to_f16(dl[r] - (float)dh[r]);
                const float dp = sdec[cb][i] * dl[r];
                ph[r] = to_f16(dp);
                pl[r] = to_f16(dp - (float)ph[r]);
            }
            *reinterpret_cast<f16x4*>(sdth + ln * KT_ + 16 * rb + 4 * g4) = dh;
            *reinterpret_cast<f16x4*>(sdtl + ln * KT_ + 16 * rb + 4 * g4) = dlo;
            *reinterpret_cast<f16x4*>(sdph + ln * KT_ + 16 * rb + 4 * g4) = ph;
            *reinterpret_cast<f16x4*>(sdpl + ln * KT_ + 16 * rb + 4 * g4) = pl;
        }
        __syncthreads();
        // phase 3: S'^T = exp(lgC) S^T + Dp^T K for state rows row0 .. row0 + 15
        {
            f32x4 acc = sv * gC, acl = {0.f, 0.f, 0.f, 0.f};
            const f16* ah = sdph + ln * KT_ + 8 * g4;
            const f16* al = sdpl + ln * KT_ + 8 * g4;
#pragma unroll
            for (int kb = 0; kb < GC / 32; ++kb) {
                const f16x8 b = frag_kt(tk, kb);
                acc = mfma16(*reinterpret_cast<const f16x8*>(ah + 32 * kb), b, acc);
                acl = mfma16(*reinterpret_cast<const f16x8*>(al + 32 * kb), b, acl);
            }
            sv = acc + acl;
        }
        if (!kside) xprev = xs;
        // S^T hi / lo were last read in phase 1 (before two barriers)
        put_state();
        // chunk n+1's small loads are waited for by the compiler where they are
        // used (below); the Q side, which issued only output stores, waits for none
        if (n + 1 < n_chunks) {
            stage_small(n + 1);
#pragma unroll
            for (int r = 0; r < 4; ++r) vcur[r] = pv[r];
        }
        __syncthreads();
    }
    if (!kside && n_chunks >= 1) {  // the last chunk's O
        form_o((n_chunks - 1) & 1);
        store_o((n_chunks - 1) * GC);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) S[(size_t)(row0 + ln) * DV + c0 + 4 * g4 + r] = sv[r];
}

}  // namespace

hipError_t launch_gdn_gates(const float* beta_raw, const float* a_raw, const float* ssm_a,
                            const float* dt_bias, float* beta, float* g, int32_t n_tok,
                            int32_t n_v_heads, hipStream_t s) {
    const int n = n_tok * n_v_heads;
    hipLaunchKernelGGL(gdn_gates_kernel, dim3((n + 255) / 256), dim3(256), 0, s, beta_raw, a_raw,
                       ssm_a, dt_bias, beta, g, n_tok, n_v_heads);
    return hipGetLastError();
}

static int grid_of(size_t total) {
    size_t b = (total + 255) / 256;
    return (int)(b > 65536 ? 65536 : (b == 0 ? 1 : b));
}

hipError_t launch_gdn_conv1d(const float* x, float* state, const float* w, float* out,
                             int32_t n_seq, int32_t n_tok, int32_t conv_dim, int32_t d_conv,
                             hipStream_t s) {
    const size_t total = (size_t)n_seq * n_tok * conv_dim;
    const bool aligned =
        (((uintptr_t)x | (uintptr_t)state | (uintptr_t)w | (uintptr_t)out) & 15) == 0;
    if (d_conv == 4 && conv_dim % 4 == 0 && aligned && n_seq <= 65535)
        hipLaunchKernelGGL(gdn_conv1d_k4_kernel,
                           dim3((unsigned)((conv_dim / 4 + 255) / 256), (unsigned)((n_tok + kConvTok - 1) / kConvTok),
                                (unsigned)n_seq),
                           dim3(256), 0, s, x, state, w, out, n_tok, conv_dim);
    else
        hipLaunchKernelGGL(gdn_conv1d_kernel, dim3(grid_of(total)), dim3(256), 0, s, x, state, w,
                           out, n_seq, n_tok, conv_dim, d_conv);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || d_conv < 2) return e;
    if (n_tok >= d_conv - 1)
        hipLaunchKernelGGL(gdn_conv_state_kernel, dim3(grid_of((size_t)n_seq * (d_conv - 1) * conv_dim)),
                           dim3(256), 0, s, x, state, n_seq, n_tok, conv_dim, d_conv);
    else
        hipLaunchKernelGGL(gdn_conv_state_shift_kernel, dim3(grid_of((size_t)n_seq * conv_dim)),
                           dim3(256), 0, s, x, state, n_seq, n_tok, conv_dim, d_conv);
    return hipGetLastError();
}

hipError_t launch_gdn_rmsnorm_gated(float* o, const float* z, const float* w, int32_t n_rows,
                                    int32_t n_v_heads, int32_t v_hd, float eps, hipStream_t s) {
    const int n = n_rows * n_v_heads;
    hipLaunchKernelGGL(gdn_rmsnorm_gated_kernel, dim3((n + 3) / 4), dim3(256), 0, s, o, z, w, n,
                       v_hd, eps);
    return hipGetLastError();
}

hipError_t launch_gdn_recur(const float* q, const float* k, const float* v, const float* beta,
                            const float* g, float* state, float* out, int32_t batch, int32_t n_tok,
                            int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd, int32_t v_hd,
                            hipStream_t s) {
    if (k_hd <= 0 || k_hd > kGdnMaxKhd || v_hd <= 0 || (batch > 1 && n_tok != 1))
        return hipErrorInvalidValue;
    // 8 columns per wavefront (8 row groups) up to k_hd 256, then 2 (32 row groups)
    const int cg = k_hd <= 256 ? 8 : 2;
    const dim3 grid((unsigned)((v_hd + 4 * cg - 1) / (4 * cg)), (unsigned)n_v_heads, (unsigned)batch);
    const int nr = (k_hd + 64 / cg - 1) / (64 / cg);
#define PI_GDN_RECUR(N, C)                                                                           \
    hipLaunchKernelGGL((gdn_recur_kernel<N, C>), grid, dim3(256), 0, s, q, k, v, beta, g, state, out, \
                       n_tok, n_k_heads, n_v_heads, k_hd, v_hd)
    if (cg == 2) {
        if (nr <= 16) PI_GDN_RECUR(16, 2);
        else PI_GDN_RECUR(32, 2);
    } else if (nr <= 4) PI_GDN_RECUR(4, 8);
    else if (nr <= 8) PI_GDN_RECUR(8, 8);
    else if (nr <= 16) PI_GDN_RECUR(16, 8);
    else PI_GDN_RECUR(32, 8);
#undef PI_GDN_RECUR
    return hipGetLastError();
}

hipError_t launch_gdn_step(const float* x, const float* cs_in, float* cs_out, const float* w,
                           const float* z, const float* beta_raw, const float* a_raw,
                           const float* ssm_a, const float* dt_bias, const float* norm_w, float eps,
                           float* state, float* out, int32_t n_k_heads, int32_t n_v_heads,
                           hipStream_t s) {
    if (n_k_heads <= 0 || n_v_heads <= 0) return hipErrorInvalidValue;
    // f32x4 accesses: conv taps (4 per channel), z / norm / out rows of 128
    if (((uintptr_t)w | (uintptr_t)z | (uintptr_t)norm_w | (uintptr_t)out | (uintptr_t)state) & 15)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gdn_step_kernel, dim3(n_v_heads), dim3(512), 0, s, x, cs_in, cs_out, w, z,
                       beta_raw, a_raw, ssm_a, dt_bias, norm_w, eps, state, out, n_k_heads, n_v_heads);
    return hipGetLastError();
}

hipError_t launch_gdn_decode(const float* q, const float* k, const float* v, const float* beta,
                             const float* g, float* state, float* out, int32_t batch,
                             int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd, int32_t v_hd,
                             hipStream_t s) {
    if (k_hd != DK || v_hd != DV)
        return launch_gdn_recur(q, k, v, beta, g, state, out, batch, 1, n_k_heads, n_v_heads, k_hd,
                                v_hd, s);
    hipLaunchKernelGGL(gdn_decode_kernel, dim3(DV / DCOLS, n_v_heads, batch), dim3(256), 0, s, q, k,
                       v, beta, g, state, out, n_k_heads, n_v_heads);
    return hipGetLastError();
}

hipError_t launch_ssm_forward(const SsmArgs& a, hipStream_t s) {
    if (a.d_inner <= 0 || a.d_state < 0 || a.d_conv < 0) return hipErrorInvalidValue;
    const unsigned g1 = (unsigned)((a.d_inner + 255) / 256);
    hipLaunchKernelGGL(ssm_conv_kernel, dim3(g1), dim3(256), 0, s, a.x, a.conv_w, a.has_conv,
                       a.conv_out, a.d_inner, a.d_conv);
    const int n_rows = a.d_inner + (a.has_b ? a.d_state : 0);
    hipLaunchKernelGGL(ssm_proj_kernel, dim3((unsigned)((n_rows + 3) / 4)), dim3(256), 0, s,
                       a.conv_out, a.alpha, a.dt_bias, a.beta, a.dt, a.bv, n_rows, a.d_inner);
    hipLaunchKernelGGL(ssm_scan_kernel, dim3(g1), dim3(256), 0, s, a.conv_out, a.a, a.dt, a.bv,
                       a.has_b, a.state, a.colsum, a.d_inner, a.d_state);
    hipLaunchKernelGGL(ssm_out_kernel, dim3((unsigned)((a.d_inner + 3) / 4)), dim3(256), 0, s,
                       a.colsum, a.out_w, a.has_out, a.y, a.d_inner);
    return hipGetLastError();
}

size_t gdn_prefill_ws_floats(int32_t n_tok, int32_t n_k_heads, int32_t n_v_heads, int32_t chunk) {
    const size_t nc = (size_t)(n_tok + chunk - 1) / chunk;
    // two f16 [64][128] tiles (q, k) per (chunk, K head) = 8192 floats
    return nc * n_k_heads * GC * DK + 2 * nc * n_v_heads * GC * GC + nc * n_v_heads * GC;
}

hipError_t launch_gdn_prefill(const float* q, const float* k, const float* v, const float* beta,
                              const float* g, float* state, float* out, int32_t n_tok,
                              int32_t n_k_heads, int32_t n_v_heads, int32_t chunk,
                              const GdnWorkspace& ws, hipStream_t s) {
    if (chunk != GC) return hipErrorInvalidValue;
    if (n_tok <= 0) return hipSuccess;  // the kernels clamp token indices to n_tok - 1
    const size_t nc = (size_t)(n_tok + GC - 1) / GC;
    GdnWs w;
    const size_t qk = nc * n_k_heads * GC * DK;  // f16 elements of one of q16 / k16
    w.q16 = reinterpret_cast<f16*>(ws.buf);
    w.k16 = w.q16 + qk;
    w.tm = reinterpret_cast<float*>(w.k16 + qk);
    w.mm = w.tm + nc * n_v_heads * GC * GC;
    w.lg = w.mm + nc * n_v_heads * GC * GC;
    // about one prep workgroup per CU: each walks nc / grid chunks of its K head
    int dev = 0, n_cu = 0;
    hipError_t e0 = hipGetDevice(&dev);
    if (e0 == hipSuccess) e0 = hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
    if (e0 != hipSuccess) return e0;
    const unsigned gx = (unsigned)std::max<size_t>(1, std::min<size_t>(nc, (size_t)n_cu / n_k_heads));
    hipLaunchKernelGGL(gdn_prep_kernel, dim3(gx, n_k_heads), dim3(512), 0, s, q, k, beta, g,
                       n_tok, n_k_heads, n_v_heads, w);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gdn_scan_kernel, dim3(n_v_heads * (DV / SCOLS)), dim3(768), 0, s, q, k, v,
                       beta, state, out, n_tok, n_k_heads, n_v_heads, w);
    return hipGetLastError();
}

}  // namespace pi

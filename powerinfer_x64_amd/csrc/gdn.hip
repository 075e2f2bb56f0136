// gdn.hip -- gated-DeltaNet (Qwen3.5 linear attention) kernels for gfx950.
//
// Replaces src/model/mod.rs:796-916 of PowerInfer_x64: the beta/g gates, the
// K->V head tiling (V head vh reads K head vh % n_k_heads), L2 normalisation
// of q and k (q also scaled by 1/sqrt(k_hd)) and the delta-rule recurrence
//   S *= exp(g); kv = S^T k; delta = (v - kv) * beta; S += k delta^T; o = S^T q
// on a per-head fp32 state S[k_hd][v_hd] (row k, v contiguous).
//
// Decode: state columns evolve independently (delta[v] only reads column v),
// so a workgroup owns (sequence, V head, 32 state columns): 8 row groups of
// 32 lanes; each thread keeps 16 state values in registers, and the two
// column sums (S^T k and S^T q) are reduced across the row groups in LDS.
#include "pi_device.hpp"
#include "pi_launch.hpp"

namespace pi {
namespace {

constexpr int DK = 128;
constexpr int DV = 128;
constexpr int COLS = 32;             // state columns per decode workgroup
constexpr int RG = 256 / COLS;       // row groups (8)
constexpr int RPT = DK / RG;         // state rows per thread (16)

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

// Block-wide sum of one value per thread; all threads get the result.
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = wave_sum_xor(v, m);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(256) void gdn_decode_kernel(const float* __restrict__ q,
                                                         const float* __restrict__ k,
                                                         const float* __restrict__ v,
                                                         const float* __restrict__ beta,
                                                         const float* __restrict__ g,
                                                         float* __restrict__ state,
                                                         float* __restrict__ out, int hk,
                                                         int hv) {
    __shared__ float s_q[DK], s_k[DK];
    __shared__ float s_red[4];
    __shared__ float s_part[2][RG][COLS];
    const int tid = threadIdx.x;
    const int c0 = blockIdx.x * COLS;
    const int vh = blockIdx.y;
    const int b = blockIdx.z;
    const int kh = vh % hk;

    // q/k of the tiled K head, L2-normalised (src/model/mod.rs:855-875)
    const float* qr = q + ((size_t)b * hk + kh) * DK;
    const float* kr = k + ((size_t)b * hk + kh) * DK;
    const float xq = tid < DK ? qr[tid] : 0.f;
    const float xk = tid < DK ? kr[tid] : 0.f;
    const float nq = fmaxf(sqrtf(block_sum(xq * xq, s_red)), 1e-12f);
    const float nk = fmaxf(sqrtf(block_sum(xk * xk, s_red)), 1e-12f);
    if (tid < DK) {
        s_q[tid] = xq / nq * (1.0f / sqrtf((float)DK));
        s_k[tid] = xk / nk;
    }
    __syncthreads();

    const int c = tid % COLS, rg = tid / COLS;
    const size_t sh = ((size_t)b * hv + vh);
    float* S = state + sh * DK * DV + c0 + c;
    const float decay = expf(g[sh]);
    float s[RPT];
    float kv = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const int row = rg * RPT + i;
        s[i] = S[(size_t)row * DV] * decay;
        kv += s[i] * s_k[row];
    }
    s_part[0][rg][c] = kv;
    __syncthreads();
    float kv_mem = 0.f;
#pragma unroll
    for (int r = 0; r < RG; ++r) kv_mem += s_part[0][r][c];
    const float delta = (v[sh * DV + c0 + c] - kv_mem) * beta[sh];
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const int row = rg * RPT + i;
        s[i] += s_k[row] * delta;
        o += s[i] * s_q[row];
        S[(size_t)row * DV] = s[i];
    }
    s_part[1][rg][c] = o;
    __syncthreads();
    if (rg == 0) {
        float acc = 0.f;
#pragma unroll
        for (int r = 0; r < RG; ++r) acc += s_part[1][r][c];
        out[sh * DV + c0 + c] = acc;
    }
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

hipError_t launch_gdn_decode(const float* q, const float* k, const float* v, const float* beta,
                             const float* g, float* state, float* out, int32_t batch,
                             int32_t n_k_heads, int32_t n_v_heads, hipStream_t s) {
    hipLaunchKernelGGL(gdn_decode_kernel, dim3(DV / COLS, n_v_heads, batch), dim3(256), 0, s, q, k,
                       v, beta, g, state, out, n_k_heads, n_v_heads);
    return hipGetLastError();
}

size_t gdn_prefill_ws_floats(int32_t, int32_t, int32_t) { return 0; }

hipError_t launch_gdn_prefill(const float*, const float*, const float*, const float*,
                              const float*, float*, float*, int32_t, int32_t, int32_t, int32_t,
                              const GdnWorkspace&, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace pi

// api.cpp -- the C ABI (include/pi_attn.h): handles, the paged KV pool,
// argument validation, error reporting and dispatch to the gfx950 kernels.
//
// Error behaviour mirrors the reference's offload seam: every failure is a
// status code plus text (Some(Err(String)) in src/cuda/mod.rs:527-537), never
// an exception or an abort across the ABI.
#include "pi_attn.h"
#include "pi_launch.hpp"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <new>
#include <string>
#include <vector>

struct pi_handle_s {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    pi::DecodeWorkspace dws{};
    pi::GdnWorkspace gws{};
    float* h2d_scratch = nullptr;  // device staging for the host-slice drop-ins
    size_t h2d_floats = 0;
    float* tq_qv = nullptr;        // TurboQuant virtual queries [batch][Hq][2 head_dim]
    size_t tq_qv_floats = 0;
    float* tq_sc = nullptr;        // TurboQuant scores of the in-order decode [batch][Hq][keys]
    size_t tq_sc_floats = 0;
    float* pfs_buf = nullptr;      // prefill key-split partials
    size_t pfs_floats = 0;
    float* pad_buf = nullptr;      // pi_attn_prefill's padded rows at a head_dim of no kernel
    size_t pad_floats = 0;
    float* pin = nullptr;          // pinned host staging of the small host-slice layer calls
    size_t pin_floats = 0;
    // Ordering of the workspaces above across caller streams: ws_event marks
    // the last workspace use, issued on ws_stream.
    hipEvent_t ws_event = nullptr;
    hipStream_t ws_stream = nullptr;
    bool ws_used = false;
    float* scratch = nullptr;      // this device's fixed scratch (pi_attn_decode_noalloc)
};

struct pi_kv_pool_s {
    pi_handle owner;
    pi::KvGeom g;
    size_t bytes;
};

struct pi_attn_layer_s {
    pi_handle owner;
    pi_kv_pool pool = nullptr;      // max_pages pages, page i at physical page i
    int32_t max_pages = 0, n_heads = 0, n_kv = 0, dim = 0, kv_dtype = 0;
    int32_t q_dim = 0, v_dim = 0;   // query / value head widths (dim: the key head width)
    int32_t pdim = 0;               // the step's row width: the smallest of 64 / 128 / 256 >= dim
    int32_t rope_dim = 0, gqa_mode = 0;
    float eps = 0.f, rope_base = 0.f;
    int32_t sections[4] = {0, 0, 0, 0};
    bool has_sections = false;
    float* d_qn = nullptr;          // per-head RMSNorm weights (null: no norm)
    float* d_kn = nullptr;
    int32_t* d_pt = nullptr;        // kLayerRows identical rows of the identity page table
    int32_t* d_ctx = nullptr;       // the start position, then per-row context lengths (kLayerRows + 1)
    float* d_buf = nullptr;         // host-slice staging: q, gate, out, k, v (f32)
    size_t buf_floats = 0;
    int32_t seq_len = 0;
};

struct pi_gdn_layer_s {
    pi_handle owner;
    int32_t hk = 0, hv = 0, dk = 0, dv = 0, d_conv = 0, conv_dim = 0;
    float eps = 0.f;
    float* d_w = nullptr;       // conv1d weights [conv_dim][d_conv]
    float* d_ssm_a = nullptr;   // [hv]
    float* d_dt = nullptr;      // [hv]
    float* d_norm = nullptr;    // [dv]
    float* d_conv_state = nullptr;  // [d_conv - 1][conv_dim]
    float* d_conv_alt = nullptr;    // the one-launch step's second conv state (swapped each step)
    float* d_state = nullptr;       // [hv][dk][dv]
    float* d_buf = nullptr;         // staging: activation, q, k, v, beta, g (+ host-slice I/O)
    size_t buf_floats = 0;
};

struct pi_tq_pool_s {
    pi_handle owner;
    pi::TqPool t;
    size_t bytes;
};

namespace {

thread_local std::string g_create_err;

int fail(pi_handle h, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (h)
        h->err = buf;
    else
        g_create_err = buf;
    return code;
}

int hip_fail(pi_handle h, hipError_t e, const char* what) {
    if (e == hipErrorOutOfMemory)
        return fail(h, PI_ERR_OUT_OF_MEMORY, "%s: out of device memory", what);
    if (e == hipErrorInvalidDeviceFunction || e == hipErrorNoBinaryForGpu)
        return fail(h, PI_ERR_INVALID_KERNEL, "%s: no gfx950 kernel for this device (%s)", what,
                    hipGetErrorString(e));
    return fail(h, PI_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

#define PI_CHECK_HANDLE(h)                                                     \
    do {                                                                       \
        if (!(h)) return fail(nullptr, PI_ERR_INVALID_ARG, "null pi_handle");  \
    } while (0)

#define PI_HIP(h, call, what)                       \
    do {                                            \
        hipError_t e_ = (call);                     \
        if (e_ != hipSuccess) return hip_fail(h, e_, what); \
    } while (0)

// NULL is HIP's default (null) stream, as for every HIP API; work is then
// ordered with everything else the caller issues on that stream.
hipStream_t pick(pi_handle, void* stream) { return reinterpret_cast<hipStream_t>(stream); }

bool dim_ok(int d) { return d == 64 || d == 128 || d == 256; }

// Grow-only device buffer (the reference grows its scratch lazily the same
// way, src/cuda/mod.rs:257-278).  Freed buffers are released after the
// stream drains so in-flight kernels never see freed memory.
template <typename T>
int grow(pi_handle h, T** ptr, size_t* cap, size_t need, hipStream_t s, const char* what,
         bool zero) {
    if (need <= *cap) return PI_OK;
    size_t n = need + need / 4;
    PI_HIP(h, hipStreamSynchronize(s), what);
    if (*ptr) PI_HIP(h, hipFree(*ptr), what);
    *ptr = nullptr;
    *cap = 0;
    PI_HIP(h, hipMalloc(reinterpret_cast<void**>(ptr), n * sizeof(T)), what);
    if (zero) PI_HIP(h, hipMemset(*ptr, 0, n * sizeof(T)), what);
    *cap = n;
    return PI_OK;
}

// The handle's workspaces serve whatever stream a call names.  A call on a
// different stream from the previous workspace user first makes its stream
// wait for that use (ws_begin); every use is marked by an event on its own
// stream (ws_end), so the wait never names a stream the caller may since have
// destroyed.
int ws_begin(pi_handle h, hipStream_t s, const char* what) {
    if (h->ws_used && s != h->ws_stream) PI_HIP(h, hipStreamWaitEvent(s, h->ws_event, 0), what);
    return PI_OK;
}

int ws_end(pi_handle h, hipStream_t s, const char* what) {
    PI_HIP(h, hipEventRecord(h->ws_event, s), what);
    h->ws_used = true;
    h->ws_stream = s;
    return PI_OK;
}

// ops::apply_rope (src/ops.rs:45-46): freq_i = 1 / base^(2i/rope_dim) in f32.
void norm_rope_freqs(float base, int rope_dim, float* f) {
    for (int i = 0; i < rope_dim / 2; ++i) {
        const float expo = 2.0f * (float)i / (float)rope_dim;
        f[i] = 1.0f / powf(base, expo);
    }
}

// ops::compute_imrope_freqs (src/ops.rs:78-122): every section track starts at
// 1 and advances by one f32 multiply by theta_scale = base^(-2/n_rot) per pair,
// so pair k gets theta_scale^k by repeated multiplication whatever its section
// (src/model/mod.rs:1080-1083 keeps the first n_rot/2).
void imrope_freqs(float base, int n_rot, float* f) {
    const float theta_scale = powf(base, -2.0f / (float)n_rot);
    float t = 1.0f;
    for (int i = 0; i < n_rot / 2; ++i) {
        f[i] = t;
        t *= theta_scale;
    }
}

// ---- TurboQuant matrices (src/turboquant/mod.rs:657-746) ----------------------
// SplitMix64 with the reference's Box-Muller Gaussian: two f64 uniforms from
// the top 53 bits, u1 clamped to 1e-10, r * cos(theta) rounded to f32.
struct SplitMix64 {
    uint64_t state;
    uint64_t next() {
        state += 0x9E3779B97F4A7C15ULL;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        return z ^ (z >> 31);
    }
    double uniform() { return (double)(next() >> 11) / (double)(1ULL << 53); }
    float gaussian() {
        const double u1 = std::max(uniform(), 1e-10);
        const double u2 = uniform();
        return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2));
    }
};

// Orthogonal Q of a seeded Gaussian A by Gram-Schmidt over columns, in f32
// with separately rounded operations (this file is built without FMA
// contraction): q_j = a_j - sum_k (q_k . a_j) q_k, then q_j /= |q_j| when
// |q_j| > 1e-10.  The projections use the original column a_j.
void tq_orthogonal(float* q, int dim, uint64_t seed) {
    std::vector<float> a((size_t)dim * dim);
    SplitMix64 rng{seed};
    for (float& x : a) x = rng.gaussian();
    for (int j = 0; j < dim; ++j) {
        for (int i = 0; i < dim; ++i) q[(size_t)i * dim + j] = a[(size_t)i * dim + j];
        for (int k = 0; k < j; ++k) {
            float dot = 0.0f;
            for (int i = 0; i < dim; ++i) dot += q[(size_t)i * dim + k] * a[(size_t)i * dim + j];
            for (int i = 0; i < dim; ++i) q[(size_t)i * dim + j] -= dot * q[(size_t)i * dim + k];
        }
        float nrm = 0.0f;
        for (int i = 0; i < dim; ++i) nrm += q[(size_t)i * dim + j] * q[(size_t)i * dim + j];
        nrm = std::sqrt(nrm);
        if (nrm > 1e-10f)
            for (int i = 0; i < dim; ++i) q[(size_t)i * dim + j] /= nrm;
    }
}

void tq_matrices(int dim, uint64_t seed, float* rot, float* qjl) {
    tq_orthogonal(rot, dim, seed);
    SplitMix64 rng{seed ^ 0xDEADBEEFULL};
    for (size_t i = 0; i < (size_t)dim * dim; ++i) qjl[i] = rng.gaussian();
}

}  // namespace

extern "C" {

int pi_abi_version(void) { return PI_ATTN_ABI_VERSION; }

int pi_create(int device, pi_handle* out) {
    if (!out) return fail(nullptr, PI_ERR_INVALID_ARG, "pi_create: out is null");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
        return fail(nullptr, PI_ERR_DEVICE, "pi_create: no HIP device (%s)",
                    e == hipSuccess ? "0 devices" : hipGetErrorString(e));
    if (device < 0 || device >= n)
        return fail(nullptr, PI_ERR_INVALID_ARG, "pi_create: device %d of %d", device, n);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return fail(nullptr, PI_ERR_DEVICE, "pi_create: %s", hipGetErrorString(e));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, PI_ERR_UNSUPPORTED, "pi_create: device %d is %s; kernels are built for gfx950",
                    device, prop.gcnArchName);
    pi_handle h = new (std::nothrow) pi_handle_s();
    if (!h) return fail(nullptr, PI_ERR_OUT_OF_MEMORY, "pi_create: host allocation");
    h->device = device;
    e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&h->ws_event, hipEventDisableTiming);
    // the device address of this GPU's fixed scratch, looked up with it current
    if (e == hipSuccess) e = pi::decode_scratch(device, &h->scratch);
    if (e != hipSuccess) {
        if (h->ws_event) (void)hipEventDestroy(h->ws_event);
        if (h->stream) (void)hipStreamDestroy(h->stream);
        delete h;
        return fail(nullptr, PI_ERR_DEVICE, "pi_create: %s", hipGetErrorString(e));
    }
    *out = h;
    return PI_OK;
}

void pi_destroy(pi_handle h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    if (h->ws_used) (void)hipEventSynchronize(h->ws_event);
    (void)hipFree(h->dws.partial_o);
    (void)hipFree(h->dws.partial_ml);
    (void)hipFree(h->dws.seg_runs);
    (void)hipFree(h->gws.buf);
    (void)hipFree(h->h2d_scratch);
    (void)hipFree(h->tq_qv);
    (void)hipFree(h->tq_sc);
    (void)hipFree(h->pfs_buf);
    (void)hipFree(h->pad_buf);
    if (h->pin) (void)hipHostFree(h->pin);
    if (h->ws_event) (void)hipEventDestroy(h->ws_event);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
}

const char* pi_last_error(pi_handle h) { return h ? h->err.c_str() : g_create_err.c_str(); }

int pi_sync(pi_handle h, void* stream) {
    PI_CHECK_HANDLE(h);
    PI_HIP(h, hipSetDevice(h->device), "pi_sync");
    PI_HIP(h, hipStreamSynchronize(pick(h, stream)), "pi_sync");
    return PI_OK;
}

// ---- KV pool ---------------------------------------------------------------

int pi_kv_pool_create(pi_handle h, int32_t n_pages, int32_t page_tokens, int32_t n_kv_heads,
                      int32_t head_dim, int32_t dtype, pi_kv_pool* out) {
    PI_CHECK_HANDLE(h);
    if (!out) return fail(h, PI_ERR_INVALID_ARG, "pi_kv_pool_create: out is null");
    *out = nullptr;
    if (page_tokens != pi::kPageTokens)
        return fail(h, PI_ERR_UNSUPPORTED, "pi_kv_pool_create: page_tokens must be 16 (got %d)", page_tokens);
    if (n_pages <= 0 || n_kv_heads <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_kv_pool_create: n_pages=%d n_kv_heads=%d", n_pages, n_kv_heads);
    if (!dim_ok(head_dim))
        return fail(h, PI_ERR_UNSUPPORTED, "pi_kv_pool_create: head_dim %d (64/128/256)", head_dim);
    if (dtype != PI_F32 && dtype != PI_F16)
        return fail(h, PI_ERR_UNSUPPORTED, "pi_kv_pool_create: pool dtype %d (f32 or f16)", dtype);
    const int eb = dtype == PI_F32 ? 4 : 2;
    const size_t bytes = (size_t)n_pages * n_kv_heads * pi::kPageTokens * head_dim * eb;
    PI_HIP(h, hipSetDevice(h->device), "pi_kv_pool_create");
    pi_kv_pool p = new (std::nothrow) pi_kv_pool_s();
    if (!p) return fail(h, PI_ERR_OUT_OF_MEMORY, "pi_kv_pool_create: host allocation");
    p->owner = h;
    p->bytes = 2 * bytes;
    // K and V blocks interleaved per (page, KV head): a segment's page is one 2 x 16 x D run
    const size_t blk = (size_t)pi::kPageTokens * head_dim * eb;
    p->g = pi::KvGeom{nullptr, nullptr, n_pages, n_kv_heads, head_dim, dtype, eb, 2 * blk, 2 * blk};
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, 2 * bytes);
    // Zero once so slack slots of partially filled pages hold finite values.
    if (e == hipSuccess) e = hipMemset(base, 0, 2 * bytes);
    if (e != hipSuccess) {
        (void)hipFree(base);
        delete p;
        return hip_fail(h, e, "pi_kv_pool_create");
    }
    p->g.k = base;
    p->g.v = static_cast<char*>(base) + blk;
    *out = p;
    return PI_OK;
}

void pi_kv_pool_destroy(pi_kv_pool pool) {
    if (!pool) return;
    (void)hipSetDevice(pool->owner->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(pool->g.k);  // one allocation: v is inside it
    delete pool;
}

size_t pi_kv_pool_bytes(pi_kv_pool pool) { return pool ? pool->bytes : 0; }

int pi_kv_append(pi_handle h, pi_kv_pool pool, const void* d_k, const void* d_v, int32_t src_dtype,
                 const int32_t* d_page_table, int32_t max_pages, const int32_t* d_start_pos,
                 int32_t n_seq, int32_t n_tok, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!pool || !d_k || !d_v || !d_page_table || !d_start_pos)
        return fail(h, PI_ERR_INVALID_ARG, "pi_kv_append: null argument");
    if (n_seq < 0 || n_tok < 0 || max_pages <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_kv_append: n_seq=%d n_tok=%d max_pages=%d", n_seq, n_tok, max_pages);
    if (src_dtype < PI_F32 || src_dtype > PI_BF16)
        return fail(h, PI_ERR_UNSUPPORTED, "pi_kv_append: src dtype %d", src_dtype);
    if (n_seq == 0 || n_tok == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_kv_append");
    PI_HIP(h, pi::launch_kv_append(pool->g, d_k, d_v, src_dtype, d_page_table, max_pages,
                                   d_start_pos, n_seq, n_tok, pick(h, stream)),
           "pi_kv_append");
    return PI_OK;
}

int pi_kv_read(pi_handle h, pi_kv_pool pool, const int32_t* d_page_table, int32_t max_pages,
               int32_t seq, int32_t start, int32_t n_tok, float* d_k_out, float* d_v_out,
               void* stream) {
    PI_CHECK_HANDLE(h);
    if (!pool || !d_page_table || !d_k_out || !d_v_out)
        return fail(h, PI_ERR_INVALID_ARG, "pi_kv_read: null argument");
    if (seq < 0 || start < 0 || n_tok < 0 || max_pages <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_kv_read: seq=%d start=%d n_tok=%d", seq, start, n_tok);
    if (n_tok == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_kv_read");
    PI_HIP(h, pi::launch_kv_read(pool->g, d_page_table, max_pages, seq, start, n_tok, d_k_out,
                                 d_v_out, pick(h, stream)),
           "pi_kv_read");
    return PI_OK;
}

// ---- prologue ----------------------------------------------------------------

int pi_head_rmsnorm(pi_handle h, float* d_x, const float* d_w, int32_t n_rows, int32_t dim,
                    int32_t row_stride, float eps, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!d_x || !d_w) return fail(h, PI_ERR_INVALID_ARG, "pi_head_rmsnorm: null argument");
    if (n_rows < 0 || dim <= 0 || row_stride < dim)
        return fail(h, PI_ERR_INVALID_ARG, "pi_head_rmsnorm: n_rows=%d dim=%d row_stride=%d", n_rows, dim, row_stride);
    if (n_rows == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_head_rmsnorm");
    PI_HIP(h, pi::launch_head_rmsnorm(d_x, d_w, n_rows, dim, row_stride, eps, pick(h, stream)),
           "pi_head_rmsnorm");
    return PI_OK;
}

int pi_rope(pi_handle h, float* d_q, float* d_k, const int32_t* d_pos, int32_t n_tok,
            int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t rope_dim, float base,
            const int32_t* h_sections, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!d_q || !d_pos) return fail(h, PI_ERR_INVALID_ARG, "pi_rope: null argument");
    if (n_tok < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim > 256)
        return fail(h, PI_ERR_INVALID_ARG, "pi_rope: n_tok=%d heads=%d/%d head_dim=%d", n_tok, n_q_heads, n_kv_heads, head_dim);
    // src/model/mod.rs:574-597,1074: rope dims are capped to the head dim.
    int rd = rope_dim <= 0 ? head_dim : (rope_dim < head_dim ? rope_dim : head_dim);
    const int n_pairs = rd / 2;
    if (n_pairs > 128) return fail(h, PI_ERR_UNSUPPORTED, "pi_rope: rope_dim %d", rd);
    if (n_tok == 0 || n_pairs == 0) return PI_OK;
    pi::RopeFreqs f;
    std::memset(&f, 0, sizeof f);
    if (h_sections == nullptr)
        norm_rope_freqs(base, rd, f.f);
    else
        imrope_freqs(base, rd, f.f);
    PI_HIP(h, hipSetDevice(h->device), "pi_rope");
    PI_HIP(h, pi::launch_rope(d_q, d_k, d_pos, n_tok, n_q_heads, n_kv_heads, head_dim, n_pairs,
                              h_sections ? 1 : 0, f, pick(h, stream)),
           "pi_rope");
    return PI_OK;
}

int pi_attn_prologue(pi_handle h, float* d_q, float* d_k, const float* d_v,
                     const float* d_q_norm_w, const float* d_k_norm_w, float eps,
                     int32_t rope_dim, float rope_base, const int32_t* h_sections,
                     pi_kv_pool pool, const int32_t* d_page_table, int32_t max_pages,
                     const int32_t* d_start_pos, int32_t n_seq, int32_t n_tok,
                     int32_t n_q_heads, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!d_q || !d_k || !d_v || !pool || !d_page_table || !d_start_pos)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prologue: null argument");
    if (n_seq < 0 || n_tok < 0 || max_pages <= 0 || n_q_heads <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prologue: n_seq=%d n_tok=%d max_pages=%d n_q_heads=%d",
                    n_seq, n_tok, max_pages, n_q_heads);
    const pi::KvGeom& g = pool->g;
    // src/model/mod.rs:1074: the rotation is capped to the head dim
    const int rd = rope_dim <= 0 ? g.head_dim : (rope_dim < g.head_dim ? rope_dim : g.head_dim);
    const int n_pairs = rd / 2;
    if (n_pairs > 128) return fail(h, PI_ERR_UNSUPPORTED, "pi_attn_prologue: rope_dim %d", rd);
    if (n_seq == 0 || n_tok == 0) return PI_OK;
    pi::RopeFreqs f;
    std::memset(&f, 0, sizeof f);
    if (h_sections == nullptr)
        norm_rope_freqs(rope_base, rd, f.f);
    else
        imrope_freqs(rope_base, rd, f.f);
    PI_HIP(h, hipSetDevice(h->device), "pi_attn_prologue");
    PI_HIP(h, pi::launch_attn_prologue(d_q, d_k, d_v, d_q_norm_w, d_k_norm_w, eps, f, n_pairs,
                                       h_sections ? 1 : 0, g, d_page_table, max_pages, d_start_pos,
                                       n_seq, n_tok, n_q_heads, pick(h, stream)),
           "pi_attn_prologue");
    return PI_OK;
}

// ---- attention -------------------------------------------------------------------

// Shape checks shared by the decode entry points.
static int decode_check(pi_handle h, const char* fn, const pi::KvGeom& g, const void* d_q,
                        const void* d_page_table, const void* d_ctx_len, const void* d_out,
                        int32_t max_pages, int32_t batch, int32_t n_q_heads, int32_t gqa_mode) {
    if (!d_q || !d_page_table || !d_ctx_len || !d_out)
        return fail(h, PI_ERR_INVALID_ARG, "%s: null argument", fn);
    if (batch < 0 || max_pages <= 0 || n_q_heads <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "%s: batch=%d max_pages=%d n_q_heads=%d", fn, batch, max_pages, n_q_heads);
    if (gqa_mode != PI_GQA_MODULO && gqa_mode != PI_GQA_GROUPED)
        return fail(h, PI_ERR_INVALID_ARG, "%s: gqa_mode %d", fn, gqa_mode);
    // the modulo map (src/model/mod.rs:1155) takes any head counts; the grouped one needs a multiple
    if (gqa_mode == PI_GQA_GROUPED && n_q_heads % g.n_kv_heads != 0)
        return fail(h, PI_ERR_INVALID_ARG, "%s: grouped head map with n_q_heads %d not a multiple of n_kv_heads %d",
                    fn, n_q_heads, g.n_kv_heads);
    if (batch > pi::kMaxBatch)
        return fail(h, PI_ERR_UNSUPPORTED, "%s: batch %d > %d", fn, batch, pi::kMaxBatch);
    const long long blocks = ((long long)n_q_heads + g.n_kv_heads - 1) / g.n_kv_heads;  // >= column blocks
    if ((long long)batch * g.n_kv_heads * blocks * ((max_pages + pi::kItemPages - 1) / pi::kItemPages) > (1LL << 30))
        return fail(h, PI_ERR_UNSUPPORTED, "%s: batch x heads x pages too large", fn);
    // q rows are read and out rows written in 16-byte groups
    if (((uintptr_t)d_q | (uintptr_t)d_out) & 15)
        return fail(h, PI_ERR_INVALID_ARG, "%s: d_q and d_out must be 16-byte aligned", fn);
    return PI_OK;
}

static int gate_check(pi_handle h, const char* fn, const float* d_gate) {
    if ((uintptr_t)d_gate & 15) return fail(h, PI_ERR_INVALID_ARG, "%s: d_gate must be 16-byte aligned", fn);
    return PI_OK;
}

static pi::DecodeParams decode_params(const float* d_q, const int32_t* d_page_table,
                                      int32_t max_pages, const int32_t* d_ctx_len, int32_t batch,
                                      int32_t n_q_heads, int32_t gqa_mode, float scale,
                                      const float* d_gate, float* d_out, const pi::DecodePlan& plan) {
    pi::DecodeParams p;
    p.q = d_q;
    p.page_table = d_page_table;
    p.ctx_len = d_ctx_len;
    p.gate = d_gate;
    p.out = d_out;
    p.max_pages = max_pages;
    p.batch = batch;
    p.n_q_heads = n_q_heads;
    p.gqa_mode = gqa_mode;
    p.scale = scale;
    p.item_pages = plan.item_pages;
    p.group = plan.group;
    p.cols = plan.cols;
    p.n_cb = plan.n_cb;
    return p;
}

// The decode launch on the handle's workspace.  max_tokens bounds every sequence's length
// (0: the table row's 16 * max_pages); the layer seam passes its exact length, so the work
// items are sized for the tokens the sequence holds, not for its whole cache.
static int attn_decode_ws(pi_handle h, const char* fn, const float* d_q, pi_kv_pool pool,
                          const int32_t* d_page_table, int32_t max_pages, const int32_t* d_ctx_len,
                          int32_t batch, int32_t n_q_heads, int32_t gqa_mode, float scale,
                          const float* d_gate, float* d_out, hipStream_t s, int32_t max_tokens) {
    const pi::KvGeom& g = pool->g;
    int rc = decode_check(h, fn, g, d_q, d_page_table, d_ctx_len, d_out, max_pages, batch,
                          n_q_heads, gqa_mode);
    if (!rc) rc = gate_check(h, fn, d_gate);
    if (rc) return rc;
    if (batch == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), fn);
    if ((rc = ws_begin(h, s, fn))) return rc;
    const pi::DecodePlan plan = pi::decode_plan(g, batch, max_pages, n_q_heads, gqa_mode, h->device, max_tokens);
    const size_t need_o = pi::decode_ws_floats_o(g, plan);
    const size_t need_ml = need_o / g.head_dim * 2;
    if ((rc = grow(h, &h->dws.partial_o, &h->dws.capacity_o, need_o, s, "decode workspace", false))) return rc;
    if ((rc = grow(h, &h->dws.partial_ml, &h->dws.capacity_ml, need_ml, s, "decode workspace", false))) return rc;
    if ((rc = grow(h, &h->dws.seg_runs, &h->dws.capacity_runs, pi::decode_ws_ints_runs(g, plan), s,
                   "decode workspace", false))) return rc;
    const pi::DecodeParams p = decode_params(d_q, d_page_table, max_pages, d_ctx_len, batch, n_q_heads,
                                             gqa_mode, scale, d_gate, d_out, plan);
    PI_HIP(h, pi::launch_decode(g, p, h->dws, plan, s), fn);
    return ws_end(h, s, fn);
}

int pi_attn_decode(pi_handle h, const float* d_q, pi_kv_pool pool, const int32_t* d_page_table,
                   int32_t max_pages, const int32_t* d_ctx_len, int32_t batch, int32_t n_q_heads,
                   int32_t gqa_mode, float scale, const float* d_gate, float* d_out,
                   void* stream) {
    PI_CHECK_HANDLE(h);
    if (!pool) return fail(h, PI_ERR_INVALID_ARG, "pi_attn_decode: null argument");
    return attn_decode_ws(h, "pi_attn_decode", d_q, pool, d_page_table, max_pages, d_ctx_len, batch,
                          n_q_heads, gqa_mode, scale, d_gate, d_out, pick(h, stream), 0);
}

int pi_attn_decode_noalloc(pi_handle h, const float* d_q, pi_kv_pool pool,
                           const int32_t* d_page_table, int32_t max_pages,
                           const int32_t* d_ctx_len, int32_t batch, int32_t n_q_heads,
                           int32_t gqa_mode, float scale, const float* d_gate, float* d_out,
                           void* stream) {
    PI_CHECK_HANDLE(h);
    if (!pool) return fail(h, PI_ERR_INVALID_ARG, "pi_attn_decode_noalloc: null argument");
    const pi::KvGeom& g = pool->g;
    int rc = decode_check(h, "pi_attn_decode_noalloc", g, d_q, d_page_table, d_ctx_len, d_out,
                          max_pages, batch, n_q_heads, gqa_mode);
    if (!rc) rc = gate_check(h, "pi_attn_decode_noalloc", d_gate);
    if (rc) return rc;
    if (batch == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_attn_decode_noalloc");
    const pi::DecodePlan plan = pi::decode_plan(g, batch, max_pages, n_q_heads, gqa_mode, h->device);
    const size_t limit = pi::kDecodeScratchFloats;
    // partial o, then (m, l), then the segments' run table, each at a 256-byte boundary
    // inside the scratch
    const size_t need_o = pi::decode_ws_floats_o(g, plan);
    const size_t off_ml = (need_o + 63) / 64 * 64;
    const size_t need_ml = need_o / g.head_dim * 2;
    const size_t off_runs = (off_ml + need_ml + 63) / 64 * 64;
    const size_t need_runs = pi::decode_ws_ints_runs(g, plan);
    if (off_runs + need_runs > limit)
        return fail(h, PI_ERR_UNSUPPORTED,
                    "pi_attn_decode_noalloc: %zu scratch floats needed (batch %d x %d kv heads + %d "
                    "workgroups, %d q heads per kv head, head_dim %d) > the fixed %zu",
                    off_runs + need_runs, batch, g.n_kv_heads, plan.grid, plan.group, g.head_dim,
                    limit);
    pi::DecodeWorkspace ws;
    ws.partial_o = h->scratch;
    ws.partial_ml = h->scratch + off_ml;
    ws.seg_runs = reinterpret_cast<int32_t*>(h->scratch + off_runs);
    ws.capacity_o = need_o;
    ws.capacity_ml = need_ml;
    ws.capacity_runs = need_runs;
    const pi::DecodeParams p = decode_params(d_q, d_page_table, max_pages, d_ctx_len, batch, n_q_heads,
                                             gqa_mode, scale, d_gate, d_out, plan);
    PI_HIP(h, pi::launch_decode(g, p, ws, plan, pick(h, stream)), "pi_attn_decode_noalloc");
    return PI_OK;
}

int pi_attn_prefill(pi_handle h, const void* d_q, const void* d_k, const void* d_v, int32_t dtype,
                    int32_t batch, int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads,
                    int32_t head_dim, int32_t causal, int32_t gqa_mode, float scale, float* d_out,
                    void* stream) {
    PI_CHECK_HANDLE(h);
    if (!d_q || !d_k || !d_v || !d_out) return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prefill: null argument");
    if (batch < 0 || seq_len < 0 || n_q_heads <= 0 || n_kv_heads <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prefill: batch=%d seq_len=%d heads=%d/%d", batch, seq_len, n_q_heads, n_kv_heads);
    if (gqa_mode != PI_GQA_MODULO && gqa_mode != PI_GQA_GROUPED)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prefill: gqa_mode %d", gqa_mode);
    if (dtype != PI_BF16 && dtype != PI_F16)
        return fail(h, PI_ERR_UNSUPPORTED, "pi_attn_prefill: dtype %d (bf16 or f16)", dtype);
    if (head_dim <= 0 || head_dim > 256)
        return fail(h, PI_ERR_UNSUPPORTED, "pi_attn_prefill: head_dim %d (1..256)", head_dim);
    if (gqa_mode == PI_GQA_GROUPED && n_q_heads % n_kv_heads != 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prefill: grouped head map with n_q_heads %d not a multiple of n_kv_heads %d",
                    n_q_heads, n_kv_heads);
    if (batch == 0 || seq_len == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_attn_prefill");
    hipStream_t s = pick(h, stream);
    int rc;
    if ((rc = ws_begin(h, s, "pi_attn_prefill"))) return rc;
    // The kernels run at 64, 128 or 256 dims; another head_dim runs zero-padded to the next
    // of them (zero dims change no q.k and give zero output dims; the caller's scale stands)
    const int W = head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
    const size_t need = pi::prefill_ws_floats(batch, seq_len, n_q_heads, n_kv_heads, W, causal ? 1 : 0);
    if (need && (rc = grow(h, &h->pfs_buf, &h->pfs_floats, need, s, "pi_attn_prefill workspace", false))) return rc;
    const void *q = d_q, *k = d_k, *v = d_v;
    float* out = d_out;
    const size_t rq = (size_t)batch * seq_len * n_q_heads, rkv = (size_t)batch * seq_len * n_kv_heads;
    if (W != head_dim) {
        if (rq > (size_t)INT32_MAX)
            return fail(h, PI_ERR_UNSUPPORTED, "pi_attn_prefill: %zu query rows at a padded head_dim", rq);
        // [out rows (f32) | q | k | v rows (16-bit)], all W wide
        const size_t half_rows = (rq + 2 * rkv) * W;
        if ((rc = grow(h, &h->pad_buf, &h->pad_floats, rq * W + (half_rows + 1) / 2, s,
                       "pi_attn_prefill padding", false)))
            return rc;
        out = h->pad_buf;
        uint16_t* pq = reinterpret_cast<uint16_t*>(h->pad_buf + rq * W);
        uint16_t *pk = pq + rq * W, *pv = pk + rkv * W;
        const struct { uint16_t* dst; const void* src; size_t rows; } ins[] = {
            {pq, d_q, rq}, {pk, d_k, rkv}, {pv, d_v, rkv}};
        for (const auto& c : ins)
            PI_HIP(h, pi::launch_pack_rows16(c.dst, static_cast<const uint16_t*>(c.src), (int32_t)c.rows, 1,
                                             head_dim, W, head_dim, 0, W, 0, s),
                   "pi_attn_prefill");
        q = pq;
        k = pk;
        v = pv;
    }
    PI_HIP(h, pi::launch_prefill(q, k, v, dtype, batch, seq_len, seq_len, 0, n_q_heads,
                                 n_kv_heads, W, causal ? 1 : 0, gqa_mode, scale, out,
                                 h->pfs_buf, h->pfs_floats, s),
           "pi_attn_prefill");
    if (W != head_dim)
        PI_HIP(h, pi::launch_pack_rows(d_out, out, (int32_t)rq, 1, head_dim, head_dim, W, 0, head_dim, 0, s),
               "pi_attn_prefill");
    return ws_end(h, s, "pi_attn_prefill");
}

int pi_attn_prefill_paged(pi_handle h, const void* d_q, pi_kv_pool pool,
                          const int32_t* d_page_table, int32_t max_pages, int32_t start_pos,
                          int32_t n_tok, int32_t n_q_heads, int32_t gqa_mode, float scale,
                          float* d_out, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!d_q || !pool || !d_page_table || !d_out)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prefill_paged: null argument");
    const pi::KvGeom& g = pool->g;
    if (start_pos < 0 || n_tok < 0 || max_pages <= 0 || n_q_heads <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prefill_paged: start_pos=%d n_tok=%d max_pages=%d n_q_heads=%d",
                    start_pos, n_tok, max_pages, n_q_heads);
    if (gqa_mode != PI_GQA_MODULO && gqa_mode != PI_GQA_GROUPED)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prefill_paged: gqa_mode %d", gqa_mode);
    if (g.dtype != PI_F16 && g.dtype != PI_F32)
        return fail(h, PI_ERR_UNSUPPORTED, "pi_attn_prefill_paged: pool dtype %d (f16 or f32)", g.dtype);
    if (gqa_mode == PI_GQA_GROUPED && n_q_heads % g.n_kv_heads != 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prefill_paged: grouped head map with n_q_heads %d not a multiple of n_kv_heads %d",
                    n_q_heads, g.n_kv_heads);
    const long long n_keys = (long long)start_pos + n_tok;
    if (n_keys > (long long)max_pages * pi::kPageTokens)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_prefill_paged: %lld keys exceed the %d-page row", n_keys, max_pages);
    if (n_tok == 0) return PI_OK;
    hipStream_t s = pick(h, stream);
    PI_HIP(h, hipSetDevice(h->device), "pi_attn_prefill_paged");
    if (g.dtype == PI_F32) {  // straight from the pages, no workspace
        PI_HIP(h, pi::launch_prefill_f32(g, static_cast<const float*>(d_q), d_page_table, max_pages,
                                         start_pos, n_tok, n_q_heads, gqa_mode, scale, d_out, s),
               "pi_attn_prefill_paged");
        return PI_OK;
    }
    int rc;
    if ((rc = ws_begin(h, s, "pi_attn_prefill_paged"))) return rc;
    // straight from the f16 pages
    const size_t need = pi::prefill_ws_floats(1, n_tok, n_q_heads, g.n_kv_heads, g.head_dim, 1);
    if (need && (rc = grow(h, &h->pfs_buf, &h->pfs_floats, need, s, "pi_attn_prefill_paged workspace", false)))
        return rc;
    PI_HIP(h, pi::launch_prefill_pool(g, d_q, 0, d_page_table, start_pos, n_tok, n_q_heads, gqa_mode,
                                      scale, d_out, h->pfs_buf, h->pfs_floats, s),
           "pi_attn_prefill_paged");
    return ws_end(h, s, "pi_attn_prefill_paged");
}

// ---- gated DeltaNet ------------------------------------------------------------------

int pi_gdn_gates(pi_handle h, const float* d_beta_raw, const float* d_a_raw, const float* d_ssm_a,
                 const float* d_dt_bias, float* d_beta, float* d_g, int32_t n_tok,
                 int32_t n_v_heads, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!d_beta_raw || !d_a_raw || !d_ssm_a || !d_dt_bias || !d_beta || !d_g)
        return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_gates: null argument");
    if (n_tok < 0 || n_v_heads <= 0) return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_gates: n_tok=%d n_v_heads=%d", n_tok, n_v_heads);
    if (n_tok == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_gdn_gates");
    PI_HIP(h, pi::launch_gdn_gates(d_beta_raw, d_a_raw, d_ssm_a, d_dt_bias, d_beta, d_g, n_tok,
                                   n_v_heads, pick(h, stream)),
           "pi_gdn_gates");
    return PI_OK;
}

int pi_gdn_conv1d(pi_handle h, const float* d_x, float* d_conv_state, const float* d_w,
                  float* d_out, int32_t n_seq, int32_t n_tok, int32_t conv_dim, int32_t d_conv,
                  void* stream) {
    PI_CHECK_HANDLE(h);
    if (!d_x || !d_conv_state || !d_w || !d_out)
        return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_conv1d: null argument");
    if (d_out == d_x) return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_conv1d: d_out must not alias d_x");
    if (n_seq < 0 || n_tok < 0 || conv_dim <= 0 || d_conv < 1 || d_conv > 16)
        return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_conv1d: n_seq=%d n_tok=%d conv_dim=%d d_conv=%d",
                    n_seq, n_tok, conv_dim, d_conv);
    if (n_seq == 0 || n_tok == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_gdn_conv1d");
    PI_HIP(h, pi::launch_gdn_conv1d(d_x, d_conv_state, d_w, d_out, n_seq, n_tok, conv_dim, d_conv,
                                    pick(h, stream)),
           "pi_gdn_conv1d");
    return PI_OK;
}

int pi_gdn_rmsnorm_gated(pi_handle h, float* d_o, const float* d_z, const float* d_w,
                         int32_t n_rows, int32_t n_v_heads, int32_t v_hd, float eps,
                         void* stream) {
    PI_CHECK_HANDLE(h);
    if (!d_o || !d_z || !d_w) return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_rmsnorm_gated: null argument");
    if (n_rows < 0 || n_v_heads <= 0 || v_hd <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_rmsnorm_gated: n_rows=%d n_v_heads=%d v_hd=%d",
                    n_rows, n_v_heads, v_hd);
    if (n_rows == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_gdn_rmsnorm_gated");
    PI_HIP(h, pi::launch_gdn_rmsnorm_gated(d_o, d_z, d_w, n_rows, n_v_heads, v_hd, eps, pick(h, stream)),
           "pi_gdn_rmsnorm_gated");
    return PI_OK;
}

static int gdn_shape_check(pi_handle h, const char* fn, int32_t n_k_heads, int32_t n_v_heads,
                           int32_t k_hd, int32_t v_hd) {
    if (n_k_heads <= 0 || n_v_heads <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "%s: n_k_heads=%d n_v_heads=%d", fn, n_k_heads, n_v_heads);
    if (k_hd <= 0 || v_hd <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "%s: k_hd=%d v_hd=%d", fn, k_hd, v_hd);
    if (k_hd > pi::kGdnMaxKhd)
        return fail(h, PI_ERR_UNSUPPORTED, "%s: k_hd=%d (at most %d)", fn, k_hd, pi::kGdnMaxKhd);
    return PI_OK;
}

int pi_gdn_decode(pi_handle h, const float* d_q, const float* d_k, const float* d_v,
                  const float* d_beta, const float* d_g, float* d_state, float* d_out,
                  int32_t batch, int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd, int32_t v_hd,
                  void* stream) {
    PI_CHECK_HANDLE(h);
    if (!d_q || !d_k || !d_v || !d_beta || !d_g || !d_state || !d_out)
        return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_decode: null argument");
    if (batch < 0) return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_decode: batch=%d", batch);
    int rc = gdn_shape_check(h, "pi_gdn_decode", n_k_heads, n_v_heads, k_hd, v_hd);
    if (rc) return rc;
    if (batch == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_gdn_decode");
    PI_HIP(h, pi::launch_gdn_decode(d_q, d_k, d_v, d_beta, d_g, d_state, d_out, batch, n_k_heads,
                                    n_v_heads, k_hd, v_hd, pick(h, stream)),
           "pi_gdn_decode");
    return PI_OK;
}

int pi_gdn_prefill(pi_handle h, const float* d_q, const float* d_k, const float* d_v,
                   const float* d_beta, const float* d_g, float* d_state, float* d_out,
                   int32_t n_tok, int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd, int32_t v_hd,
                   int32_t chunk, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!d_q || !d_k || !d_v || !d_beta || !d_g || !d_state || !d_out)
        return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_prefill: null argument");
    if (n_tok < 0) return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_prefill: n_tok=%d", n_tok);
    int rc = gdn_shape_check(h, "pi_gdn_prefill", n_k_heads, n_v_heads, k_hd, v_hd);
    if (rc) return rc;
    if (chunk != 64 && chunk != 1)
        return fail(h, PI_ERR_UNSUPPORTED, "pi_gdn_prefill: chunk %d (64, or 1: token by token)", chunk);
    if (n_tok == 0) return PI_OK;
    hipStream_t s = pick(h, stream);
    PI_HIP(h, hipSetDevice(h->device), "pi_gdn_prefill");
    if (chunk == 1 || k_hd != 128 || v_hd != 128) {  // the per-token recurrence, any widths
        PI_HIP(h, pi::launch_gdn_recur(d_q, d_k, d_v, d_beta, d_g, d_state, d_out, 1, n_tok, n_k_heads,
                                       n_v_heads, k_hd, v_hd, s),
               "pi_gdn_prefill");
        return PI_OK;
    }
    if ((rc = ws_begin(h, s, "pi_gdn_prefill"))) return rc;
    const size_t need = pi::gdn_prefill_ws_floats(n_tok, n_k_heads, n_v_heads, chunk);
    if (need) {
        rc = grow(h, &h->gws.buf, &h->gws.capacity, need, s, "pi_gdn_prefill workspace", false);
        if (rc) return rc;
    }
    hipError_t e = pi::launch_gdn_prefill(d_q, d_k, d_v, d_beta, d_g, d_state, d_out, n_tok,
                                          n_k_heads, n_v_heads, chunk, h->gws, s);
    if (e != hipSuccess) return hip_fail(h, e, "pi_gdn_prefill");
    return ws_end(h, s, "pi_gdn_prefill");
}

// ---- host-slice drop-ins -------------------------------------------------------------

int pi_ops_attention_head(pi_handle h, float* h_out, const float* h_q, const float* h_k_cache,
                          const float* h_v_cache, size_t seq_len, size_t head_dim) {
    PI_CHECK_HANDLE(h);
    if (!h_out || !h_q || (seq_len && (!h_k_cache || !h_v_cache)))
        return fail(h, PI_ERR_INVALID_ARG, "attention_head: null slice");
    if (head_dim == 0 || head_dim > 256)
        return fail(h, PI_ERR_UNSUPPORTED, "attention_head: head_dim %zu (1..256 on the device)", head_dim);
    if (seq_len > (size_t)1 << 24) return fail(h, PI_ERR_UNSUPPORTED, "attention_head: seq_len %zu", seq_len);
    PI_HIP(h, hipSetDevice(h->device), "attention_head");
    hipStream_t s = h->stream;
    // Rows are zero-padded to a kernel head size (64, 128 or 256): zero q and key
    // dims leave every dot product unchanged, the scale stays 1/sqrt(head_dim),
    // and the padded output dims are dropped.
    const size_t pd = head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
    // One f32 sequence, one head: a pool with ceil(seq_len/16) pages and the identity table.
    const int n_pages = (int)((seq_len + 15) / 16) + 1;
    pi_kv_pool pool = nullptr;
    int rc = pi_kv_pool_create(h, n_pages, 16, 1, (int)pd, PI_F32, &pool);
    if (rc) return rc;
    const size_t kv = seq_len * pd;
    const size_t raw = pd == head_dim ? 0 : seq_len * head_dim;  // unpadded rows, copied whole
    const size_t need = 2 * kv + 2 * pd + (size_t)n_pages + 2 + 2 * raw;
    rc = grow(h, &h->h2d_scratch, &h->h2d_floats, need, s, "attention_head staging", false);
    if (rc) {
        pi_kv_pool_destroy(pool);
        return rc;
    }
    float* dk = h->h2d_scratch;
    float* dv = dk + kv;
    float* dq = dv + kv;
    float* dout = dq + pd;
    int32_t* dpt = reinterpret_cast<int32_t*>(dout + pd);
    int32_t* dmeta = dpt + n_pages;  // [start_pos=0, ctx_len]
    float* rk = reinterpret_cast<float*>(dmeta + 2);
    float* rv = rk + raw;
    int32_t* hpt = new (std::nothrow) int32_t[n_pages + 2];
    if (!hpt) {
        pi_kv_pool_destroy(pool);
        return fail(h, PI_ERR_OUT_OF_MEMORY, "attention_head: host allocation");
    }
    for (int i = 0; i < n_pages; ++i) hpt[i] = i;
    hpt[n_pages] = 0;
    hpt[n_pages + 1] = (int32_t)seq_len;
    const size_t rb = head_dim * 4, pb = pd * 4;
    hipError_t e = hipMemsetAsync(dk, 0, (2 * kv + pd) * 4, s);
    if (kv && !raw) {
        if (e == hipSuccess) e = hipMemcpyAsync(dk, h_k_cache, kv * 4, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipMemcpyAsync(dv, h_v_cache, kv * 4, hipMemcpyHostToDevice, s);
    } else if (kv) {  // one host copy per cache, then rows padded on the device
        if (e == hipSuccess) e = hipMemcpyAsync(rk, h_k_cache, raw * 4, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipMemcpyAsync(rv, h_v_cache, raw * 4, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipMemcpy2DAsync(dk, pb, rk, rb, rb, seq_len, hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess) e = hipMemcpy2DAsync(dv, pb, rv, rb, rb, seq_len, hipMemcpyDeviceToDevice, s);
    }
    if (e == hipSuccess) e = hipMemcpyAsync(dq, h_q, rb, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(dpt, hpt, (n_pages + 2) * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    delete[] hpt;
    if (e != hipSuccess) {
        pi_kv_pool_destroy(pool);
        return hip_fail(h, e, "attention_head");
    }
    rc = seq_len ? pi_kv_append(h, pool, dk, dv, PI_F32, dpt, n_pages, dmeta, 1, (int)seq_len, s) : PI_OK;
    if (!rc)
        rc = pi_attn_decode(h, dq, pool, dpt, n_pages, dmeta + 1, 1, 1, PI_GQA_MODULO,
                            1.0f / std::sqrt((float)head_dim), nullptr, dout, s);
    if (!rc) {
        e = hipMemcpyAsync(h_out, dout, rb, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(h, e, "attention_head");
    }
    pi_kv_pool_destroy(pool);
    return rc;
}

// Synchronous host-slice calls: copy in on the handle's stream, run, copy out.
static int stage_in(pi_handle h, size_t floats, float** dev) {
    int rc = grow(h, &h->h2d_scratch, &h->h2d_floats, floats, h->stream, "host-slice staging", false);
    if (rc) return rc;
    *dev = h->h2d_scratch;
    return PI_OK;
}

static int copy_sync(pi_handle h, void* dst, const void* src, size_t bytes, hipMemcpyKind kind,
                     const char* what) {
    if (bytes) PI_HIP(h, hipMemcpyAsync(dst, src, bytes, kind, h->stream), what);
    return PI_OK;
}

int pi_ops_rms_norm(pi_handle h, float* h_out, const float* h_x, const float* h_w, size_t n,
                    float eps) {
    PI_CHECK_HANDLE(h);
    if (!h_out || !h_x || !h_w) return fail(h, PI_ERR_INVALID_ARG, "rms_norm: null slice");
    if (n == 0 || n > (1u << 24)) return fail(h, PI_ERR_INVALID_ARG, "rms_norm: n=%zu", n);
    PI_HIP(h, hipSetDevice(h->device), "rms_norm");
    float* d;
    int rc = stage_in(h, 2 * n, &d);
    if (rc) return rc;
    if ((rc = copy_sync(h, d, h_x, n * 4, hipMemcpyHostToDevice, "rms_norm"))) return rc;
    if ((rc = copy_sync(h, d + n, h_w, n * 4, hipMemcpyHostToDevice, "rms_norm"))) return rc;
    PI_HIP(h, pi::launch_head_rmsnorm(d, d + n, 1, (int)n, (int)n, eps, h->stream), "rms_norm");
    if ((rc = copy_sync(h, h_out, d, n * 4, hipMemcpyDeviceToHost, "rms_norm"))) return rc;
    PI_HIP(h, hipStreamSynchronize(h->stream), "rms_norm");
    return PI_OK;
}

int pi_ops_softmax(pi_handle h, float* h_x, size_t n) {
    PI_CHECK_HANDLE(h);
    if (n == 0) return PI_OK;  // src/ops.rs:161-163
    if (!h_x) return fail(h, PI_ERR_INVALID_ARG, "softmax: null slice");
    if (n > (1u << 28)) return fail(h, PI_ERR_UNSUPPORTED, "softmax: n=%zu", n);
    PI_HIP(h, hipSetDevice(h->device), "softmax");
    float* d;
    int rc = stage_in(h, n, &d);
    if (rc) return rc;
    if ((rc = copy_sync(h, d, h_x, n * 4, hipMemcpyHostToDevice, "softmax"))) return rc;
    PI_HIP(h, pi::launch_softmax(d, (int)n, h->stream), "softmax");
    if ((rc = copy_sync(h, h_x, d, n * 4, hipMemcpyDeviceToHost, "softmax"))) return rc;
    PI_HIP(h, hipStreamSynchronize(h->stream), "softmax");
    return PI_OK;
}

// One q head and one k head rotated in place at `position` with the frequency
// table f (n_pairs entries), NORM (adjacent pairs) or NeoX pairing.
static int rope_one(pi_handle h, float* h_q, float* h_k, size_t position, size_t head_dim,
                    const pi::RopeFreqs& f, int n_pairs, int neox, const char* what) {
    PI_CHECK_HANDLE(h);
    if (!h_q || !h_k) return fail(h, PI_ERR_INVALID_ARG, "%s: null slice", what);
    if (head_dim == 0 || head_dim > 256) return fail(h, PI_ERR_UNSUPPORTED, "%s: head_dim %zu", what, head_dim);
    if (position > (size_t)INT32_MAX) return fail(h, PI_ERR_UNSUPPORTED, "%s: position %zu", what, position);
    if (n_pairs == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), what);
    float* d;
    int rc = stage_in(h, 2 * head_dim + 1, &d);
    if (rc) return rc;
    int32_t* dpos = reinterpret_cast<int32_t*>(d + 2 * head_dim);
    const int32_t pos32 = (int32_t)position;
    if ((rc = copy_sync(h, d, h_q, head_dim * 4, hipMemcpyHostToDevice, what))) return rc;
    if ((rc = copy_sync(h, d + head_dim, h_k, head_dim * 4, hipMemcpyHostToDevice, what))) return rc;
    if ((rc = copy_sync(h, dpos, &pos32, 4, hipMemcpyHostToDevice, what))) return rc;
    PI_HIP(h, pi::launch_rope(d, d + head_dim, dpos, 1, 1, 1, (int)head_dim, n_pairs, neox, f, h->stream), what);
    if ((rc = copy_sync(h, h_q, d, head_dim * 4, hipMemcpyDeviceToHost, what))) return rc;
    if ((rc = copy_sync(h, h_k, d + head_dim, head_dim * 4, hipMemcpyDeviceToHost, what))) return rc;
    PI_HIP(h, hipStreamSynchronize(h->stream), what);
    return PI_OK;
}

int pi_ops_apply_rope(pi_handle h, float* h_q, float* h_k, size_t position, size_t head_dim,
                      size_t rope_dim, float base_freq) {
    if (rope_dim > 256) return fail(h, PI_ERR_UNSUPPORTED, "apply_rope: rope_dim %zu", rope_dim);
    pi::RopeFreqs f;
    std::memset(&f, 0, sizeof f);
    norm_rope_freqs(base_freq, (int)rope_dim, f.f);
    // src/ops.rs:52-64: pairs with 2i+1 >= head_dim are skipped (the kernel checks)
    return rope_one(h, h_q, h_k, position, head_dim, f, (int)(rope_dim / 2), 0, "apply_rope");
}

int pi_ops_apply_rope_with_freqs(pi_handle h, float* h_q, float* h_k, size_t position,
                                 size_t head_dim, const float* h_freqs, size_t n_freqs) {
    if (n_freqs && !h_freqs) return fail(h, PI_ERR_INVALID_ARG, "apply_rope_with_freqs: null freqs");
    if (n_freqs > 128) return fail(h, PI_ERR_UNSUPPORTED, "apply_rope_with_freqs: %zu freqs", n_freqs);
    pi::RopeFreqs f;
    std::memset(&f, 0, sizeof f);
    for (size_t i = 0; i < n_freqs; ++i) f.f[i] = h_freqs[i];
    return rope_one(h, h_q, h_k, position, head_dim, f, (int)n_freqs, 1, "apply_rope_with_freqs");
}

int pi_compute_imrope_freqs(float base, size_t n_rot, const int32_t* sections, float* out) {
    if (!sections || (!out && n_rot >= 2)) return fail(nullptr, PI_ERR_INVALID_ARG, "compute_imrope_freqs: null argument");
    if (n_rot / 2 > 128) return fail(nullptr, PI_ERR_UNSUPPORTED, "compute_imrope_freqs: n_rot %zu", n_rot);
    if (n_rot >= 2) imrope_freqs(base, (int)n_rot, out);
    return PI_OK;
}

int pi_ssm_gated_delta_step(pi_handle h, float* h_out, float* h_state, const float* h_q,
                            const float* h_k, const float* h_v, const float* h_beta,
                            const float* h_g, int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd,
                            int32_t v_hd) {
    PI_CHECK_HANDLE(h);
    if (!h_out || !h_state || !h_q || !h_k || !h_v || !h_beta || !h_g)
        return fail(h, PI_ERR_INVALID_ARG, "gated_delta_step: null slice");
    int rc = gdn_shape_check(h, "gated_delta_step", n_k_heads, n_v_heads, k_hd, v_hd);
    if (rc) return rc;
    PI_HIP(h, hipSetDevice(h->device), "gated_delta_step");
    const size_t nq = (size_t)n_k_heads * k_hd, nv = (size_t)n_v_heads * v_hd;
    const size_t ns = (size_t)n_v_heads * k_hd * v_hd, nh = (size_t)n_v_heads;
    float* d;
    if ((rc = stage_in(h, ns + 2 * nq + 2 * nv + 2 * nh, &d))) return rc;
    float *ds = d, *dq = ds + ns, *dk = dq + nq, *dv = dk + nq, *db = dv + nv, *dg = db + nh,
          *dout = dg + nh;
    if ((rc = copy_sync(h, ds, h_state, ns * 4, hipMemcpyHostToDevice, "gated_delta_step"))) return rc;
    if ((rc = copy_sync(h, dq, h_q, nq * 4, hipMemcpyHostToDevice, "gated_delta_step"))) return rc;
    if ((rc = copy_sync(h, dk, h_k, nq * 4, hipMemcpyHostToDevice, "gated_delta_step"))) return rc;
    if ((rc = copy_sync(h, dv, h_v, nv * 4, hipMemcpyHostToDevice, "gated_delta_step"))) return rc;
    if ((rc = copy_sync(h, db, h_beta, nh * 4, hipMemcpyHostToDevice, "gated_delta_step"))) return rc;
    if ((rc = copy_sync(h, dg, h_g, nh * 4, hipMemcpyHostToDevice, "gated_delta_step"))) return rc;
    PI_HIP(h, pi::launch_gdn_decode(dq, dk, dv, db, dg, ds, dout, 1, n_k_heads, n_v_heads, k_hd,
                                    v_hd, h->stream),
           "gated_delta_step");
    if ((rc = copy_sync(h, h_state, ds, ns * 4, hipMemcpyDeviceToHost, "gated_delta_step"))) return rc;
    if ((rc = copy_sync(h, h_out, dout, nv * 4, hipMemcpyDeviceToHost, "gated_delta_step"))) return rc;
    PI_HIP(h, hipStreamSynchronize(h->stream), "gated_delta_step");
    return PI_OK;
}

int pi_ssm_forward(pi_handle h, float* h_y, const float* h_x, const float* h_conv1d,
                   size_t conv1d_len, const float* h_ssm_a, const float* h_dt_bias,
                   const float* h_alpha, const float* h_beta, size_t beta_len,
                   const float* h_out_w, size_t out_len, float* h_state, size_t d_inner,
                   size_t d_state, size_t d_conv) {
    PI_CHECK_HANDLE(h);
    const char* fn = "ssm_forward";
    if (!h_y || !h_x || !h_ssm_a || !h_dt_bias || !h_alpha || !h_state ||
        (conv1d_len && !h_conv1d) || (beta_len && !h_beta) || (out_len && !h_out_w))
        return fail(h, PI_ERR_INVALID_ARG, "%s: null slice", fn);
    if (d_inner == 0 || d_inner > (1u << 16) || d_state > (1u << 16) || d_conv > (1u << 16))
        return fail(h, PI_ERR_INVALID_ARG, "%s: d_inner=%zu d_state=%zu d_conv=%zu", fn, d_inner,
                    d_state, d_conv);
    // src/ssm/mod.rs:63,101,131 pick the branches by slice length
    const bool has_conv = conv1d_len == d_inner * d_conv;
    const bool has_b = d_state > 0 && beta_len == d_state * d_inner;
    const bool has_out = out_len == d_inner * d_inner;
    const size_t ns = d_state * d_inner, na = d_inner * d_inner;
    const size_t nc = has_conv ? conv1d_len : 0, nb = has_b ? beta_len : 0, no = has_out ? out_len : 0;
    PI_HIP(h, hipSetDevice(h->device), fn);
    // inputs: x, conv, a, dt_bias, alpha, beta, out_w, state; outputs y; scratch 3 d_inner + d_state
    const size_t need = d_inner + nc + ns + d_inner + na + nb + no + ns + d_inner + 3 * d_inner + d_state;
    float* d;
    int rc = stage_in(h, need, &d);
    if (rc) return rc;
    pi::SsmArgs a{};
    float* p = d;
    auto take = [&](size_t n) { float* r = p; p += n; return r; };
    float *dx = take(d_inner), *dw = take(nc), *da = take(ns), *ddt = take(d_inner),
          *dal = take(na), *dbe = take(nb), *dow = take(no), *dst = take(ns), *dy = take(d_inner);
    a.conv_out = take(d_inner);
    a.dt = take(d_inner);
    a.colsum = take(d_inner);
    a.bv = take(d_state);
    const struct { float* dst; const float* src; size_t n; } ins[] = {
        {dx, h_x, d_inner}, {dw, h_conv1d, nc}, {da, h_ssm_a, ns}, {ddt, h_dt_bias, d_inner},
        {dal, h_alpha, na}, {dbe, h_beta, nb}, {dow, h_out_w, no}, {dst, h_state, ns}};
    for (const auto& c : ins)
        if ((rc = copy_sync(h, c.dst, c.src, c.n * 4, hipMemcpyHostToDevice, fn))) return rc;
    a.x = dx;
    a.conv_w = dw;
    a.a = da;
    a.dt_bias = ddt;
    a.alpha = dal;
    a.beta = dbe;
    a.out_w = dow;
    a.state = dst;
    a.y = dy;
    a.d_inner = (int32_t)d_inner;
    a.d_state = (int32_t)d_state;
    a.d_conv = (int32_t)d_conv;
    a.has_conv = has_conv;
    a.has_b = has_b;
    a.has_out = has_out;
    PI_HIP(h, pi::launch_ssm_forward(a, h->stream), fn);
    if ((rc = copy_sync(h, h_y, dy, d_inner * 4, hipMemcpyDeviceToHost, fn))) return rc;
    if ((rc = copy_sync(h, h_state, dst, ns * 4, hipMemcpyDeviceToHost, fn))) return rc;
    PI_HIP(h, hipStreamSynchronize(h->stream), fn);
    return PI_OK;
}

// ---- attention layer cache ------------------------------------------------------------

namespace {
constexpr int kLayerRows = 256;  // query rows per decode launch of a multi-token forward
}

int pi_attn_layer_create(pi_handle h, int32_t max_tokens, int32_t n_heads, int32_t n_kv_heads,
                         int32_t head_dim, int32_t kv_dtype, const float* h_q_norm_w,
                         const float* h_k_norm_w, float eps, int32_t rope_dim, float rope_base,
                         const int32_t* h_sections, int32_t gqa_mode, pi_attn_layer* out) {
    return pi_attn_layer_create_dims(h, max_tokens, n_heads, n_kv_heads, head_dim, head_dim,
                                     head_dim, kv_dtype, h_q_norm_w, h_k_norm_w, eps, rope_dim,
                                     rope_base, h_sections, gqa_mode, out);
}

int pi_attn_layer_create_dims(pi_handle h, int32_t max_tokens, int32_t n_heads,
                              int32_t n_kv_heads, int32_t q_head_dim, int32_t head_dim,
                              int32_t v_head_dim, int32_t kv_dtype, const float* h_q_norm_w,
                              const float* h_k_norm_w, float eps, int32_t rope_dim,
                              float rope_base, const int32_t* h_sections, int32_t gqa_mode,
                              pi_attn_layer* out) {
    PI_CHECK_HANDLE(h);
    if (!out) return fail(h, PI_ERR_INVALID_ARG, "pi_attn_layer_create: out is null");
    *out = nullptr;
    // src/model/mod.rs:976-982,1043-1190: attention reads the first head_dim dims of each
    // query head, so the query head is at least that wide; any value width
    if (q_head_dim < head_dim || v_head_dim <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_layer_create: q_head_dim=%d head_dim=%d v_head_dim=%d",
                    q_head_dim, head_dim, v_head_dim);
    if (head_dim <= 0 || head_dim > 256)
        return fail(h, PI_ERR_UNSUPPORTED, "pi_attn_layer_create: head_dim %d (1..256)", head_dim);
    if (max_tokens <= 0 || n_heads <= 0 || n_kv_heads <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_layer_create: max_tokens=%d n_heads=%d n_kv_heads=%d",
                    max_tokens, n_heads, n_kv_heads);
    if (gqa_mode != PI_GQA_MODULO && gqa_mode != PI_GQA_GROUPED)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_layer_create: gqa_mode %d", gqa_mode);
    if (gqa_mode == PI_GQA_GROUPED && n_heads % n_kv_heads != 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_layer_create: grouped head map with n_heads %d not a multiple of n_kv_heads %d",
                    n_heads, n_kv_heads);
    pi_attn_layer L = new (std::nothrow) pi_attn_layer_s();
    if (!L) return fail(h, PI_ERR_OUT_OF_MEMORY, "pi_attn_layer_create: host allocation");
    L->owner = h;
    L->max_pages = (max_tokens + pi::kPageTokens - 1) / pi::kPageTokens;
    L->n_heads = n_heads;
    L->n_kv = n_kv_heads;
    L->dim = head_dim;
    // a head narrower than a kernel width runs zero-padded to the next one: zero dims add
    // nothing to q.k and give zero output dims, and the scale and the norm keep head_dim
    L->pdim = head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
    L->q_dim = q_head_dim;
    L->v_dim = v_head_dim;
    L->kv_dtype = kv_dtype;
    L->rope_dim = rope_dim;
    L->gqa_mode = gqa_mode;
    L->eps = eps;
    L->rope_base = rope_base;
    if (h_sections) {
        L->has_sections = true;
        std::memcpy(L->sections, h_sections, sizeof L->sections);
    }
    auto undo = [&](int rc) {
        pi_attn_layer_destroy(L);
        return rc;
    };
    int rc = pi_kv_pool_create(h, L->max_pages, pi::kPageTokens, n_kv_heads, L->pdim, kv_dtype, &L->pool);
    if (rc) return undo(rc);
    hipError_t e = hipSuccess;
    const size_t pt = (size_t)kLayerRows * L->max_pages;
    const size_t wb = (size_t)L->pdim * sizeof(float);
    e = hipMalloc(reinterpret_cast<void**>(&L->d_pt), pt * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&L->d_ctx), (kLayerRows + 1) * sizeof(int32_t));
    // norm weights zero past head_dim, so the padding dims stay zero after the norm
    for (auto [dst, src] : {std::pair<float**, const float*>{&L->d_qn, h_q_norm_w}, {&L->d_kn, h_k_norm_w}}) {
        if (e != hipSuccess || !src) continue;
        e = hipMalloc(reinterpret_cast<void**>(dst), wb);
        if (e == hipSuccess) e = hipMemset(*dst, 0, wb);
        if (e == hipSuccess) e = hipMemcpy(*dst, src, head_dim * sizeof(float), hipMemcpyHostToDevice);
    }
    if (e == hipSuccess) {
        std::vector<int32_t> rows(pt);
        for (size_t i = 0; i < pt; ++i) rows[i] = (int32_t)(i % L->max_pages);
        e = hipMemcpy(L->d_pt, rows.data(), pt * sizeof(int32_t), hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) return undo(hip_fail(h, e, "pi_attn_layer_create"));
    *out = L;
    return PI_OK;
}

void pi_attn_layer_destroy(pi_attn_layer L) {
    if (!L) return;
    (void)hipSetDevice(L->owner->device);
    (void)hipDeviceSynchronize();
    pi_kv_pool_destroy(L->pool);
    (void)hipFree(L->d_pt);
    (void)hipFree(L->d_ctx);
    (void)hipFree(L->d_qn);
    (void)hipFree(L->d_kn);
    (void)hipFree(L->d_buf);
    delete L;
}

void pi_attn_layer_reset(pi_attn_layer L) {
    if (L) L->seq_len = 0;
}

int32_t pi_attn_layer_seq_len(pi_attn_layer L) { return L ? L->seq_len : 0; }

// The attention step of forward for n tokens whose q, k, v (and gate) are on the
// device, in rows of pdim floats (zero past head_dim): norm + RoPE + append at
// positions seq_len .., then attention for every token over the keys up to its own.
// For n > 1 an f16 cache runs the flash prefill and an f32 cache the f32 prefill,
// both reading K / V straight from the layer's pages; a single token runs one decode
// row.  Positions and row lengths are written on the device, so the step enqueues
// work on `s` and never waits for it.
static int attn_layer_step(pi_handle h, pi_attn_layer L, float* dq, float* dk, const float* dv,
                           const float* dg, int32_t n, float* dout, hipStream_t s) {
    const int prev = L->seq_len;
    if ((long long)prev + n > (long long)L->max_pages * pi::kPageTokens)
        return fail(h, PI_ERR_OUT_OF_MEMORY, "attention layer: %d + %d tokens exceed the layer cache of %d",
                    prev, n, L->max_pages * pi::kPageTokens);
    void* sv = reinterpret_cast<void*>(s);
    const int D = L->pdim;  // row width; the head's own width is L->dim
    const size_t nq = (size_t)n * L->n_heads * D;
    int rc;
    // the callers stage anything else; checked here too, before the first launch
    if (((uintptr_t)dq | (uintptr_t)dout | (uintptr_t)dg) & 15)
        return fail(h, PI_ERR_INVALID_ARG, "attention layer: q, gate and out rows must be 16-byte aligned");
    // The prologue (norm, RoPE, append at positions prev ..) takes its start position as a
    // scalar and writes the context lengths of the decode rows of the step (row i: prev + i +
    // 1 keys) into d_ctx, so no launch of its own fills them.
    const bool rows = !(n > 1 && (L->kv_dtype == PI_F16 || L->kv_dtype == PI_F32));
    {
        const pi::KvGeom& g = L->pool->g;
        const int rd = L->rope_dim <= 0 ? L->dim : std::min(L->rope_dim, L->dim);
        if (rd / 2 > 128) return fail(h, PI_ERR_UNSUPPORTED, "attention layer: rope_dim %d", rd);
        pi::RopeFreqs f;
        std::memset(&f, 0, sizeof f);
        if (L->has_sections) imrope_freqs(L->rope_base, rd, f.f);
        else norm_rope_freqs(L->rope_base, rd, f.f);
        PI_HIP(h, pi::launch_attn_prologue(dq, dk, dv, L->d_qn, L->d_kn, L->eps, f, rd / 2,
                                           L->has_sections ? 1 : 0, g, L->d_pt, L->max_pages, nullptr,
                                           1, n, L->n_heads, s, prev, L->d_ctx,
                                           rows ? std::min(n, kLayerRows) : 0, L->dim),
               "attention layer");
    }
    const float scale = 1.0f / std::sqrt((float)L->dim);
    // the prefill kernels apply a 16-byte-aligned gate where they write the output; another
    // gate takes a launch of its own after them
    const float* dg_fused = dg && !((uintptr_t)dg & 15) ? dg : nullptr;
    if (n > 1 && L->kv_dtype == PI_F16) {
        // causal flash attention over the sequence's pages (the chunk's own K / V appended by
        // the prologue), q read in f32
        if ((rc = ws_begin(h, s, "attention layer"))) return rc;
        const size_t need = pi::prefill_ws_floats(1, n, L->n_heads, L->n_kv, D, 1);
        if (need && (rc = grow(h, &h->pfs_buf, &h->pfs_floats, need, s, "attention layer workspace", false)))
            return rc;
        PI_HIP(h, pi::launch_prefill_pool(L->pool->g, dq, 1, L->d_pt, prev, n, L->n_heads, L->gqa_mode,
                                          scale, dout, h->pfs_buf, h->pfs_floats, s, dg_fused),
               "attention layer");
        if ((rc = ws_end(h, s, "attention layer"))) return rc;
        if (dg && !dg_fused) PI_HIP(h, pi::launch_apply_gate(dout, dg, nq, s), "attention layer");
    } else if (n > 1 && L->kv_dtype == PI_F32) {
        // causal attention straight from the f32 pages, at f32 accuracy
        PI_HIP(h, pi::launch_prefill_f32(L->pool->g, dq, L->d_pt, L->max_pages, prev, n, L->n_heads,
                                         L->gqa_mode, scale, dout, s, dg_fused),
               "attention layer");
        if (dg && !dg_fused) PI_HIP(h, pi::launch_apply_gate(dout, dg, nq, s), "attention layer");
    } else {
        // one decode row per token over the paged cache: row i sees prev + i + 1 keys (the
        // prologue wrote the first kLayerRows lengths)
        for (int r0 = 0; r0 < n; r0 += kLayerRows) {
            const int nr = std::min(kLayerRows, n - r0);
            if (r0 > 0) PI_HIP(h, pi::launch_fill_iota(L->d_ctx, nr, prev + r0 + 1, s), "attention layer");
            const size_t off = (size_t)r0 * L->n_heads * D;
            if ((rc = attn_decode_ws(h, "attention layer", dq + off, L->pool, L->d_pt, L->max_pages, L->d_ctx,
                                     nr, L->n_heads, L->gqa_mode, scale, dg ? dg + off : nullptr,
                                     dout + off, s, prev + r0 + nr)))
                return rc;
        }
    }
    L->seq_len = prev + n;
    return PI_OK;
}

// The layer's inputs in the step's packed form, [n][H][pdim] rows (src/model/mod.rs:
// 1043-1190): the first head_dim dims of each query head; V cut or zero-padded to head_dim
// (output dims at or past the value width stay zero, as the reference's head_out); the gate
// as the flat prefix of n_heads * head_dim values of each token's n_heads * q_head_dim
// (the reference multiplies attn_out[i] by sigmoid(output_gate[i]), :1192-1196), head h's
// dims the values h * head_dim ..  Every row is zero past head_dim out to pdim.  k (at
// head_dim wide rows) is packed only when dk is given (pdim > head_dim).
static int pack_layer_inputs(pi_handle h, pi_attn_layer L, const float* q, const float* k,
                             const float* v, const float* g, int32_t n, float* dq, float* dk,
                             float* dv, float* dg, hipStream_t s, const char* what) {
    const size_t D = L->dim, W = L->pdim, Hq = L->n_heads, Hkv = L->n_kv, qd = L->q_dim, vd = L->v_dim;
    const int d = (int)D, w = (int)W;
    PI_HIP(h, pi::launch_pack_rows(dq, q, n, (int)Hq, d, w, Hq * qd, qd, Hq * W, W, s), what);
    if (dk) PI_HIP(h, pi::launch_pack_rows(dk, k, n, (int)Hkv, d, w, Hkv * D, D, Hkv * W, W, s), what);
    PI_HIP(h, pi::launch_pack_rows(dv, v, n, (int)Hkv, (int)std::min(D, vd), w, Hkv * vd, vd, Hkv * W, W, s),
           what);
    if (g) PI_HIP(h, pi::launch_pack_rows(dg, g, n, (int)Hq, d, w, Hq * qd, D, Hq * W, W, s), what);
    return PI_OK;
}

// The step's outputs back to the caller's widths: q's first head_dim dims of each query
// head (normalised and rotated; the rest of a q_head_dim row untouched), and, where the
// step ran on wider rows (dk / dout given), k and out cut to head_dim.
static int unpack_layer_outputs(pi_handle h, pi_attn_layer L, int32_t n, const float* dq, float* q,
                                const float* dk, float* k, const float* dout, float* out,
                                hipStream_t s, const char* what) {
    const size_t D = L->dim, W = L->pdim, Hq = L->n_heads, Hkv = L->n_kv, qd = L->q_dim;
    const int d = (int)D;
    PI_HIP(h, pi::launch_pack_rows(q, dq, n, (int)Hq, d, d, Hq * W, W, Hq * qd, qd, s), what);
    if (dk) PI_HIP(h, pi::launch_pack_rows(k, dk, n, (int)Hkv, d, d, Hkv * W, W, Hkv * D, D, s), what);
    if (dout) PI_HIP(h, pi::launch_pack_rows(out, dout, n, (int)Hq, d, d, Hq * W, W, Hq * D, D, s), what);
    return PI_OK;
}

// A small host-slice call (a decode token) stages its slices through one pinned host
// buffer: one host-to-device and one device-to-host copy per call instead of one per
// slice.  Larger calls copy each slice directly (their time is the bytes, not the copies).
constexpr size_t kPinnedMaxFloats = (size_t)1 << 20;  // 4 MiB each way

static bool pinned_staging(pi_handle h, size_t floats) {
    if (floats > kPinnedMaxFloats) return false;
    if (floats <= h->pin_floats) return true;
    if (h->pin) (void)hipHostFree(h->pin);  // the previous call has synchronised
    h->pin = nullptr;
    h->pin_floats = 0;
    const size_t n = kPinnedMaxFloats;
    if (hipHostMalloc(reinterpret_cast<void**>(&h->pin), n * sizeof(float), hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        h->pin = nullptr;
        return false;
    }
    h->pin_floats = n;
    return true;
}

int pi_attn_layer_forward(pi_handle h, pi_attn_layer L, float* h_q, float* h_k, const float* h_v,
                          const float* h_gate, int32_t n_tokens, float* h_out) {
    PI_CHECK_HANDLE(h);
    if (!L || !h_q || !h_k || !h_v || !h_out)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_layer_forward: null argument");
    if (n_tokens < 0) return fail(h, PI_ERR_INVALID_ARG, "pi_attn_layer_forward: n_tokens=%d", n_tokens);
    if (n_tokens == 0) return PI_OK;
    if ((long long)L->seq_len + n_tokens > (long long)L->max_pages * pi::kPageTokens)
        return fail(h, PI_ERR_OUT_OF_MEMORY, "pi_attn_layer_forward: %d + %d tokens exceed the layer cache of %d",
                    L->seq_len, n_tokens, L->max_pages * pi::kPageTokens);
    hipStream_t s = h->stream;
    const char* what = "pi_attn_layer_forward";
    PI_HIP(h, hipSetDevice(h->device), what);
    const int D = L->dim, W = L->pdim;
    const size_t nq = (size_t)n_tokens * L->n_heads * D, nk = (size_t)n_tokens * L->n_kv * D;
    const size_t nqw = (size_t)n_tokens * L->n_heads * W, nkw = (size_t)n_tokens * L->n_kv * W;
    // Slices as the caller holds them: q and gate [n][Hq][q_dim], v [n][Hkv][v_dim], k and
    // out [n][H][head_dim].  With distinct widths, or a head_dim the step runs padded to
    // pdim, they arrive whole in "io" regions and are packed on the device (2D copies from
    // pageable memory would go row by row).
    const bool packed = L->q_dim == D && L->v_dim == D && W == D;
    const bool wide = W != D;
    const size_t qin = (size_t)n_tokens * L->n_heads * L->q_dim;
    const size_t vin = (size_t)n_tokens * L->n_kv * L->v_dim;
    const size_t gin = h_gate ? qin : 0;
    // device staging: [out | q io | k | v io | gate io] (+ packed q, v, gate, and k and out
    // at pdim wide rows, when not packed), so the inputs (q, k, v, gate) and the outputs
    // (out, q, k) are each one contiguous run.  Every region the kernels address starts on
    // a 16-byte boundary: with distinct widths the io regions' lengths need not be
    // multiples of 4 floats, so the packed regions after them start at the next 16-byte
    // boundary (the packed regions are whole pdim rows).
    const size_t pk0 = (nq + qin + nk + vin + qin + 3) & ~(size_t)3;
    const size_t need = packed ? pk0 : pk0 + 2 * nqw + nkw + (wide ? nkw + nqw : 0);
    int rc = grow(h, &L->d_buf, &L->buf_floats, need, s, "pi_attn_layer_forward staging", false);
    if (rc) return rc;
    float *dout = L->d_buf, *qio = dout + nq, *dk = qio + qin, *vio = dk + nk, *gio = vio + vin;
    float *dq = qio, *dv = vio, *dg = gio, *dkw = dk, *doutw = dout;
    if (!packed) {
        dq = L->d_buf + pk0;
        dv = dq + nqw;
        dg = dv + nkw;
        if (wide) {
            dkw = dg + nqw;
            doutw = dkw + nkw;
        }
    }
    const size_t in_f = qin + nk + vin + gin, out_f = nq + qin + nk;
    const bool pin = pinned_staging(h, std::max(in_f, out_f));
    if (pin) {
        float* p = h->pin;
        std::memcpy(p, h_q, qin * 4);
        std::memcpy(p + qin, h_k, nk * 4);
        std::memcpy(p + qin + nk, h_v, vin * 4);
        if (h_gate) std::memcpy(p + qin + nk + vin, h_gate, gin * 4);
        if ((rc = copy_sync(h, qio, p, in_f * 4, hipMemcpyHostToDevice, what))) return rc;
    } else {
        if ((rc = copy_sync(h, qio, h_q, qin * 4, hipMemcpyHostToDevice, what))) return rc;
        if ((rc = copy_sync(h, dk, h_k, nk * 4, hipMemcpyHostToDevice, what))) return rc;
        if ((rc = copy_sync(h, vio, h_v, vin * 4, hipMemcpyHostToDevice, what))) return rc;
        if (h_gate && (rc = copy_sync(h, gio, h_gate, gin * 4, hipMemcpyHostToDevice, what))) return rc;
    }
    if (!packed && (rc = pack_layer_inputs(h, L, qio, dk, vio, h_gate ? gio : nullptr, n_tokens, dq,
                                           wide ? dkw : nullptr, dv, dg, s, what)))
        return rc;
    if ((rc = attn_layer_step(h, L, dq, dkw, dv, h_gate ? dg : nullptr, n_tokens, doutw, s))) return rc;
    // q and k go back normalised and rotated (only the first head_dim dims of a query head)
    if (!packed && (rc = unpack_layer_outputs(h, L, n_tokens, dq, qio, wide ? dkw : nullptr, dk,
                                              wide ? doutw : nullptr, dout, s, what)))
        return rc;
    if (pin) {
        if ((rc = copy_sync(h, h->pin, dout, out_f * 4, hipMemcpyDeviceToHost, what))) return rc;
        PI_HIP(h, hipStreamSynchronize(s), what);
        std::memcpy(h_out, h->pin, nq * 4);
        std::memcpy(h_q, h->pin + nq, qin * 4);
        std::memcpy(h_k, h->pin + nq + qin, nk * 4);
        return PI_OK;
    }
    if ((rc = copy_sync(h, h_out, dout, nq * 4, hipMemcpyDeviceToHost, what))) return rc;
    if ((rc = copy_sync(h, h_q, qio, qin * 4, hipMemcpyDeviceToHost, what))) return rc;
    if ((rc = copy_sync(h, h_k, dk, nk * 4, hipMemcpyDeviceToHost, what))) return rc;
    PI_HIP(h, hipStreamSynchronize(s), what);
    return PI_OK;
}

int pi_attn_layer_forward_dev(pi_handle h, pi_attn_layer L, float* d_q, float* d_k,
                              const float* d_v, const float* d_gate, int32_t n_tokens,
                              float* d_out, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!L || !d_q || !d_k || !d_v || !d_out)
        return fail(h, PI_ERR_INVALID_ARG, "pi_attn_layer_forward_dev: null argument");
    if (n_tokens < 0) return fail(h, PI_ERR_INVALID_ARG, "pi_attn_layer_forward_dev: n_tokens=%d", n_tokens);
    if (n_tokens == 0) return PI_OK;
    const char* what = "pi_attn_layer_forward_dev";
    if ((long long)L->seq_len + n_tokens > (long long)L->max_pages * pi::kPageTokens)
        return fail(h, PI_ERR_OUT_OF_MEMORY, "%s: %d + %d tokens exceed the layer cache of %d", what,
                    L->seq_len, n_tokens, L->max_pages * pi::kPageTokens);
    PI_HIP(h, hipSetDevice(h->device), what);
    hipStream_t s = pick(h, stream);
    // The step's kernels move q, the gate and out in 16-byte groups.  Rows already in the
    // step's packed form at such addresses go straight in; otherwise they are staged in the
    // layer's buffer (decided before anything is launched, so a call never fails half done).
    const bool wide = L->pdim != L->dim;
    const bool packed = L->q_dim == L->dim && L->v_dim == L->dim && !wide;
    const bool out_ok = !((uintptr_t)d_out & 15);
    if (packed && out_ok && !(((uintptr_t)d_q | (uintptr_t)d_gate) & 15))
        return attn_layer_step(h, L, d_q, d_k, d_v, d_gate, n_tokens, d_out, s);
    const int W = L->pdim;
    const size_t nqw = (size_t)n_tokens * L->n_heads * W, nkw = (size_t)n_tokens * L->n_kv * W;
    int rc = grow(h, &L->d_buf, &L->buf_floats, 3 * nqw + nkw + (wide ? nkw : 0), s,
                  "pi_attn_layer_forward_dev staging", false);
    if (rc) return rc;
    // [q | gate | v | out | k (pdim wide rows, when wider than head_dim)]
    float *dq = L->d_buf, *dg = dq + nqw, *dv = dg + nqw, *ds = dv + nkw, *dkw = wide ? ds + nqw : nullptr;
    if ((rc = pack_layer_inputs(h, L, d_q, d_k, d_v, d_gate, n_tokens, dq, dkw, dv, dg, s, what))) return rc;
    const bool direct = out_ok && !wide;  // out written in place
    if ((rc = attn_layer_step(h, L, dq, wide ? dkw : d_k, dv, d_gate ? dg : nullptr, n_tokens,
                              direct ? d_out : ds, s)))
        return rc;
    if (!direct && !wide) PI_HIP(h, hipMemcpyAsync(d_out, ds, nqw * 4, hipMemcpyDeviceToDevice, s), what);
    return unpack_layer_outputs(h, L, n_tokens, dq, d_q, dkw, d_k, wide ? ds : nullptr, d_out, s, what);
}

// ---- gated-DeltaNet layer state -------------------------------------------------------

// A layer with k_hd = v_hd = 128 and d_conv 4 runs a one-token step as one
// launch (gdn_step_kernel), alternating two conv-state buffers.
static bool gdn_one_launch_step(const pi_gdn_layer_s* L) {
    return L->dk == 128 && L->dv == 128 && L->d_conv == 4;
}

int pi_gdn_layer_create(pi_handle h, int32_t n_k_heads, int32_t n_v_heads, int32_t k_hd,
                        int32_t v_hd, int32_t d_conv, const float* h_conv_w, const float* h_ssm_a,
                        const float* h_dt_bias, const float* h_norm_w, float eps,
                        pi_gdn_layer* out) {
    PI_CHECK_HANDLE(h);
    if (!out || !h_conv_w || !h_ssm_a || !h_dt_bias || !h_norm_w)
        return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_layer_create: null argument");
    *out = nullptr;
    int rc = gdn_shape_check(h, "pi_gdn_layer_create", n_k_heads, n_v_heads, k_hd, v_hd);
    if (rc) return rc;
    if (d_conv < 1 || d_conv > 8) return fail(h, PI_ERR_UNSUPPORTED, "pi_gdn_layer_create: d_conv %d", d_conv);
    pi_gdn_layer L = new (std::nothrow) pi_gdn_layer_s();
    if (!L) return fail(h, PI_ERR_OUT_OF_MEMORY, "pi_gdn_layer_create: host allocation");
    L->owner = h;
    L->hk = n_k_heads;
    L->hv = n_v_heads;
    L->dk = k_hd;
    L->dv = v_hd;
    L->d_conv = d_conv;
    L->conv_dim = 2 * n_k_heads * k_hd + n_v_heads * v_hd;
    L->eps = eps;
    const size_t wn = (size_t)L->conv_dim * d_conv, cs = (size_t)(d_conv - 1) * L->conv_dim;
    const size_t sn = (size_t)n_v_heads * k_hd * v_hd;
    hipError_t e = hipSetDevice(h->device);
    auto alloc = [&](float** p, size_t n) {
        if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(p), std::max<size_t>(n, 1) * sizeof(float));
    };
    alloc(&L->d_w, wn);
    alloc(&L->d_ssm_a, n_v_heads);
    alloc(&L->d_dt, n_v_heads);
    alloc(&L->d_norm, v_hd);
    alloc(&L->d_conv_state, cs);
    if (gdn_one_launch_step(L)) alloc(&L->d_conv_alt, cs);
    alloc(&L->d_state, sn);
    if (e == hipSuccess) e = hipMemcpy(L->d_w, h_conv_w, wn * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(L->d_ssm_a, h_ssm_a, n_v_heads * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(L->d_dt, h_dt_bias, n_v_heads * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(L->d_norm, h_norm_w, v_hd * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess && cs) e = hipMemset(L->d_conv_state, 0, cs * 4);
    if (e == hipSuccess) e = hipMemset(L->d_state, 0, sn * 4);
    if (e != hipSuccess) {
        rc = hip_fail(h, e, "pi_gdn_layer_create");
        pi_gdn_layer_destroy(L);
        return rc;
    }
    *out = L;
    return PI_OK;
}

void pi_gdn_layer_destroy(pi_gdn_layer L) {
    if (!L) return;
    (void)hipSetDevice(L->owner->device);
    (void)hipDeviceSynchronize();
    for (float* p : {L->d_w, L->d_ssm_a, L->d_dt, L->d_norm, L->d_conv_state, L->d_conv_alt, L->d_state,
                     L->d_buf})
        (void)hipFree(p);
    delete L;
}

int pi_gdn_layer_reset(pi_handle h, pi_gdn_layer L) {
    PI_CHECK_HANDLE(h);
    if (!L) return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_layer_reset: null layer");
    PI_HIP(h, hipSetDevice(h->device), "pi_gdn_layer_reset");
    // forward_dev may have left steps on any stream (a caller's non-blocking stream
    // included) that still read and write these states: wait for all of the device's
    // work, then zero on the handle's stream and wait for that too
    PI_HIP(h, hipDeviceSynchronize(), "pi_gdn_layer_reset");
    const size_t cs = (size_t)(L->d_conv - 1) * L->conv_dim;
    if (cs) PI_HIP(h, hipMemsetAsync(L->d_conv_state, 0, cs * 4, h->stream), "pi_gdn_layer_reset");
    if (cs && L->d_conv_alt) PI_HIP(h, hipMemsetAsync(L->d_conv_alt, 0, cs * 4, h->stream), "pi_gdn_layer_reset");
    PI_HIP(h, hipMemsetAsync(L->d_state, 0, (size_t)L->hv * L->dk * L->dv * 4, h->stream), "pi_gdn_layer_reset");
    PI_HIP(h, hipStreamSynchronize(h->stream), "pi_gdn_layer_reset");
    return PI_OK;
}

// The GDN step of forward for n tokens on the device (src/model/mod.rs:750-932):
// conv1d + SiLU with the rolling state, the q / k / v split, the gates, the
// delta rule (chunked for n > 1) and RMSNormGated x SiLU(z).  Enqueued on `s`.
static int gdn_layer_step(pi_handle h, pi_gdn_layer L, const float* dx, const float* dz,
                          const float* dbr, const float* dar, int32_t n_tokens, float* dout,
                          hipStream_t s) {
    void* sv = reinterpret_cast<void*>(s);
    if (n_tokens == 1 && L->d_conv_alt && !(((uintptr_t)dz | (uintptr_t)dout) & 15)) {
        PI_HIP(h, pi::launch_gdn_step(dx, L->d_conv_state, L->d_conv_alt, L->d_w, dz, dbr, dar,
                                      L->d_ssm_a, L->d_dt, L->d_norm, L->eps, L->d_state, dout,
                                      L->hk, L->hv, s),
               "gdn layer step");
        std::swap(L->d_conv_state, L->d_conv_alt);  // later launches on this stream see the new state
        return PI_OK;
    }
    const size_t n = (size_t)n_tokens, C = L->conv_dim, kd = (size_t)L->hk * L->dk;
    const size_t vd = (size_t)L->hv * L->dv, nh = (size_t)L->hv;
    // activation, q, k, v, beta, g
    const size_t need = n * C + 2 * n * kd + n * vd + 2 * n * nh;
    int rc = grow(h, &L->d_buf, &L->buf_floats, need, s, "gdn layer staging", false);
    if (rc) return rc;
    float *act = L->d_buf, *dq = act + n * C, *dk = dq + n * kd, *dv = dk + n * kd;
    float *db = dv + n * vd, *dg = db + n * nh;
    if ((rc = pi_gdn_conv1d(h, dx, L->d_conv_state, L->d_w, act, 1, n_tokens, (int32_t)C, L->d_conv, sv)))
        return rc;
    if (n == 1) {  // one token's row already holds q, k and v back to back
        dq = act;
        dk = act + kd;
        dv = act + 2 * kd;
    } else {
        PI_HIP(h, hipMemcpy2DAsync(dq, kd * 4, act, C * 4, kd * 4, n, hipMemcpyDeviceToDevice, s), "gdn layer");
        PI_HIP(h, hipMemcpy2DAsync(dk, kd * 4, act + kd, C * 4, kd * 4, n, hipMemcpyDeviceToDevice, s), "gdn layer");
        PI_HIP(h, hipMemcpy2DAsync(dv, vd * 4, act + 2 * kd, C * 4, vd * 4, n, hipMemcpyDeviceToDevice, s), "gdn layer");
    }
    if ((rc = pi_gdn_gates(h, dbr, dar, L->d_ssm_a, L->d_dt, db, dg, n_tokens, L->hv, sv))) return rc;
    if (n_tokens > 1)
        rc = pi_gdn_prefill(h, dq, dk, dv, db, dg, L->d_state, dout, n_tokens, L->hk, L->hv, L->dk,
                            L->dv, 64, sv);
    else
        rc = pi_gdn_decode(h, dq, dk, dv, db, dg, L->d_state, dout, 1, L->hk, L->hv, L->dk, L->dv, sv);
    if (rc) return rc;
    return pi_gdn_rmsnorm_gated(h, dout, dz, L->d_norm, n_tokens, L->hv, L->dv, L->eps, sv);
}

int pi_gdn_layer_forward(pi_handle h, pi_gdn_layer L, const float* h_qkv, const float* h_z,
                         const float* h_beta_raw, const float* h_a_raw, int32_t n_tokens,
                         float* h_out) {
    PI_CHECK_HANDLE(h);
    if (!L || !h_qkv || !h_z || !h_beta_raw || !h_a_raw || !h_out)
        return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_layer_forward: null argument");
    if (n_tokens < 0) return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_layer_forward: n_tokens=%d", n_tokens);
    if (n_tokens == 0) return PI_OK;
    hipStream_t s = h->stream;
    PI_HIP(h, hipSetDevice(h->device), "pi_gdn_layer_forward");
    const size_t n = (size_t)n_tokens, C = L->conv_dim;
    const size_t vd = (size_t)L->hv * L->dv, nh = (size_t)L->hv;
    // host-slice I/O: qkv, z, beta_raw, a_raw, out
    const size_t need = n * C + 2 * n * vd + 2 * n * nh;
    int rc = grow(h, &h->h2d_scratch, &h->h2d_floats, need, s, "pi_gdn_layer_forward staging", false);
    if (rc) return rc;
    float *dx = h->h2d_scratch, *dz = dx + n * C, *dbr = dz + n * vd, *dar = dbr + n * nh;
    float* dout = dar + n * nh;
    const size_t in_f = n * C + n * vd + 2 * n * nh;
    const bool pin = pinned_staging(h, in_f);  // the four inputs as one copy (small calls)
    if (pin) {
        std::memcpy(h->pin, h_qkv, n * C * 4);
        std::memcpy(h->pin + n * C, h_z, n * vd * 4);
        std::memcpy(h->pin + n * C + n * vd, h_beta_raw, n * nh * 4);
        std::memcpy(h->pin + n * C + n * vd + n * nh, h_a_raw, n * nh * 4);
        if ((rc = copy_sync(h, dx, h->pin, in_f * 4, hipMemcpyHostToDevice, "pi_gdn_layer_forward"))) return rc;
    } else {
        if ((rc = copy_sync(h, dx, h_qkv, n * C * 4, hipMemcpyHostToDevice, "pi_gdn_layer_forward"))) return rc;
        if ((rc = copy_sync(h, dz, h_z, n * vd * 4, hipMemcpyHostToDevice, "pi_gdn_layer_forward"))) return rc;
        if ((rc = copy_sync(h, dbr, h_beta_raw, n * nh * 4, hipMemcpyHostToDevice, "pi_gdn_layer_forward"))) return rc;
        if ((rc = copy_sync(h, dar, h_a_raw, n * nh * 4, hipMemcpyHostToDevice, "pi_gdn_layer_forward"))) return rc;
    }
    if ((rc = gdn_layer_step(h, L, dx, dz, dbr, dar, n_tokens, dout, s))) return rc;
    if (pin && n * vd <= h->pin_floats) {
        if ((rc = copy_sync(h, h->pin, dout, n * vd * 4, hipMemcpyDeviceToHost, "pi_gdn_layer_forward"))) return rc;
        PI_HIP(h, hipStreamSynchronize(s), "pi_gdn_layer_forward");
        std::memcpy(h_out, h->pin, n * vd * 4);
        return PI_OK;
    }
    if ((rc = copy_sync(h, h_out, dout, n * vd * 4, hipMemcpyDeviceToHost, "pi_gdn_layer_forward"))) return rc;
    PI_HIP(h, hipStreamSynchronize(s), "pi_gdn_layer_forward");
    return PI_OK;
}

int pi_gdn_layer_forward_dev(pi_handle h, pi_gdn_layer L, const float* d_qkv, const float* d_z,
                             const float* d_beta_raw, const float* d_a_raw, int32_t n_tokens,
                             float* d_out, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!L || !d_qkv || !d_z || !d_beta_raw || !d_a_raw || !d_out)
        return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_layer_forward_dev: null argument");
    if (n_tokens < 0) return fail(h, PI_ERR_INVALID_ARG, "pi_gdn_layer_forward_dev: n_tokens=%d", n_tokens);
    if (n_tokens == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_gdn_layer_forward_dev");
    return gdn_layer_step(h, L, d_qkv, d_z, d_beta_raw, d_a_raw, n_tokens, d_out, pick(h, stream));
}

// ---- TurboQuant compressed KV ------------------------------------------------------

int pi_tq_generate(int32_t dim, uint64_t seed, float* h_rotation, float* h_qjl) {
    if (!h_rotation || !h_qjl) return fail(nullptr, PI_ERR_INVALID_ARG, "pi_tq_generate: null argument");
    if (dim <= 0 || dim > 4096) return fail(nullptr, PI_ERR_INVALID_ARG, "pi_tq_generate: dim %d", dim);
    tq_matrices(dim, seed, h_rotation, h_qjl);
    return PI_OK;
}

int pi_tq_pool_create(pi_handle h, int32_t n_pages, int32_t page_tokens, int32_t n_kv_heads,
                      int32_t head_dim, pi_tq_pool* out) {
    PI_CHECK_HANDLE(h);
    if (!out) return fail(h, PI_ERR_INVALID_ARG, "pi_tq_pool_create: out is null");
    *out = nullptr;
    if (page_tokens != pi::kPageTokens)
        return fail(h, PI_ERR_UNSUPPORTED, "pi_tq_pool_create: page_tokens must be 16 (got %d)", page_tokens);
    if (n_pages <= 0 || n_kv_heads <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_tq_pool_create: n_pages=%d n_kv_heads=%d", n_pages, n_kv_heads);
    if (head_dim < 1 || head_dim > pi::kTqMaxDim)
        return fail(h, PI_ERR_UNSUPPORTED, "pi_tq_pool_create: head_dim %d (1..%d)", head_dim, pi::kTqMaxDim);
    const int D = head_dim;
    const size_t nblk = (size_t)n_pages * n_kv_heads;
    const size_t kbytes = nblk * pi::kPageTokens * (pi::tq_key_bytes(D) + 4);
    const size_t vbytes = nblk * pi::kPageTokens * D * 2;
    const size_t mbytes = (size_t)n_kv_heads * D * D * sizeof(float);
    // per-head matrices, transposed for the kernels (TurboQuant::new(3, D, D,
    // 0xCAFE_BABE + h), src/turboquant/mod.rs:430-437)
    std::vector<float> rot((size_t)D * D), qjl((size_t)D * D);
    // and G.R (double sums, rounded once), which turns a query into its virtual
    // query in one product
    std::vector<float> rt((size_t)n_kv_heads * D * D), gt((size_t)n_kv_heads * D * D),
        grt((size_t)n_kv_heads * D * D);
    std::vector<double> gr_row(D);
    for (int kh = 0; kh < n_kv_heads; ++kh) {
        tq_matrices(D, 0xCAFEBABEULL + (uint64_t)kh, rot.data(), qjl.data());
        for (int i = 0; i < D; ++i)
            for (int j = 0; j < D; ++j) {
                rt[((size_t)kh * D + j) * D + i] = rot[(size_t)i * D + j];
                gt[((size_t)kh * D + j) * D + i] = qjl[(size_t)i * D + j];
            }
        for (int i = 0; i < D; ++i) {
            std::fill(gr_row.begin(), gr_row.end(), 0.0);
            for (int k = 0; k < D; ++k) {
                const double gik = qjl[(size_t)i * D + k];
                const float* rk = &rot[(size_t)k * D];
                for (int j = 0; j < D; ++j) gr_row[j] += gik * rk[j];
            }
            for (int j = 0; j < D; ++j) grt[((size_t)kh * D + j) * D + i] = (float)gr_row[j];
        }
    }
    PI_HIP(h, hipSetDevice(h->device), "pi_tq_pool_create");
    pi_tq_pool p = new (std::nothrow) pi_tq_pool_s();
    if (!p) return fail(h, PI_ERR_OUT_OF_MEMORY, "pi_tq_pool_create: host allocation");
    p->owner = h;
    p->bytes = kbytes + vbytes + 3 * mbytes;
    pi::TqPool& t = p->t;
    // separate K (packed records + norms) and V (f16) arrays
    t.g = pi::KvGeom{nullptr, nullptr, n_pages, n_kv_heads, D, pi::kTqDtype, 0,
                     (size_t)pi::kPageTokens * (pi::tq_key_bytes(D) + 4),
                     (size_t)pi::kPageTokens * D * 2};
    t.rt = t.gt = t.grt = nullptr;
    t.scale = std::sqrt((float)D);
    // residual_norm * qjl_scale of the 3-bit estimator (src/turboquant/mod.rs:297-316)
    t.corr = std::sqrt(0.043f * (1.0f / t.scale)) * std::sqrt(3.14159274f / (2.0f * (float)D));
    hipError_t e = hipMalloc(&t.g.k, kbytes);
    if (e == hipSuccess) e = hipMalloc(&t.g.v, vbytes);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&t.rt), mbytes);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&t.gt), mbytes);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&t.grt), mbytes);
    if (e == hipSuccess) e = hipMemset(t.g.k, 0, kbytes);
    if (e == hipSuccess) e = hipMemset(t.g.v, 0, vbytes);
    if (e == hipSuccess) e = hipMemcpy(t.rt, rt.data(), mbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(t.gt, gt.data(), mbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(t.grt, grt.data(), mbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(t.g.k);
        (void)hipFree(t.g.v);
        (void)hipFree(t.rt);
        (void)hipFree(t.gt);
        (void)hipFree(t.grt);
        delete p;
        return hip_fail(h, e, "pi_tq_pool_create");
    }
    *out = p;
    return PI_OK;
}

void pi_tq_pool_destroy(pi_tq_pool pool) {
    if (!pool) return;
    (void)hipSetDevice(pool->owner->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(pool->t.g.k);
    (void)hipFree(pool->t.g.v);
    (void)hipFree(pool->t.rt);
    (void)hipFree(pool->t.gt);
    (void)hipFree(pool->t.grt);
    delete pool;
}

size_t pi_tq_pool_bytes(pi_tq_pool pool) { return pool ? pool->bytes : 0; }

int pi_tq_append(pi_handle h, pi_tq_pool pool, const float* d_k, const float* d_v,
                 const int32_t* d_page_table, int32_t max_pages, const int32_t* d_start_pos,
                 int32_t n_seq, int32_t n_tok, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!pool || !d_k || !d_v || !d_page_table || !d_start_pos)
        return fail(h, PI_ERR_INVALID_ARG, "pi_tq_append: null argument");
    if (n_seq < 0 || n_tok < 0 || max_pages <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_tq_append: n_seq=%d n_tok=%d max_pages=%d", n_seq, n_tok, max_pages);
    if (n_seq == 0 || n_tok == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_tq_append");
    PI_HIP(h, pi::launch_tq_append(pool->t, d_k, d_v, d_page_table, max_pages, d_start_pos, n_seq,
                                   n_tok, pick(h, stream)),
           "pi_tq_append");
    return PI_OK;
}

int pi_tq_read(pi_handle h, pi_tq_pool pool, const int32_t* d_page_table, int32_t max_pages,
               int32_t seq, int32_t start, int32_t n_tok, uint8_t* d_keys_out, float* d_norms_out,
               uint16_t* d_values_out, void* stream) {
    PI_CHECK_HANDLE(h);
    if (!pool || !d_page_table || !d_keys_out || !d_norms_out || !d_values_out)
        return fail(h, PI_ERR_INVALID_ARG, "pi_tq_read: null argument");
    if (seq < 0 || start < 0 || n_tok < 0 || max_pages <= 0)
        return fail(h, PI_ERR_INVALID_ARG, "pi_tq_read: seq=%d start=%d n_tok=%d", seq, start, n_tok);
    if (n_tok == 0) return PI_OK;
    PI_HIP(h, hipSetDevice(h->device), "pi_tq_read");
    PI_HIP(h, pi::launch_tq_read(pool->t, d_page_table, max_pages, seq, start, n_tok, d_keys_out,
                                 d_norms_out, d_values_out, pick(h, stream)),
           "pi_tq_read");
    return PI_OK;
}

int pi_tq_attn_decode(pi_handle h, const float* d_q, pi_tq_pool pool, const int32_t* d_page_table,
                      int32_t max_pages, const int32_t* d_ctx_len, int32_t batch,
                      int32_t n_q_heads, int32_t gqa_mode, const float* d_gate, float* d_out,
                      void* stream) {
    PI_CHECK_HANDLE(h);
    if (!pool) return fail(h, PI_ERR_INVALID_ARG, "pi_tq_attn_decode: null argument");
    const pi::KvGeom& g = pool->t.g;
    int rc = decode_check(h, "pi_tq_attn_decode", g, d_q, d_page_table, d_ctx_len, d_out, max_pages,
                          batch, n_q_heads, gqa_mode);
    if (!rc) rc = gate_check(h, "pi_tq_attn_decode", d_gate);
    if (rc) return rc;
    if (batch == 0) return PI_OK;
    hipStream_t s = pick(h, stream);
    PI_HIP(h, hipSetDevice(h->device), "pi_tq_attn_decode");
    if ((rc = ws_begin(h, s, "pi_tq_attn_decode"))) return rc;
    const size_t need_qv = (size_t)batch * n_q_heads * 2 * g.head_dim;
    if ((rc = grow(h, &h->tq_qv, &h->tq_qv_floats, need_qv, s, "pi_tq_attn_decode workspace", false))) return rc;
    if (!pi::tq_mfma_dim(g.head_dim)) {
        // the reference's order: every score, the softmax, the value sum without weights < 1e-7
        const size_t need_sc = (size_t)batch * n_q_heads * max_pages * pi::kPageTokens;
        if ((rc = grow(h, &h->tq_sc, &h->tq_sc_floats, need_sc, s, "pi_tq_attn_decode workspace", false)))
            return rc;
        PI_HIP(h, pi::launch_tq_query(pool->t, d_q, h->tq_qv, batch, n_q_heads, gqa_mode, s),
               "pi_tq_attn_decode");
        PI_HIP(h, pi::launch_tq_decode_any(pool->t, h->tq_qv, d_page_table, max_pages, d_ctx_len, batch,
                                           n_q_heads, gqa_mode, d_gate, d_out, h->tq_sc, s),
               "pi_tq_attn_decode");
        return ws_end(h, s, "pi_tq_attn_decode");
    }
    const pi::DecodePlan plan = pi::decode_plan(g, batch, max_pages, n_q_heads, gqa_mode, h->device);
    const size_t need_o = pi::decode_ws_floats_o(g, plan);
    const size_t need_ml = need_o / g.head_dim * 2;
    if ((rc = grow(h, &h->dws.partial_o, &h->dws.capacity_o, need_o, s, "pi_tq_attn_decode workspace", false))) return rc;
    if ((rc = grow(h, &h->dws.partial_ml, &h->dws.capacity_ml, need_ml, s, "pi_tq_attn_decode workspace", false))) return rc;
    if ((rc = grow(h, &h->dws.seg_runs, &h->dws.capacity_runs, pi::decode_ws_ints_runs(g, plan), s,
                   "pi_tq_attn_decode workspace", false))) return rc;
    PI_HIP(h, pi::launch_tq_query(pool->t, d_q, h->tq_qv, batch, n_q_heads, gqa_mode, s),
           "pi_tq_attn_decode");
    // the score scale is 1/sqrt(d) (src/turboquant/mod.rs:490)
    const pi::DecodeParams p = decode_params(h->tq_qv, d_page_table, max_pages, d_ctx_len, batch,
                                             n_q_heads, gqa_mode, 1.0f / std::sqrt((float)g.head_dim),
                                             d_gate, d_out, plan);
    PI_HIP(h, pi::launch_decode(g, p, h->dws, plan, s), "pi_tq_attn_decode");
    return ws_end(h, s, "pi_tq_attn_decode");
}

}  // extern "C"

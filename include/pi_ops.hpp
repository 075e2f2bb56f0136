// pi_ops.hpp -- C++ mirror of PowerInfer_x64's attention / SSM call signatures
// over the C ABI in pi_attn.h (header-only, C++20).
//
// The reference is Rust; this header keeps its function names, argument order
// and meaning so a C++ caller (or a test written like the reference's own
// #[test]s) reads the same:
//   powerinfer::ops  -- src/ops.rs: rms_norm, apply_rope, compute_imrope_freqs,
//                       apply_rope_with_freqs, softmax, attention_head
//   powerinfer::ssm  -- src/ssm/mod.rs: ssm_forward, create_ssm_state, plus the gated-delta
//                       step of src/model/mod.rs:841-916
//   powerinfer::rocm -- the offload seam of src/cuda/mod.rs:373-537:
//                       Device::init() -> std::optional (None = CPU path) and
//                       try_* calls -> std::optional<Result> (Option<Result<(),
//                       String>>); DeviceLayerCache, the device-resident
//                       LayerCache with forward's attention step.
// The ops / ssm free functions run on the calling thread's default device and
// throw BackendError where the reference would panic (a size mismatch, its
// debug_assert_eq!) or where the device fails.
#pragma once

#include "pi_attn.h"

#include <array>
#include <cstddef>
#include <cstdint>
#include <optional>
#include <span>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace powerinfer {

// src/runtime/mod.rs:6-18 (BackendError), keyed by pi_status.
enum class ErrorKind : int {
    InvalidArgument = PI_ERR_INVALID_ARG,
    OutOfMemory = PI_ERR_OUT_OF_MEMORY,
    InvalidKernel = PI_ERR_INVALID_KERNEL,
    Device = PI_ERR_DEVICE,
    Unsupported = PI_ERR_UNSUPPORTED,
};

class BackendError : public std::runtime_error {
public:
    BackendError(int status, std::string msg)
        : std::runtime_error(std::move(msg)), kind_(static_cast<ErrorKind>(status)) {}
    ErrorKind kind() const { return kind_; }

private:
    ErrorKind kind_;
};

// Result<(), String>: ok() or the error text (with its status class).
struct Result {
    int status = PI_OK;
    std::string message;
    bool ok() const { return status == PI_OK; }
};

namespace rocm {

// One pi_handle bound to a GPU (GpuResources / GpuDevice, src/cuda/mod.rs:141-460).
class Device {
public:
    // GpuResources::init: None when no gfx950 device can be opened (the caller
    // then takes the CPU path, src/model/mod.rs:373-375).
    static std::optional<Device> init(int device = 0) {
        pi_handle h = nullptr;
        if (pi_create(device, &h) != PI_OK) return std::nullopt;
        return Device(h);
    }
    // Text of the last pi_create failure on this thread.
    static std::string init_error() { return pi_last_error(nullptr); }

    Device(Device&& o) noexcept : h_(std::exchange(o.h_, nullptr)) {}
    Device& operator=(Device&& o) noexcept {
        if (this != &o) {
            pi_destroy(h_);
            h_ = std::exchange(o.h_, nullptr);
        }
        return *this;
    }
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;
    ~Device() { pi_destroy(h_); }

    pi_handle raw() const { return h_; }
    Result result(int rc) const { return rc == PI_OK ? Result{} : Result{rc, pi_last_error(h_)}; }
    void check(int rc) const {
        if (rc != PI_OK) throw BackendError(rc, pi_last_error(h_));
    }

    // The seams (Option<Result<(), String>>): always Some on a live device.
    std::optional<Result> try_attention_head(std::span<float> out, std::span<const float> q,
                                             std::span<const float> k_cache,
                                             std::span<const float> v_cache, size_t seq_len,
                                             size_t head_dim) const {
        if (out.size() < head_dim || q.size() < head_dim || k_cache.size() < seq_len * head_dim ||
            v_cache.size() < seq_len * head_dim)
            return Result{PI_ERR_INVALID_ARG, "attention_head: slice shorter than seq_len * head_dim"};
        return result(pi_ops_attention_head(h_, out.data(), q.data(), k_cache.data(),
                                            v_cache.data(), seq_len, head_dim));
    }
    std::optional<Result> try_gated_delta_step(std::span<float> out, std::span<float> state,
                                               std::span<const float> q, std::span<const float> k,
                                               std::span<const float> v,
                                               std::span<const float> beta,
                                               std::span<const float> g, size_t n_k_heads,
                                               size_t n_v_heads, size_t k_hd, size_t v_hd) const {
        if (q.size() != n_k_heads * k_hd || k.size() != q.size() || v.size() != n_v_heads * v_hd ||
            out.size() != v.size() || beta.size() != n_v_heads || g.size() != n_v_heads ||
            state.size() != n_v_heads * k_hd * v_hd)
            return Result{PI_ERR_INVALID_ARG, "gated_delta_step: slice sizes do not match the heads"};
        return result(pi_ssm_gated_delta_step(h_, out.data(), state.data(), q.data(), k.data(),
                                              v.data(), beta.data(), g.data(), (int32_t)n_k_heads,
                                              (int32_t)n_v_heads, (int32_t)k_hd, (int32_t)v_hd));
    }

    std::optional<Result> try_ssm_forward(std::span<float> y, std::span<const float> x,
                                          std::span<const float> ssm_conv1d,
                                          std::span<const float> ssm_a,
                                          std::span<const float> ssm_dt_bias,
                                          std::span<const float> ssm_alpha,
                                          std::span<const float> ssm_beta,
                                          std::span<const float> ssm_out, std::span<float> state,
                                          size_t d_inner, size_t d_state, size_t d_conv) const {
        // the reference's debug_assert_eq!s (src/ssm/mod.rs:53-54) and the slices it indexes
        if (x.size() != d_inner || y.size() != d_inner || state.size() != d_state * d_inner ||
            ssm_a.size() != d_state * d_inner || ssm_dt_bias.size() != d_inner ||
            ssm_alpha.size() != d_inner * d_inner)
            return Result{PI_ERR_INVALID_ARG, "ssm_forward: slice sizes do not match d_inner / d_state"};
        return result(pi_ssm_forward(h_, y.data(), x.data(), ssm_conv1d.data(), ssm_conv1d.size(),
                                     ssm_a.data(), ssm_dt_bias.data(), ssm_alpha.data(),
                                     ssm_beta.data(), ssm_beta.size(), ssm_out.data(),
                                     ssm_out.size(), state.data(), d_inner, d_state, d_conv));
    }

private:
    explicit Device(pi_handle h) : h_(h) {}
    pi_handle h_ = nullptr;
};

// LayerCache (src/model/mod.rs:73-106) of one attention layer for one sequence on the device,
// with the attention step of forward (src/model/mod.rs:1035-1196) as the offload seam: the
// caller hands over host slices as forward holds them; try_forward returns Some(Ok) or
// Some(Err(text)), and the caller aborts forward on an error as at src/model/mod.rs:619.
class DeviceLayerCache {
public:
    struct Config {
        size_t max_tokens = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0;
        int kv_dtype = PI_F16;
        std::span<const float> q_norm, k_norm;  // empty: the layer has no Q/K norm
        float eps = 1e-6f;
        size_t rope_dim = 0;  // 0: head_dim
        float rope_base = 1e6f;
        std::optional<std::array<int32_t, 4>> sections;  // IMRoPE sections, else NORM RoPE
        int gqa_mode = PI_GQA_MODULO;
    };
    DeviceLayerCache(const Device& dev, const Config& c) : dev_(&dev), c_(c) {
        if ((!c.q_norm.empty() && c.q_norm.size() != c.head_dim) ||
            (!c.k_norm.empty() && c.k_norm.size() != c.head_dim))
            throw BackendError(PI_ERR_INVALID_ARG, "DeviceLayerCache: norm weights must hold head_dim values");
        const int32_t rd = (int32_t)(c.rope_dim ? c.rope_dim : c.head_dim);
        dev.check(pi_attn_layer_create(dev.raw(), (int32_t)c.max_tokens, (int32_t)c.n_heads,
                                       (int32_t)c.n_kv_heads, (int32_t)c.head_dim, c.kv_dtype,
                                       c.q_norm.empty() ? nullptr : c.q_norm.data(),
                                       c.k_norm.empty() ? nullptr : c.k_norm.data(), c.eps, rd,
                                       c.rope_base, c.sections ? c.sections->data() : nullptr,
                                       c.gqa_mode, &l_));
    }
    DeviceLayerCache(const DeviceLayerCache&) = delete;
    DeviceLayerCache& operator=(const DeviceLayerCache&) = delete;
    ~DeviceLayerCache() { pi_attn_layer_destroy(l_); }

    // The tokens of this forward call: q, k rotated in place; out written.
    std::optional<Result> try_forward(std::span<float> q, std::span<float> k,
                                      std::span<const float> v, std::span<const float> gate,
                                      size_t n_tokens, std::span<float> out) {
        const size_t nq = n_tokens * c_.n_heads * c_.head_dim;
        const size_t nk = n_tokens * c_.n_kv_heads * c_.head_dim;
        if (q.size() != nq || out.size() != nq || k.size() != nk || v.size() != nk ||
            (!gate.empty() && gate.size() != nq))
            return Result{PI_ERR_INVALID_ARG, "layer forward: slice sizes do not match the heads"};
        return dev_->result(pi_attn_layer_forward(dev_->raw(), l_, q.data(), k.data(), v.data(),
                                                  gate.empty() ? nullptr : gate.data(),
                                                  (int32_t)n_tokens, out.data()));
    }
    // LayerCache::reset (src/model/mod.rs:1854-1856)
    void reset() { pi_attn_layer_reset(l_); }
    size_t seq_len() const { return (size_t)pi_attn_layer_seq_len(l_); }

private:
    const Device* dev_;
    Config c_;
    pi_attn_layer l_ = nullptr;
};

// One gated-DeltaNet layer of one sequence on the device: the rolling conv state and the
// recurrent state (src/model/mod.rs:122-127), with the layer's GDN step (src/model/mod.rs:
// 750-932) as the offload seam over host slices: qkv [n][conv_dim], z [n][n_v_heads][v_hd],
// beta_raw, a_raw [n][n_v_heads]; out like z.
class DeviceGdnLayer {
public:
    struct Config {
        size_t n_k_heads = 0, n_v_heads = 0, k_hd = 128, v_hd = 128, d_conv = 4;
        std::span<const float> conv_w;   // [conv_dim][d_conv]
        std::span<const float> ssm_a, dt_bias;  // [n_v_heads]
        std::span<const float> norm_w;   // [v_hd]
        float eps = 1e-6f;
    };
    DeviceGdnLayer(const Device& dev, const Config& c) : dev_(&dev), c_(c) {
        conv_dim_ = 2 * c.n_k_heads * c.k_hd + c.n_v_heads * c.v_hd;
        if (c.conv_w.size() != conv_dim_ * c.d_conv || c.ssm_a.size() != c.n_v_heads ||
            c.dt_bias.size() != c.n_v_heads || c.norm_w.size() != c.v_hd)
            throw BackendError(PI_ERR_INVALID_ARG, "DeviceGdnLayer: weight sizes do not match");
        dev.check(pi_gdn_layer_create(dev.raw(), (int32_t)c.n_k_heads, (int32_t)c.n_v_heads,
                                      (int32_t)c.k_hd, (int32_t)c.v_hd, (int32_t)c.d_conv,
                                      c.conv_w.data(), c.ssm_a.data(), c.dt_bias.data(),
                                      c.norm_w.data(), c.eps, &l_));
    }
    DeviceGdnLayer(const DeviceGdnLayer&) = delete;
    DeviceGdnLayer& operator=(const DeviceGdnLayer&) = delete;
    ~DeviceGdnLayer() { pi_gdn_layer_destroy(l_); }

    std::optional<Result> try_forward(std::span<const float> qkv, std::span<const float> z,
                                      std::span<const float> beta_raw,
                                      std::span<const float> a_raw, size_t n_tokens,
                                      std::span<float> out) {
        const size_t nz = n_tokens * c_.n_v_heads * c_.v_hd, nh = n_tokens * c_.n_v_heads;
        if (qkv.size() != n_tokens * conv_dim_ || z.size() != nz || out.size() != nz ||
            beta_raw.size() != nh || a_raw.size() != nh)
            return Result{PI_ERR_INVALID_ARG, "gdn layer forward: slice sizes do not match the heads"};
        return dev_->result(pi_gdn_layer_forward(dev_->raw(), l_, qkv.data(), z.data(),
                                                 beta_raw.data(), a_raw.data(),
                                                 (int32_t)n_tokens, out.data()));
    }
    // The GDN part of InferenceContext::reset (src/model/mod.rs:1867-1869)
    void reset() { dev_->check(pi_gdn_layer_reset(dev_->raw(), l_)); }
    size_t conv_dim() const { return conv_dim_; }

private:
    const Device* dev_;
    Config c_;
    size_t conv_dim_ = 0;
    pi_gdn_layer l_ = nullptr;
};

// The calling thread's default device (device 0), opened on first use.
inline Device& current() {
    thread_local std::optional<Device> dev = Device::init(0);
    if (!dev) throw BackendError(PI_ERR_DEVICE, Device::init_error());
    return *dev;
}

}  // namespace rocm

namespace detail {
inline void require(bool ok, const char* what) {
    if (!ok) throw BackendError(PI_ERR_INVALID_ARG, what);
}
}  // namespace detail

namespace ops {

// src/ops.rs:13-27
inline void rms_norm(std::span<float> out, std::span<const float> x, std::span<const float> weight,
                     float eps) {
    detail::require(out.size() == x.size() && weight.size() == x.size(), "rms_norm: length mismatch");
    if (x.empty()) return;
    auto& d = rocm::current();
    d.check(pi_ops_rms_norm(d.raw(), out.data(), x.data(), weight.data(), x.size(), eps));
}

// src/ops.rs:35-67 (one q head and one k head, adjacent pairs)
inline void apply_rope(std::span<float> q, std::span<float> k, size_t position, size_t head_dim,
                       size_t rope_dim, float base_freq) {
    detail::require(q.size() >= head_dim && k.size() >= head_dim, "apply_rope: slice shorter than head_dim");
    auto& d = rocm::current();
    d.check(pi_ops_apply_rope(d.raw(), q.data(), k.data(), position, head_dim, rope_dim, base_freq));
}

// src/ops.rs:78-122
inline std::vector<float> compute_imrope_freqs(float base_freq, size_t n_rot,
                                               const std::array<int32_t, 4>& sections) {
    std::vector<float> f(n_rot / 2);
    const int rc = pi_compute_imrope_freqs(base_freq, n_rot, sections.data(), f.data());
    if (rc != PI_OK) throw BackendError(rc, pi_last_error(nullptr));
    return f;
}

// src/ops.rs:130-157 (NeoX pairs (i, i + freqs.len()))
inline void apply_rope_with_freqs(std::span<float> q, std::span<float> k, size_t position,
                                  size_t head_dim, std::span<const float> freqs) {
    detail::require(q.size() >= head_dim && k.size() >= head_dim,
                    "apply_rope_with_freqs: slice shorter than head_dim");
    auto& d = rocm::current();
    d.check(pi_ops_apply_rope_with_freqs(d.raw(), q.data(), k.data(), position, head_dim,
                                         freqs.data(), freqs.size()));
}

// src/ops.rs:160-180
inline void softmax(std::span<float> x) {
    if (x.empty()) return;
    auto& d = rocm::current();
    d.check(pi_ops_softmax(d.raw(), x.data(), x.size()));
}

// src/ops.rs:213-247
inline void attention_head(std::span<float> out, std::span<const float> q,
                           std::span<const float> k_cache, std::span<const float> v_cache,
                           size_t seq_len, size_t head_dim) {
    auto& d = rocm::current();
    const Result r = *d.try_attention_head(out, q, k_cache, v_cache, seq_len, head_dim);
    if (!r.ok()) throw BackendError(r.status, r.message);
}

}  // namespace ops

namespace ssm {

// src/ssm/mod.rs:40-52: ssm_forward, one token of the Mamba-2-style selective
// scan (the reference keeps it beside the gated-DeltaNet path and does not call
// it from forward), computed on the device; returns y [d_inner], updates state.
inline std::vector<float> ssm_forward(std::span<const float> x, std::span<const float> ssm_conv1d,
                                      std::span<const float> ssm_a,
                                      std::span<const float> ssm_dt_bias,
                                      std::span<const float> ssm_alpha,
                                      std::span<const float> ssm_beta,
                                      std::span<const float> ssm_out, std::span<float> state,
                                      size_t d_inner, size_t d_state, size_t d_conv) {
    std::vector<float> y(d_inner);
    auto& d = rocm::current();
    const Result r = *d.try_ssm_forward(y, x, ssm_conv1d, ssm_a, ssm_dt_bias, ssm_alpha, ssm_beta,
                                        ssm_out, state, d_inner, d_state, d_conv);
    if (!r.ok()) throw BackendError(r.status, r.message);
    return y;
}

// src/ssm/mod.rs:164-166: a zeroed [d_state * d_inner] state.  For a Qwen3.5
// gated-DeltaNet layer d_state * d_inner = n_v_heads * k_hd * v_hd, laid out
// [n_v_heads][k_hd][v_hd] (src/model/mod.rs:877-916).
inline std::vector<float> create_ssm_state(size_t d_state, size_t d_inner) {
    return std::vector<float>(d_state * d_inner, 0.0f);
}

// One token of the gated delta rule (src/model/mod.rs:841-916): q/k raw (the
// L2 norm and the 1/sqrt(k_hd) q scale are applied inside), beta and g
// per V head, state updated in place, out = S^T q before RMSNormGated.
inline void gated_delta_step(std::span<float> out, std::span<float> state, std::span<const float> q,
                             std::span<const float> k, std::span<const float> v,
                             std::span<const float> beta, std::span<const float> g,
                             size_t n_k_heads, size_t n_v_heads, size_t k_hd, size_t v_hd) {
    auto& d = rocm::current();
    const Result r =
        *d.try_gated_delta_step(out, state, q, k, v, beta, g, n_k_heads, n_v_heads, k_hd, v_hd);
    if (!r.ok()) throw BackendError(r.status, r.message);
}

}  // namespace ssm
}  // namespace powerinfer

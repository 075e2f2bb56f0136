// test_ops.cpp -- the reference's own unit tests for the attention / SSM ops
// (src/ops.rs:299-395, tests/smoke.rs:44-61, src/ssm/mod.rs:164-166,
// src/bin/layer_trace.rs:180-196), written against the C++ mirror
// (include/pi_ops.hpp) so every op runs on the GPU through libpi_attn.so.
// Each test keeps the reference's assertions; tests that only had qualitative
// assertions also check the exact values the mathematics fixes.
//
// Exit status: 0 all passed, 1 a test failed, 2 no usable device (the message
// names the backend error, BackendError::CudaError in the reference).
#include "pi_ops.hpp"

#include <cmath>
#include <cstdio>
#include <functional>
#include <string>
#include <vector>

namespace ops = powerinfer::ops;
namespace ssm = powerinfer::ssm;

static int g_failed = 0;
#define CHECK(cond)                                                        \
    do {                                                                   \
        if (!(cond)) {                                                     \
            std::printf("    check failed: %s (line %d)\n", #cond, __LINE__); \
            throw std::runtime_error("check");                            \
        }                                                                  \
    } while (0)

static void run(const char* name, const std::function<void()>& fn) {
    try {
        fn();
        std::printf("PASS %s\n", name);
    } catch (const powerinfer::BackendError& e) {
        std::printf("FAIL %s: backend error %d: %s\n", name, (int)e.kind(), e.what());
        ++g_failed;
    } catch (const std::exception& e) {
        std::printf("FAIL %s\n", name);
        ++g_failed;
    }
    std::fflush(stdout);
}

// src/ops.rs:303-315
static void test_rms_norm() {
    float x[4] = {1.0f, 2.0f, 3.0f, 4.0f};
    float weight[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    float out[4] = {0, 0, 0, 0};
    ops::rms_norm(out, x, weight, 1e-6f);
    const float val = (1.0f + 4.0f + 9.0f + 16.0f) / 4.0f + 1e-6f;
    const float rms = std::sqrt(val);
    CHECK(std::fabs(out[0] - 1.0f / rms) < 1e-5f);
    CHECK(std::fabs(out[3] - 4.0f / rms) < 1e-5f);
}

// src/ops.rs:317-327
static void test_softmax() {
    float x[3] = {1.0f, 2.0f, 3.0f};
    ops::softmax(x);
    const float sum = x[0] + x[1] + x[2];
    CHECK(std::fabs(sum - 1.0f) < 1e-6f);
    CHECK(x[0] < x[1]);
    CHECK(x[1] < x[2]);
    // closed form: e^(i-3) / (e^-2 + e^-1 + 1)
    const double z = std::exp(-2.0) + std::exp(-1.0) + 1.0;
    for (int i = 0; i < 3; ++i) CHECK(std::fabs(x[i] - std::exp(i - 2.0) / z) < 1e-6);
    // empty slice: no-op (src/ops.rs:161-163)
    ops::softmax(std::span<float>());
}

// src/ops.rs:339-371: q = e0, keys e0, e1, e2, values 10 e0, 20 e1, 30 e2.
static void test_attention_head() {
    const size_t head_dim = 4, seq_len = 3;
    const float q[4] = {1.0f, 0.0f, 0.0f, 0.0f};
    const float k_cache[12] = {1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 1, 0};
    const float v_cache[12] = {10, 0, 0, 0, 0, 20, 0, 0, 0, 0, 30, 0};
    std::vector<float> out(head_dim, 0.0f);
    ops::attention_head(out, q, k_cache, v_cache, seq_len, head_dim);
    CHECK(out[0] > 0.0f);
    CHECK(out[1] >= 0.0f);
    CHECK(out[0] + out[1] + out[2] + out[3] > 0.0f);
    // scores (0.5, 0, 0) -> weights e^0.5 / (e^0.5 + 2), 1 / (e^0.5 + 2) x2
    const double e = std::exp(0.5), z = e + 2.0;
    CHECK(std::fabs(out[0] - 10.0 * e / z) < 1e-5);
    CHECK(std::fabs(out[1] - 20.0 / z) < 1e-5);
    CHECK(std::fabs(out[2] - 30.0 / z) < 1e-5);
    CHECK(out[3] == 0.0f);
}

// src/ops.rs:373-383 and tests/smoke.rs:45-52: RoPE at position 0 is the identity.
static void test_rope() {
    const size_t head_dim = 4, rope_dim = 4;
    float q[4] = {1.0f, 2.0f, 3.0f, 4.0f};
    float k[4] = {5.0f, 6.0f, 7.0f, 8.0f};
    ops::apply_rope(q, k, 0, head_dim, rope_dim, 10000.0f);
    CHECK(std::fabs(q[0] - 1.0f) < 1e-6f);
    CHECK(std::fabs(q[1] - 2.0f) < 1e-6f);
    for (float v : q) CHECK(std::isfinite(v));
    for (float v : k) CHECK(std::isfinite(v));
    // position 1, rope_dim 4: pair 0 turns by 1 rad, pair 1 by 1e-2 rad
    float q1[4] = {1.0f, 0.0f, 1.0f, 0.0f};
    float k1[4] = {0.0f, 1.0f, 0.0f, 1.0f};
    ops::apply_rope(q1, k1, 1, head_dim, rope_dim, 10000.0f);
    CHECK(std::fabs(q1[0] - std::cos(1.0)) < 1e-6 && std::fabs(q1[1] - std::sin(1.0)) < 1e-6);
    CHECK(std::fabs(q1[2] - std::cos(0.01)) < 1e-6 && std::fabs(q1[3] - std::sin(0.01)) < 1e-6);
    CHECK(std::fabs(k1[0] + std::sin(1.0)) < 1e-6 && std::fabs(k1[1] - std::cos(1.0)) < 1e-6);
}

// tests/smoke.rs:54-60, plus its exact value: weights e^0.5 / (e^0.5 + 1), 1 / (e^0.5 + 1).
static void test_smoke_attention() {
    const float q[4] = {1, 0, 0, 0};
    const float k_cache[8] = {1, 0, 0, 0, 0, 1, 0, 0};
    const float v_cache[8] = {10, 0, 0, 0, 0, 20, 0, 0};
    std::vector<float> out(4, 0.0f);
    ops::attention_head(out, q, k_cache, v_cache, 2, 4);
    for (float v : out) CHECK(std::isfinite(v));
    const double e = std::exp(0.5);
    CHECK(std::fabs(out[0] - 10.0 * e / (e + 1.0)) < 1e-5);
    CHECK(std::fabs(out[1] - 20.0 / (e + 1.0)) < 1e-5);
}

// src/ops.rs:78-122: freq[k] = theta_scale^k, theta_scale = base^(-2/n_rot).
static void test_imrope_freqs() {
    const auto f = ops::compute_imrope_freqs(1e7f, 64, {11, 11, 10, 0});
    CHECK(f.size() == 32);
    const double ts = std::pow(1e7, -2.0 / 64.0);
    for (size_t i = 0; i < f.size(); ++i) CHECK(std::fabs(f[i] - std::pow(ts, (double)i)) <= 1e-6 * std::pow(ts, (double)i) + 1e-12);
    // position 0 is the identity; NeoX pairs (i, i + 32) turn at position 1
    std::vector<float> q(256), k(256);
    for (int i = 0; i < 256; ++i) q[i] = k[i] = 0.01f * (float)i;
    auto q0 = q, k0 = k;
    ops::apply_rope_with_freqs(q, k, 0, 256, f);
    CHECK(q == q0 && k == k0);
    std::vector<float> e(256, 0.0f), z(256, 0.0f);
    e[0] = 1.0f;  // pair (0, 32), frequency 1: turns by 1 rad
    ops::apply_rope_with_freqs(e, z, 1, 256, f);
    CHECK(std::fabs(e[0] - std::cos(1.0)) < 1e-6 && std::fabs(e[32] - std::sin(1.0)) < 1e-6);
    for (int i = 64; i < 256; ++i) CHECK(e[i] == 0.0f);  // dims >= n_rot untouched
}

// src/ssm/mod.rs:164-166 and the zero-state closed form of
// src/bin/layer_trace.rs:180-196: out[v] = beta * (q.k) * v[v] (q, k L2-normed, q / sqrt(k_hd)).
static void test_gated_delta_zero_state() {
    const size_t hk = 2, hv = 4, dk = 128, dv = 128;
    auto state = ssm::create_ssm_state(dk * hv, dv);
    CHECK(state.size() == hv * dk * dv);
    for (float s : state) CHECK(s == 0.0f);
    std::vector<float> q(hk * dk), k(hk * dk), v(hv * dv), beta(hv), g(hv), out(hv * dv);
    for (size_t i = 0; i < q.size(); ++i) {
        q[i] = std::sin(0.37f * (float)i + 0.1f);
        k[i] = std::cos(0.23f * (float)i + 0.2f);
    }
    for (size_t i = 0; i < v.size(); ++i) v[i] = std::sin(0.11f * (float)i);
    for (size_t h = 0; h < hv; ++h) {
        beta[h] = 0.2f + 0.15f * (float)h;
        g[h] = -0.3f * (float)h;
    }
    ssm::gated_delta_step(out, state, q, k, v, beta, g, hk, hv, dk, dv);
    for (size_t h = 0; h < hv; ++h) {
        const size_t kh = h % hk;  // V head h reads K head h % n_k_heads (src/model/mod.rs:845-853)
        double nq = 0, nk = 0, qk = 0;
        for (size_t i = 0; i < dk; ++i) {
            nq += (double)q[kh * dk + i] * q[kh * dk + i];
            nk += (double)k[kh * dk + i] * k[kh * dk + i];
            qk += (double)q[kh * dk + i] * k[kh * dk + i];
        }
        const double c = beta[h] * qk / (std::sqrt(nq) * std::sqrt(nk) * std::sqrt((double)dk));
        for (size_t j = 0; j < dv; ++j) CHECK(std::fabs(out[h * dv + j] - c * v[h * dv + j]) < 2e-5);
        // S = beta k_hat v^T after one step from zero
        const double kn = std::sqrt(nk);
        for (size_t i = 0; i < dk; i += 17)
            for (size_t j = 0; j < dv; j += 13)
                CHECK(std::fabs(state[(h * dk + i) * dv + j] - beta[h] * (k[kh * dk + i] / kn) * v[h * dv + j]) < 2e-6);
    }
}

// src/ssm/mod.rs:176-231, the reference's ssm_forward tests, on the device.
static void test_ssm_forward() {
    {
        const size_t d_inner = 4, d_state = 2, d_conv = 4;
        const std::vector<float> x = {1, 2, 3, 4}, conv(d_inner * d_conv, 0.1f),
                                 a(d_state * d_inner, -0.5f), dt_bias(d_inner, 0.0f),
                                 alpha(d_inner * d_inner, 0.1f), beta(d_state * d_inner, 0.1f),
                                 out(d_inner * d_inner, 0.1f);
        auto state = ssm::create_ssm_state(d_state, d_inner);
        const auto y = ssm::ssm_forward(x, conv, a, dt_bias, alpha, beta, out, state, d_inner,
                                        d_state, d_conv);
        CHECK(y.size() == d_inner);
        for (float v : y) CHECK(std::isfinite(v));
        bool moved = false;
        for (float s : state) moved |= s != 0.0f;
        CHECK(moved);
    }
    {
        const size_t d_inner = 8, d_state = 4, d_conv = 4;
        const std::vector<float> x(d_inner, 1.0f), conv(d_inner * d_conv, 0.2f),
                                 a(d_state * d_inner, -1.0f), dt_bias(d_inner, 0.5f),
                                 alpha(d_inner * d_inner, 0.1f), beta(d_state * d_inner, 0.1f),
                                 out(d_inner * d_inner, 0.05f), x2(d_inner, 2.0f);
        auto state = ssm::create_ssm_state(d_state, d_inner);
        const auto y1 = ssm::ssm_forward(x, conv, a, dt_bias, alpha, beta, out, state, d_inner,
                                         d_state, d_conv);
        const auto y2 = ssm::ssm_forward(x2, conv, a, dt_bias, alpha, beta, out, state, d_inner,
                                         d_state, d_conv);
        CHECK(y1 != y2);
    }
}

// Size mismatches raise InvalidArgument, as the reference's debug_assert_eq! would panic.
static void test_size_checks() {
    float x[4] = {1, 2, 3, 4}, w[3] = {1, 1, 1}, out[4];
    bool threw = false;
    try {
        ops::rms_norm(out, x, w, 1e-6f);
    } catch (const powerinfer::BackendError& e) {
        threw = e.kind() == powerinfer::ErrorKind::InvalidArgument;
    }
    CHECK(threw);
    auto& dev = powerinfer::rocm::current();
    const auto r = dev.try_attention_head(out, x, x, x, 2, 4);  // caches shorter than 2 x 4
    CHECK(r && !r->ok() && r->status == PI_ERR_INVALID_ARG);
}

int main() {
    if (!powerinfer::rocm::Device::init(0)) {
        std::printf("NO_DEVICE %s\n", powerinfer::rocm::Device::init_error().c_str());
        return 2;
    }
    run("ops::rms_norm", test_rms_norm);
    run("ops::softmax", test_softmax);
    run("ops::attention_head", test_attention_head);
    run("ops::apply_rope", test_rope);
    run("smoke::attention_head", test_smoke_attention);
    run("ops::compute_imrope_freqs + apply_rope_with_freqs", test_imrope_freqs);
    run("ssm::gated_delta_step zero state", test_gated_delta_zero_state);
    run("ssm::ssm_forward", test_ssm_forward);
    run("size checks", test_size_checks);
    std::printf("%d failed\n", g_failed);
    return g_failed ? 1 : 0;
}

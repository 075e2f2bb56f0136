// test_layer.cpp -- the device-resident LayerCache (powerinfer::rocm::DeviceLayerCache over
// pi_attn_layer_*) driven as InferenceContext::forward drives an attention layer
// (src/model/mod.rs:668-1219): a prompt in one call must give the same outputs as the same
// tokens fed one forward call at a time (the reference's own per-token loop), the try_* seam
// reports errors as Some(Err) without changing the cache, and reset() restarts the sequence
// (src/model/mod.rs:1854-1856).  The same for a gated-DeltaNet layer (DeviceGdnLayer over
// pi_gdn_layer_*, src/model/mod.rs:750-932): a chunked prompt against its own token loop.
//
// Exit status: 0 all passed, 1 a test failed, 2 no usable device.
#include "pi_ops.hpp"

#include <cmath>
#include <cstdio>
#include <random>
#include <vector>

using powerinfer::rocm::Device;
using powerinfer::rocm::DeviceGdnLayer;
using powerinfer::rocm::DeviceLayerCache;

static int g_failed = 0;
#define CHECK(cond)                                                          \
    do {                                                                     \
        if (!(cond)) {                                                       \
            std::printf("    check failed: %s (line %d)\n", #cond, __LINE__); \
            ++g_failed;                                                      \
            return;                                                          \
        }                                                                    \
    } while (0)

static std::vector<float> randn(size_t n, std::mt19937& g) {
    std::normal_distribution<float> d(0.f, 1.f);
    std::vector<float> v(n);
    for (float& x : v) x = d(g);
    return v;
}

// ||a - b||_2 / ||b||_2 over each row of `dim`
static double max_row_rel(const std::vector<float>& a, const std::vector<float>& b, size_t dim) {
    double worst = 0;
    for (size_t r = 0; r * dim < a.size(); ++r) {
        double num = 0, den = 0;
        for (size_t i = 0; i < dim; ++i) {
            const double d = (double)a[r * dim + i] - b[r * dim + i];
            num += d * d;
            den += (double)b[r * dim + i] * b[r * dim + i];
        }
        worst = std::max(worst, std::sqrt(num / std::max(den, 1e-30)));
    }
    return worst;
}

static void test_prompt_equals_token_loop(const Device& dev) {
    const size_t H = 8, HKV = 2, D = 128, N = 96;
    DeviceLayerCache::Config c;
    c.max_tokens = 128;
    c.n_heads = H;
    c.n_kv_heads = HKV;
    c.head_dim = D;
    c.rope_base = 1e6f;
    DeviceLayerCache whole(dev, c), loop(dev, c);
    std::mt19937 g(7);
    auto q = randn(N * H * D, g), k = randn(N * HKV * D, g), v = randn(N * HKV * D, g);
    auto q1 = q, k1 = k;
    std::vector<float> out_whole(N * H * D), out_loop(N * H * D);
    auto r = whole.try_forward(q1, k1, v, {}, N, out_whole);
    CHECK(r && r->ok());
    CHECK(whole.seq_len() == N);
    for (size_t t = 0; t < N; ++t) {
        std::vector<float> qt(q.begin() + t * H * D, q.begin() + (t + 1) * H * D);
        std::vector<float> kt(k.begin() + t * HKV * D, k.begin() + (t + 1) * HKV * D);
        std::vector<float> vt(v.begin() + t * HKV * D, v.begin() + (t + 1) * HKV * D);
        std::vector<float> ot(H * D);
        auto rt = loop.try_forward(qt, kt, vt, {}, 1, ot);
        CHECK(rt && rt->ok());
        std::copy(ot.begin(), ot.end(), out_loop.begin() + t * H * D);
    }
    CHECK(loop.seq_len() == N);
    const double err = max_row_rel(out_whole, out_loop, D);
    std::printf("    prompt vs token loop: max row rel err %.3e\n", err);
    CHECK(err <= 1e-2);
}

static void test_errors_and_reset(const Device& dev) {
    const size_t H = 4, HKV = 4, D = 128;
    DeviceLayerCache::Config c;
    c.max_tokens = 16;
    c.n_heads = H;
    c.n_kv_heads = HKV;
    c.head_dim = D;
    c.kv_dtype = PI_F32;
    c.rope_base = 1e4f;
    DeviceLayerCache layer(dev, c);
    std::mt19937 g(11);
    auto q = randn(12 * H * D, g), k = randn(12 * HKV * D, g), v = randn(12 * HKV * D, g);
    std::vector<float> out(12 * H * D), again(12 * H * D);
    auto qa = q, ka = k;
    CHECK(layer.try_forward(qa, ka, v, {}, 12, out)->ok());
    // 12 + 12 > 16: Some(Err(OutOfMemory)), the sequence unchanged
    auto qb = q, kb = k;
    auto r = layer.try_forward(qb, kb, v, {}, 12, again);
    CHECK(r && !r->ok() && r->status == PI_ERR_OUT_OF_MEMORY && !r->message.empty());
    CHECK(layer.seq_len() == 12);
    // a slice of the wrong size is Some(Err(InvalidArgument))
    std::vector<float> short_out(3);
    auto r2 = layer.try_forward(qb, kb, v, {}, 12, short_out);
    CHECK(r2 && r2->status == PI_ERR_INVALID_ARG);
    layer.reset();
    CHECK(layer.seq_len() == 0);
    auto qc = q, kc = k;
    CHECK(layer.try_forward(qc, kc, v, {}, 12, again)->ok());
    CHECK(again == out);
    CHECK(qc == qa && kc == ka);  // the same rotated q / k
    // norm weights that do not hold head_dim values are refused before anything reads them
    std::vector<float> short_norm(D / 2, 1.0f);
    DeviceLayerCache::Config bad = c;
    bad.k_norm = short_norm;
    bool threw = false;
    try {
        DeviceLayerCache l2(dev, bad);
    } catch (const powerinfer::BackendError& e) {
        threw = e.kind() == powerinfer::ErrorKind::InvalidArgument;
    }
    CHECK(threw);
}

static void test_gdn_prompt_equals_token_loop(const Device& dev) {
    const size_t HK = 2, HV = 4, D = 128, N = 130, DC = 4;
    const size_t C = 2 * HK * D + HV * D;
    std::mt19937 g(13);
    auto w = randn(C * DC, g);
    for (float& x : w) x *= 0.5f;
    std::vector<float> a(HV), dt = randn(HV, g), nw(D);
    for (size_t i = 0; i < HV; ++i) a[i] = -0.5f - 0.4f * (float)i;
    for (size_t i = 0; i < D; ++i) nw[i] = 0.5f + (float)i / D;
    DeviceGdnLayer::Config c;
    c.n_k_heads = HK;
    c.n_v_heads = HV;
    c.d_conv = DC;
    c.conv_w = w;
    c.ssm_a = a;
    c.dt_bias = dt;
    c.norm_w = nw;
    DeviceGdnLayer whole(dev, c), loop(dev, c);
    CHECK(whole.conv_dim() == C);
    auto qkv = randn(N * C, g), z = randn(N * HV * D, g), br = randn(N * HV, g), ar = randn(N * HV, g);
    std::vector<float> out_whole(N * HV * D), out_loop(N * HV * D), again(N * HV * D);
    CHECK(whole.try_forward(qkv, z, br, ar, N, out_whole)->ok());
    for (size_t t = 0; t < N; ++t) {
        std::span<const float> xs(qkv.data() + t * C, C), zs(z.data() + t * HV * D, HV * D);
        std::span<const float> bs(br.data() + t * HV, HV), as(ar.data() + t * HV, HV);
        auto r = loop.try_forward(xs, zs, bs, as, 1, std::span<float>(out_loop.data() + t * HV * D, HV * D));
        CHECK(r && r->ok());
    }
    // per (token, V head) row: RMSNormGated rescales each row by 1 / rms, so compare rows
    const double err = max_row_rel(out_whole, out_loop, D);
    std::printf("    gdn prompt vs token loop: max row rel err %.3e\n", err);
    CHECK(err <= 1e-2);
    auto r = whole.try_forward(qkv, z, br, ar, N, std::span<float>(again.data(), 7));
    CHECK(r && r->status == PI_ERR_INVALID_ARG);
    whole.reset();
    CHECK(whole.try_forward(qkv, z, br, ar, N, again)->ok());
    CHECK(again == out_whole);
}

int main() {
    auto dev = Device::init(0);
    if (!dev) {
        std::printf("no device: %s\n", Device::init_error().c_str());
        return 2;
    }
    struct T {
        const char* name;
        void (*fn)(const Device&);
    } tests[] = {{"prompt_equals_token_loop", test_prompt_equals_token_loop},
                 {"errors_and_reset", test_errors_and_reset},
                 {"gdn_prompt_equals_token_loop", test_gdn_prompt_equals_token_loop}};
    for (const T& t : tests) {
        const int before = g_failed;
        try {
            t.fn(*dev);
        } catch (const powerinfer::BackendError& e) {
            std::printf("    backend error %d: %s\n", (int)e.kind(), e.what());
            ++g_failed;
        }
        std::printf("%s %s\n", g_failed == before ? "PASS" : "FAIL", t.name);
    }
    return g_failed ? 1 : 0;
}

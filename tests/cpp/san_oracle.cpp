// Address / undefined-behaviour sanitizer run of the CPU oracle (oracle/oracle.c): every
// entry point on small shapes with exactly sized heap buffers, including the edge shapes the
// tests use (empty and one-token inputs, lengths that are not multiples of the 4-lane dot
// product, distinct query / key / value widths, every ssm_forward branch), so an index past a
// buffer or an undefined operation is reported.  Built and run by tests/test_sanitizers_cpu.py.
#include "oracle.h"

#include <cstdio>
#include <random>
#include <vector>

namespace {
std::mt19937 rng(7);
std::vector<float> vec(size_t n, float scale = 1.0f) {
    std::normal_distribution<float> d(0.f, scale);
    std::vector<float> v(n);
    for (auto& x : v) x = d(rng);
    return v;
}
float* P(std::vector<float>& v) { return v.empty() ? nullptr : v.data(); }
}  // namespace

int main() {
    for (size_t n : {0u, 1u, 3u, 4u, 5u, 17u, 128u}) {
        auto a = vec(n), b = vec(n), o = vec(n);
        (void)or_dot_product(P(a), P(b), n);
        (void)or_sum_squares(P(a), n);
        or_scale(P(o), P(a), 0.5f, n);
        if (n) {
            auto w = vec(n);
            or_rms_norm(P(o), P(a), P(w), n, 1e-6f);
            or_softmax(P(o), n);
        }
    }
    for (size_t hd : {4u, 64u, 128u, 256u}) {
        auto q = vec(hd), k = vec(hd);
        or_apply_rope(P(q), P(k), 513, hd, hd, 1e4f);
        or_apply_rope(P(q), P(k), 7, hd, hd / 2, 1e6f);
        const int32_t sec[4] = {11, 11, 10, 0};
        std::vector<float> f(hd / 4);
        or_compute_imrope_freqs(1e7f, hd / 2, sec, f.data());
        or_apply_rope_with_freqs(P(q), P(k), 65535, hd, f.data(), f.size());
        for (size_t T : {1u, 2u, 33u}) {
            auto kc = vec(T * hd), vc = vec(T * hd), out = vec(hd);
            or_attention_head(P(out), P(q), P(kc), P(vc), T, hd);
        }
    }
    // layer tokens with distinct widths (dq >= dk, dv below and above dk), gate and norms
    const size_t dims[][3] = {{32, 32, 32}, {48, 32, 20}, {40, 32, 44}};
    for (const auto& dd : dims) {
        const size_t dq = dd[0], dk = dd[1], dv = dd[2], n = 5, hq = 4, hkv = 3, prev = 2;
        auto q = vec(n * hq * dq), k = vec(n * hkv * dk), v = vec(n * hkv * dv), g = vec(n * hq * dq);
        auto qn = vec(dk), kn = vec(dk), out = vec(n * hq * dk);
        std::vector<float> kc((prev + n) * hkv * dk), vc((prev + n) * hkv * dv);
        const int32_t sec[4] = {11, 11, 10, 0};
        std::vector<float> f(dk / 4);
        or_compute_imrope_freqs(1e7f, dk / 2, sec, f.data());
        or_attn_layer_tokens(P(out), P(q), P(g), P(k), P(v), n, hq, hkv, dq, dk, dv, P(qn), P(kn),
                             1e-6f, dk, 1e6f, nullptr, 0, kc.data(), vc.data(), prev);
        or_attn_layer_tokens(P(out), P(q), nullptr, P(k), P(v), n, hq, hkv, dq, dk, dv, nullptr,
                             nullptr, 1e-6f, dk / 2, 1e7f, f.data(), f.size(), kc.data(), vc.data(),
                             prev);
        or_attn_prepare(P(q), nullptr, n, hq, hkv, dq, dk, P(qn), nullptr, 1e-6f, dk, 1e4f, nullptr,
                        0, 3);
        auto od = vec(hq * dk);
        or_attn_decode(P(od), P(q), dq, kc.data(), vc.data(), prev + n, hq, hkv, dk, dv);
        or_apply_gate(P(od), P(g), hq * dk);
    }
    // gated DeltaNet
    for (const auto& dd : {std::pair<size_t, size_t>{128, 128}, {64, 96}, {17, 5}}) {
        const size_t hk = 3, hv = 5, dk = dd.first, dv = dd.second, T = 4;
        auto q = vec(T * hk * dk), k = vec(T * hk * dk), v = vec(T * hv * dv);
        auto br = vec(T * hv), ar = vec(T * hv), sa = vec(hv), db = vec(hv), beta = vec(T * hv),
             g = vec(T * hv);
        for (size_t t = 0; t < T; ++t)  // one token's [n_v_heads] gates per call
            or_gdn_gates(P(beta) + t * hv, P(g) + t * hv, P(br) + t * hv, P(ar) + t * hv, P(sa),
                         P(db), hv);
        std::vector<float> st(hv * dk * dv), out(T * hv * dv);
        or_gdn_tokens(out.data(), st.data(), P(q), P(k), P(v), P(beta), P(g), T, hk, hv, dk, dv);
        or_gdn_step(out.data(), st.data(), P(q), P(k), P(v), P(beta), P(g), hk, hv, dk, dv);
        auto z = vec(T * hv * dv), w = vec(dv);
        or_rmsnorm_gated(out.data(), P(z), P(w), T * hv, dv, 1e-6f);
        const size_t cd = 2 * hk * dk + hv * dv, dc = 4;
        auto x = vec(cd), cw = vec(cd * dc);
        std::vector<float> hist((dc - 1) * cd);
        or_conv1d_silu(P(x), hist.data(), P(cw), cd, dc);
    }
    // ssm_forward, every slice-length branch
    for (int br = 0; br < 4; ++br) {
        const size_t di = 24, ds = 5, dc = 4;
        auto x = vec(di), conv = vec(br & 1 ? 3 : di * dc), a = vec(ds * di), bias = vec(di);
        auto alpha = vec(di * di, 0.2f), beta = vec(br & 2 ? di : ds * di, 0.2f);
        auto ow = vec(br == 3 ? 5 : di * di, 0.2f), st = vec(ds * di), y = vec(di);
        or_ssm_forward(P(y), P(x), P(conv), conv.size(), P(a), P(bias), P(alpha), P(beta),
                       beta.size(), P(ow), ow.size(), P(st), di, ds, dc);
    }
    // TurboQuant
    for (size_t dim : {16u, 128u, 256u}) {
        std::vector<float> R(dim * dim), G(dim * dim);
        or_tq_orthogonal(R.data(), dim, 0xCAFEBABEull);
        or_tq_gaussian_matrix(G.data(), dim, dim, 0xCAFEBABEull + 1);
        const size_t bytes = or_tq_compressed_bytes(3, dim, dim);
        std::vector<uint8_t> packed(bytes);
        auto x = vec(dim), y = vec(dim), qr = vec(dim), qp = vec(dim);
        or_tq_quantize(packed.data(), P(x), R.data(), G.data(), dim, 3, dim);
        or_tq_dequantize(P(y), packed.data(), R.data(), dim, 3);
        (void)or_tq_dot(P(x), packed.data(), R.data(), G.data(), dim, 3, dim);
        or_tq_precompute_query(P(qr), P(qp), P(x), R.data(), G.data(), dim, dim);
        (void)or_tq_dot_precomputed(P(qr), P(qp), packed.data(), dim, 3, dim);
        const size_t n_kv = 2, T = 3;
        std::vector<float> RR(n_kv * dim * dim), GG(n_kv * dim * dim);
        for (size_t h = 0; h < n_kv; ++h) {
            or_tq_orthogonal(RR.data() + h * dim * dim, dim, 1 + h);
            or_tq_gaussian_matrix(GG.data() + h * dim * dim, dim, dim, 9 + h);
        }
        std::vector<uint8_t> pk(T * n_kv * bytes);
        std::vector<float> norms(T * n_kv);
        std::vector<uint16_t> vals(T * n_kv * dim, 0x3c00);
        for (size_t t = 0; t < T; ++t) {
            auto keys = vec(n_kv * dim);
            or_tq_cache_append_keys(pk.data() + t * n_kv * bytes, norms.data() + t * n_kv, P(keys),
                                    RR.data(), GG.data(), n_kv, dim);
        }
        auto out = vec(dim);
        or_tq_cache_attend(P(out), P(x), pk.data(), norms.data(), vals.data(), RR.data() + dim * dim,
                           GG.data() + dim * dim, T, n_kv, 1, dim);
    }
    std::printf("san_oracle: ok\n");
    return 0;
}

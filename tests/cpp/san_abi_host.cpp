// Address / undefined-behaviour sanitizer run of the C ABI's host-side code
// (powerinfer_x64_amd/csrc/api.cpp built with host sanitizers): the entry points that run
// on the host alone -- the IMRoPE frequency table, the TurboQuant matrix generation, the
// error reporting -- and the argument checks every device entry point makes before it
// touches a GPU (a null handle, null pointers), with exactly sized buffers.  Needs no GPU.
// Built and run by tests/test_sanitizers_cpu.py.
#include "pi_attn.h"

#include <cstdio>
#include <cstring>
#include <vector>

static int g_fail = 0;
#define CHECK(c)                                                       \
    do {                                                               \
        if (!(c)) {                                                    \
            std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c);    \
            ++g_fail;                                                  \
        }                                                              \
    } while (0)

int main() {
    CHECK(pi_abi_version() > 0);
    const int32_t sec[4] = {11, 11, 10, 0};
    for (size_t n_rot : {2u, 64u, 128u, 256u}) {
        std::vector<float> f(n_rot / 2);
        CHECK(pi_compute_imrope_freqs(1e7f, n_rot, sec, f.data()) == PI_OK);
        CHECK(pi_compute_imrope_freqs(1e6f, n_rot, nullptr, f.data()) != PI_OK);  // sections required
    }
    CHECK(pi_compute_imrope_freqs(1e7f, 64, sec, nullptr) != PI_OK);
    for (int32_t dim : {16, 64, 128, 256}) {
        std::vector<float> R((size_t)dim * dim), G((size_t)dim * dim);
        CHECK(pi_tq_generate(dim, 0xCAFEBABEull, R.data(), G.data()) == PI_OK);
    }
    CHECK(pi_tq_generate(0, 1, nullptr, nullptr) != PI_OK);
    CHECK(std::strlen(pi_last_error(nullptr)) > 0);
    // every handle-taking entry point rejects a null handle before anything else
    float x[8] = {0};
    CHECK(pi_sync(nullptr, nullptr) != PI_OK);
    CHECK(pi_ops_rms_norm(nullptr, x, x, x, 8, 1e-6f) != PI_OK);
    CHECK(pi_ops_softmax(nullptr, x, 8) != PI_OK);
    CHECK(pi_ops_attention_head(nullptr, x, x, x, x, 1, 8) != PI_OK);
    CHECK(pi_attn_decode(nullptr, x, nullptr, nullptr, 1, nullptr, 1, 1, 0, 1.f, nullptr, x, nullptr) != PI_OK);
    CHECK(pi_gdn_decode(nullptr, x, x, x, x, x, x, x, 1, 1, 1, 128, 128, nullptr) != PI_OK);
    CHECK(pi_ssm_forward(nullptr, x, x, x, 0, x, x, x, x, 0, x, 0, x, 2, 1, 4) != PI_OK);
    pi_attn_layer destroyed = nullptr;
    pi_attn_layer_destroy(destroyed);
    pi_destroy(nullptr);
    // without a GPU pi_create fails cleanly with a message
    pi_handle h = nullptr;
    if (pi_create(0, &h) != PI_OK) {
        CHECK(h == nullptr);
        CHECK(std::strlen(pi_last_error(nullptr)) > 0);
    } else {
        pi_destroy(h);
    }
    std::printf("san_abi_host: %d failed\n", g_fail);
    return g_fail ? 1 : 0;
}

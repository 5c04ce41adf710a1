// test_hip_attention.cpp — exercises ingot::HipAttention (the C++ host side above the C ABI)
// the way Ingot's forward_batch drives its attention step (src/metal_backend.mm:443-445): per
// layer, kv_store (rope q, rope k, K/V to the f16 cache) and then attention, over a chunked
// prompt followed by decode steps. Every output is compared with the CPU oracle (test
// infrastructure: oracle/attn_oracle.cpp) doing the same steps; the error behaviour of the
// reference (std::runtime_error on a range error, src/metal_backend.mm:421-424) is checked too.
// Prints one line per check and "ALL PASSED" at the end; exits non-zero on a failure.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../oracle/attn_oracle.h"
#include "ingot_hip_attention.hpp"

namespace {

constexpr int kHead = 24, kHeadKv = 8, kHd = 128, kLayers = 2, kCtx = 300, kBatch = 128;
constexpr double kMaxAbs = 2e-3, kRelL2 = 1e-3;  // BASELINE.json north_star parity bar
int g_fail = 0;

void expect(bool ok, const std::string& what) {
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
    if (!ok) g_fail++;
}

void parity(const std::vector<float>& got, const std::vector<float>& want, const std::string& what) {
    double max_abs = 0, num = 0, den = 0;
    bool finite = true;
    for (size_t i = 0; i < got.size(); i++) {
        finite &= std::isfinite(got[i]);
        const double d = double(got[i]) - want[i];
        max_abs = std::max(max_abs, std::fabs(d));
        num += d * d;
        den += double(want[i]) * want[i];
    }
    const double rel = std::sqrt(num / den);
    char buf[160];
    std::snprintf(buf, sizeof buf, "%s: max|d|=%.3e rel-L2=%.3e", what.c_str(), max_abs, rel);
    expect(finite && max_abs <= kMaxAbs && rel <= kRelL2, buf);
}

template <typename T>
T* to_device(const std::vector<T>& h) {
    T* d = nullptr;
    if (hipMalloc(&d, h.size() * sizeof(T)) != hipSuccess) throw std::runtime_error("hipMalloc");
    if (hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
        throw std::runtime_error("hipMemcpy");
    return d;
}

template <typename T>
std::vector<T> to_host(const T* d, size_t n) {
    std::vector<T> h(n);
    if (hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
        throw std::runtime_error("hipMemcpy");
    return h;
}

std::vector<float> randn(std::mt19937_64& rng, size_t n) {
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<float> v(n);
    for (float& x : v) x = nd(rng);
    return v;
}

}  // namespace

int main() {
    std::mt19937_64 rng(20240611);
    ingot::HipAttention::Config cfg;
    cfg.n_layer = kLayers;
    cfg.n_head = kHead;
    cfg.n_head_kv = kHeadKv;
    cfg.head_dim = kHd;
    cfg.n_ctx = kCtx;
    cfg.n_batch = kBatch;
    cfg.rope_inv_freq.resize(kHd / 2);
    oracle_rope_inv_freq(500000.0f, kHd, nullptr, cfg.rope_inv_freq.data());

    const size_t q_dim = size_t(kHead) * kHd, kv_dim = size_t(kHeadKv) * kHd;
    ingot::HipAttention attn(cfg);
    // The oracle's cache for the same layer, f16 bits, zero-initialised like nothing.
    std::vector<uint16_t> kc(size_t(kCtx) * kv_dim, 0), vc(size_t(kCtx) * kv_dim, 0);
    const int layer = 1;

    // A prompt of 160 tokens in chunks of 100 and 60, then 3 decode steps.
    const int chunks[][2] = {{0, 100}, {100, 60}, {160, 1}, {161, 1}, {162, 1}};
    for (const auto& ch : chunks) {
        const int pos = ch[0], n = ch[1];
        std::vector<float> q = randn(rng, n * q_dim), k = randn(rng, n * kv_dim), v = randn(rng, n * kv_dim);
        float* qd = to_device(q);
        float* kd = to_device(k);
        float* vd = to_device(v);
        float* od = to_device(std::vector<float>(n * q_dim, 0.f));
        attn.kv_store(layer, pos, n, qd, kd, vd);
        attn.attention(layer, pos, n, qd, od);
        attn.synchronize();
        // oracle: the same steps on the host
        std::vector<float> qo = q;
        oracle_rope_kv_store(qo.data(), int(q_dim), kHead, k.data(), v.data(), int(kv_dim), kc.data(),
                             vc.data(), size_t(pos) * kv_dim, kHeadKv, kHd, pos, n, cfg.rope_inv_freq.data());
        std::vector<float> want(n * q_dim);
        const float scale = 1.0f / std::sqrt(float(kHd));
        if (n == 1)
            oracle_attn_decode(qo.data(), kc.data(), vc.data(), want.data(), kHead, kHeadKv, kHd, pos + 1, scale, 8);
        else
            oracle_attn_prefill(qo.data(), kc.data(), vc.data(), want.data(), kHead, kHeadKv, kHd, pos, n,
                                int(q_dim), scale, 8);
        parity(to_host(od, n * q_dim), want, "attention pos=" + std::to_string(pos) + " n=" + std::to_string(n));
        for (float* p : {qd, kd, vd, od}) (void)hipFree(p);
    }
    // The V rows written so far are bit-identical to the oracle's f16 rounding; layer 0 is untouched.
    const std::vector<uint16_t> vcache = to_host(attn.v_cache(), size_t(kLayers) * kCtx * kv_dim);
    expect(std::memcmp(vcache.data() + size_t(layer) * kCtx * kv_dim, vc.data(), 163 * kv_dim * 2) == 0,
           "V cache rows 0..162 of layer 1 equal the oracle's f16 bits");
    bool layer0_untouched = true;
    for (size_t i = 0; i < size_t(kCtx) * kv_dim && layer0_untouched; i++) layer0_untouched = vcache[i] == 0;
    expect(layer0_untouched, "layer 0 untouched");

    // Error behaviour of the reference: std::runtime_error, nothing launched.
    auto throws = [&](auto&& f, const char* msg) {
        try {
            f();
        } catch (const std::runtime_error& e) {
            expect(std::strstr(e.what(), msg) != nullptr, std::string("throws \"") + e.what() + "\"");
            return;
        }
        expect(false, std::string("expected an exception containing \"") + msg + "\"");
    };
    throws([&] { attn.attention(layer, kCtx - 10, 20, nullptr, nullptr); }, "context window exceeded");
    throws([&] { attn.kv_store(layer, 0, kBatch + 1, nullptr, nullptr, nullptr); }, "batch size out of range");
    throws([&] { attn.attention(kLayers, 0, 1, nullptr, nullptr); }, "layer out of range");
    throws([&] { attn.kv_store(layer, 0, 4, nullptr, nullptr, nullptr); }, "kv store failed");

    if (g_fail == 0) std::printf("ALL PASSED\n");
    return g_fail == 0 ? 0 : 1;
}

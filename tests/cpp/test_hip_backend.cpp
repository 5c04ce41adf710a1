// test_hip_backend.cpp — exercises ingot::HipBackend (the C++ Llama forward above the C ABIs)
// as Ingot's engine drives a Backend: token-by-token decode (forward), a prompt chunk
// (forward_batch) followed by decode steps, and the reference's range errors
// (src/metal_backend.mm:421-424). The model is a small synthetic Llama with GGUF-layout weights
// (F16, Q8_0 and Q4_0 encoded here with ggml's published quantizers, tied Q8_0 embeddings); the
// logits are compared with the CPU oracle's forward (oracle/model_oracle.cpp, test
// infrastructure) over the same bytes. Tolerances (relative L2 of the logits): decode 1e-4
// (f32 arithmetic on both sides); a chunk and the steps after it 5e-3 (the batched path rounds
// activations and weights to f16, as the reference's Metal path does; the oracle applies the
// same roundings). Prints one line per check and "ALL PASSED"; exits non-zero on a failure.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../oracle/attn_oracle.h"
#include "ingot_hip_backend.hpp"
#include "synth_model.hpp"

namespace {

int g_fail = 0;

void expect(bool ok, const std::string& what) {
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
    if (!ok) g_fail++;
}

double rel_l2(const float* a, const float* b, int n) {
    double num = 0, den = 0;
    for (int i = 0; i < n; i++) {
        const double d = double(a[i]) - b[i];
        num += d * d;
        den += double(b[i]) * b[i];
    }
    return std::sqrt(num / den);
}

}  // namespace

int main() {
    try {
        synth::Owned own;
        const ingot::HostModel m = synth::make_model(own, 11);
        std::mt19937 rng(11);
        const int kvd = m.n_head_kv * m.head_dim;

        // the oracle's view of the same bytes
        std::vector<OracleLayer> ol;
        for (const ingot::HostLayer& L : m.layers) {
            auto t = [](const ingot::HostTensor& x) { return OracleTensor{int(x.type), x.data}; };
            ol.push_back(OracleLayer{L.attn_norm.data(), L.ffn_norm.data(), t(L.wq), t(L.wk), t(L.wv), t(L.wo),
                                     t(L.w_gate), t(L.w_up), t(L.w_down)});
        }
        OracleModel om{m.n_layer, m.n_embd, m.n_head, m.n_head_kv, m.head_dim, m.n_ff, m.n_vocab, m.rms_eps,
                       m.rope_inv_freq.data(), OracleTensor{8, m.tok_embd.data}, OracleTensor{8, m.output.data},
                       m.output_norm.data(), ol.data()};
        const int n_ctx = 96;
        std::vector<uint16_t> kc(size_t(m.n_layer) * n_ctx * kvd), vc(kc.size());
        std::vector<float> want(size_t(m.n_vocab));
        std::uniform_int_distribution<int> tok(0, m.n_vocab - 1);
        std::vector<int32_t> toks(60);
        for (int32_t& t : toks) t = tok(rng);

        {   // token by token
            ingot::HipBackend b(m, n_ctx, 8);
            expect(std::string(b.name()) == "hip" && b.n_ctx() == n_ctx, "name and n_ctx");
            for (int p = 0; p < 6; p++) {
                const float* got = b.forward(toks[size_t(p)], p);
                oracle_forward(&om, kc.data(), vc.data(), n_ctx, toks[size_t(p)], p, want.data(), 0, 8);
                const double r = rel_l2(got, want.data(), m.n_vocab);
                char buf[96];
                std::snprintf(buf, sizeof buf, "decode pos %d: rel-L2 %.3e", p, r);
                expect(r <= 1e-4, buf);
            }
        }
        {   // a 40-token chunk, then decode steps
            ingot::HipBackend b(m, n_ctx, 48);
            const int n = 40;
            const float* got = b.forward_batch(toks.data(), n, 0);
            for (int p = 0; p < n; p++)
                oracle_forward(&om, kc.data(), vc.data(), n_ctx, toks[size_t(p)], p, want.data(), 1, 8);
            double r = rel_l2(got, want.data(), m.n_vocab);
            char buf[96];
            std::snprintf(buf, sizeof buf, "prefill 40 tokens: rel-L2 %.3e", r);
            expect(r <= 5e-3, buf);
            for (int p = n; p < n + 3; p++) {
                got = b.forward(toks[size_t(p)], p);
                oracle_forward(&om, kc.data(), vc.data(), n_ctx, toks[size_t(p)], p, want.data(), 0, 8);
                r = rel_l2(got, want.data(), m.n_vocab);
                std::snprintf(buf, sizeof buf, "decode after prefill pos %d: rel-L2 %.3e", p, r);
                expect(r <= 5e-3, buf);
            }
            auto throws = [&](auto fn, const char* msg) {
                try {
                    fn();
                } catch (const std::runtime_error& e) {
                    return std::string(e.what()).find(msg) != std::string::npos;
                }
                return false;
            };
            expect(throws([&] { b.forward_batch(toks.data(), 49, 0); }, "batch size out of range"),
                   "batch size error");
            expect(throws([&] { b.forward_batch(toks.data(), 2, n_ctx - 1); }, "context window exceeded"),
                   "context error");
            const int32_t bad[2] = {1, m.n_vocab};
            expect(throws([&] { b.forward_batch(bad, 2, 0); }, "token id out of range"), "token id error");
        }
        {   // wq, wk, wv of one type and the one-launch q/k/v path forced: a chunk, then decode steps
            synth::Owned own2;
            const ingot::HostModel m2 = synth::make_model(own2, 12, true);
            std::vector<OracleLayer> ol2;
            for (const ingot::HostLayer& L : m2.layers) {
                auto t = [](const ingot::HostTensor& x) { return OracleTensor{int(x.type), x.data}; };
                ol2.push_back(OracleLayer{L.attn_norm.data(), L.ffn_norm.data(), t(L.wq), t(L.wk), t(L.wv), t(L.wo),
                                          t(L.w_gate), t(L.w_up), t(L.w_down)});
            }
            OracleModel om2{m2.n_layer, m2.n_embd, m2.n_head, m2.n_head_kv, m2.head_dim, m2.n_ff, m2.n_vocab,
                            m2.rms_eps, m2.rope_inv_freq.data(), OracleTensor{8, m2.tok_embd.data},
                            OracleTensor{8, m2.output.data}, m2.output_norm.data(), ol2.data()};
            std::fill(kc.begin(), kc.end(), 0);
            std::fill(vc.begin(), vc.end(), 0);
            ingot::HipBackend b(m2, n_ctx, 48);
            b.qkv_one_launch_min_tiles = 0;
            b.ffn_one_launch_min_tiles = 0;
            const int n = 40;
            const float* got = b.forward_batch(toks.data(), n, 0);
            for (int p = 0; p < n; p++)
                oracle_forward(&om2, kc.data(), vc.data(), n_ctx, toks[size_t(p)], p, want.data(), 1, 8);
            double r = rel_l2(got, want.data(), m2.n_vocab);
            char buf[96];
            std::snprintf(buf, sizeof buf, "one-launch q/k/v and gate/up prefill 40 tokens: rel-L2 %.3e", r);
            expect(r <= 5e-3, buf);
            for (int p = n; p < n + 3; p++) {
                got = b.forward(toks[size_t(p)], p);
                oracle_forward(&om2, kc.data(), vc.data(), n_ctx, toks[size_t(p)], p, want.data(), 0, 8);
                r = rel_l2(got, want.data(), m2.n_vocab);
                std::snprintf(buf, sizeof buf, "one-launch q/k/v, decode pos %d: rel-L2 %.3e", p, r);
                expect(r <= 5e-3, buf);
            }
        }
    } catch (const std::exception& e) {
        std::printf("FAIL exception: %s\n", e.what());
        return 1;
    }
    if (g_fail) {
        std::printf("%d FAILED\n", g_fail);
        return 1;
    }
    std::printf("ALL PASSED\n");
    return 0;
}

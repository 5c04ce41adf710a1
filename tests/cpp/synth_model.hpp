// synth_model.hpp — small synthetic Llama models in the GGUF tensor layout for the C++ tests
// (test data only): F16 rows, and Q8_0 / Q4_0 blocks encoded with ggml's published quantizers.
#pragma once

#include <cmath>
#include <cstring>
#include <random>
#include <vector>

#include "../../oracle/attn_oracle.h"
#include "ingot_hip_backend.hpp"

namespace synth {

inline uint16_t f16(float x) {
    uint16_t h;
    oracle_f32_to_f16(&x, &h, 1);
    return h;
}

// quantize_row_q8_0 / quantize_row_q4_0 (ggml's reference quantizers), one row.
inline std::vector<uint8_t> encode(uint32_t type, const float* x, int n) {
    std::vector<uint8_t> out;
    if (type == 1) {
        out.resize(size_t(n) * 2);
        for (int i = 0; i < n; i++) {
            const uint16_t h = f16(x[i]);
            std::memcpy(&out[2 * size_t(i)], &h, 2);
        }
        return out;
    }
    for (int b = 0; b < n / 32; b++) {
        const float* v = x + 32 * b;
        if (type == 8) {
            float amax = 0;
            for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(v[i]));
            const float d = amax / 127.f, id = d ? 1.f / d : 0.f;
            const uint16_t dh = f16(d);
            out.push_back(uint8_t(dh & 0xFF));
            out.push_back(uint8_t(dh >> 8));
            for (int i = 0; i < 32; i++) out.push_back(uint8_t(int8_t(roundf(v[i] * id))));
        } else {  // Q4_0
            float amax = 0, mx = 0;
            for (int i = 0; i < 32; i++)
                if (std::fabs(v[i]) > amax) { amax = std::fabs(v[i]); mx = v[i]; }
            const float d = mx / -8.f, id = d ? 1.f / d : 0.f;
            const uint16_t dh = f16(d);
            out.push_back(uint8_t(dh & 0xFF));
            out.push_back(uint8_t(dh >> 8));
            for (int i = 0; i < 16; i++) {
                const int a = std::min(15, int(int8_t(v[i] * id + 8.5f)));
                const int c = std::min(15, int(int8_t(v[i + 16] * id + 8.5f)));
                out.push_back(uint8_t(a | (c << 4)));
            }
        }
    }
    return out;
}

struct Owned {
    std::vector<std::vector<uint8_t>> blobs;
    ingot::HostTensor make(uint32_t type, int n_out, int n_in, float scale, std::mt19937& rng) {
        std::normal_distribution<float> nd(0.f, scale);
        std::vector<uint8_t> bytes;
        std::vector<float> row(static_cast<size_t>(n_in));
        for (int r = 0; r < n_out; r++) {
            for (float& v : row) v = nd(rng);
            const std::vector<uint8_t> e = encode(type, row.data(), n_in);
            bytes.insert(bytes.end(), e.begin(), e.end());
        }
        blobs.push_back(std::move(bytes));
        return ingot::HostTensor{type, uint64_t(n_in), uint64_t(n_out), blobs.back().data()};
    }
};


// A two-layer model (512 wide, 4 Q / 2 KV heads of 128, FFN 1024, 500 tokens) with mixed
// types and tied Q8_0 embeddings.
// uniform_qkv: wq, wk and wv all Q4_0 and w_gate, w_up both Q8_0 (one batched q/k/v launch and
// one batched gate/up + silu launch are possible); otherwise different types.
inline ingot::HostModel make_model(Owned& own, unsigned seed, bool uniform_qkv = false) {
    ingot::HostModel m;
    m.n_layer = 2; m.n_embd = 512; m.n_head = 4; m.n_head_kv = 2; m.head_dim = 128;
    m.n_ff = 1024; m.n_vocab = 500; m.rms_eps = 1e-5f;
    std::mt19937 rng(seed);
    own.blobs.reserve(64);
    std::normal_distribution<float> nd(0.f, 0.1f);
    const int qd = m.n_head * m.head_dim, kvd = m.n_head_kv * m.head_dim;
    m.tok_embd = own.make(8, m.n_vocab, m.n_embd, 1.f, rng);
    m.output = m.tok_embd;  // tied
    m.output_norm.resize(size_t(m.n_embd));
    for (float& v : m.output_norm) v = 1.f + nd(rng);
    m.rope_inv_freq.resize(size_t(m.head_dim / 2));
    oracle_rope_inv_freq(500000.f, m.head_dim, nullptr, m.rope_inv_freq.data());
    for (int l = 0; l < m.n_layer; l++) {
        ingot::HostLayer L;
        L.attn_norm.resize(size_t(m.n_embd));
        L.ffn_norm.resize(size_t(m.n_embd));
        for (float& v : L.attn_norm) v = 1.f + nd(rng);
        for (float& v : L.ffn_norm) v = 1.f + nd(rng);
        const float s = 1.f / std::sqrt(float(m.n_embd));
        L.wq = own.make(2, qd, m.n_embd, s, rng);
        L.wk = own.make(uniform_qkv ? 2 : 1, kvd, m.n_embd, s, rng);
        L.wv = own.make(uniform_qkv ? 2 : 8, kvd, m.n_embd, s, rng);
        L.wo = own.make(2, m.n_embd, qd, 0.5f / std::sqrt(float(qd)), rng);
        L.w_gate = own.make(8, m.n_ff, m.n_embd, s, rng);
        L.w_up = own.make(uniform_qkv ? 8 : 1, m.n_ff, m.n_embd, s, rng);
        L.w_down = own.make(2, m.n_embd, m.n_ff, 0.5f / std::sqrt(float(m.n_ff)), rng);
        m.layers.push_back(L);
    }
    return m;
}

}  // namespace synth

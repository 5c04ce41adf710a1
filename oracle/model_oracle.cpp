// model_oracle.cpp — CPU restatement of Ingot's Llama forward pass, used ONLY as the checker.
//
// TEST INFRASTRUCTURE. Nothing on the product path links, loads or calls this file; only
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it (liboracle.so, ctypes).
//
// What it restates (reference files under /root/reference, read as text, never compiled here):
//   - ops::rmsnorm, src/ops.cpp:226-231: ss = sum x^2 (left to right), scale = 1/sqrtf(ss/n + eps),
//     out = x * scale * w;
//   - ops::silu, src/ops.h:35: x / (1 + expf(-x)); the gate product of src/cpu_backend.cpp:77;
//   - ops::dequant_row (src/ops.cpp:196-198) for the embedding row (src/cpu_backend.cpp:33);
//   - CpuBackend::forward, src/cpu_backend.cpp:22-90, per token: embedding row; per layer
//     rmsnorm, q/k/v matvecs, rope on q and k, K/V into the cache row of pos, attention over rows
//     0..pos, x += wo·attn, rmsnorm, gate/up matvecs, silu(gate)*up, x += down·gate; final rmsnorm
//     and the logits matvec.
// The cache holds K/V rounded to f16 (round to nearest even), as the GPU backends store it
// (src/metal_backend.mm:197-198, shaders/kernels.metal:280-281, 781); the reference CPU cache is
// f32. The linear layers are oracle_linear (ops::matvec numerics) or, with f16_linear set,
// oracle_linear_f16 (the Metal batched path: x and the weights rounded to f16).
#include <cmath>
#include <cstring>
#include <vector>

#include "attn_oracle.h"

extern "C" {

void oracle_rmsnorm(const float* x, const float* w, float* out, int n, int n_rows, float eps) {
    for (int r = 0; r < n_rows; r++) {
        const float* xr = x + size_t(r) * n;
        float* o = out + size_t(r) * n;
        float ss = 0.f;
        for (int i = 0; i < n; i++) ss += xr[i] * xr[i];
        const float scale = 1.0f / sqrtf(ss / float(n) + eps);
        for (int i = 0; i < n; i++) o[i] = xr[i] * scale * w[i];
    }
}

void oracle_silu_mul(float* gate, const float* up, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float g = gate[i];
        gate[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

int oracle_forward(const OracleModel* m, uint16_t* k_cache, uint16_t* v_cache, int n_ctx, int token,
                   int pos, float* logits, int f16_linear, int n_threads) {
    if (!m || !k_cache || !v_cache || !logits || pos < 0 || pos >= n_ctx) return -1;
    if (token < 0 || token >= m->n_vocab) return -1;
    const int hd = m->head_dim, ne = m->n_embd;
    const int q_dim = m->n_head * hd, kv_dim = m->n_head_kv * hd;
    auto lin = [&](const OracleTensor& W, const float* in, float* out, int n_in, int n_out, int acc) {
        return f16_linear ? oracle_linear_f16(W.type, static_cast<const uint8_t*>(W.data), in, out, n_in,
                                              n_out, 1, acc, n_threads)
                          : oracle_linear(W.type, static_cast<const uint8_t*>(W.data), in, out, n_in,
                                          n_out, 1, acc, n_threads);
    };
    std::vector<float> x(ne), h(ne), q(q_dim), k(kv_dim), v(kv_dim), attn(q_dim), gate(m->n_ff),
        up(m->n_ff);
    std::vector<uint16_t> kh(kv_dim), vh(kv_dim);
    // embedding row (src/cpu_backend.cpp:33)
    {
        const OracleTensor& E = m->tok_embd;
        const int be = E.type == 0 || E.type == 1 || E.type == 30 ? 1 : E.type == 14 ? 256 : 32;
        const int bb = E.type == 0 ? 4 : E.type == 1 || E.type == 30 ? 2 : E.type == 8 ? 34
                     : E.type == 2 ? 18 : E.type == 3 ? 20 : 210;
        const size_t row_bytes = size_t(ne / be) * bb;
        if (oracle_dequant_row(E.type, static_cast<const uint8_t*>(E.data) + size_t(token) * row_bytes,
                               x.data(), ne))
            return -1;
    }
    const float scale = 1.0f / sqrtf(float(hd));
    for (int l = 0; l < m->n_layer; l++) {
        const OracleLayer& L = m->layers[l];
        oracle_rmsnorm(x.data(), L.attn_norm, h.data(), ne, 1, m->rms_eps);
        if (lin(L.wq, h.data(), q.data(), ne, q_dim, 0) || lin(L.wk, h.data(), k.data(), ne, kv_dim, 0) ||
            lin(L.wv, h.data(), v.data(), ne, kv_dim, 0))
            return -1;
        oracle_rope(q.data(), 1, q_dim, m->n_head, hd, pos, m->rope_inv_freq);
        oracle_rope(k.data(), 1, kv_dim, m->n_head_kv, hd, pos, m->rope_inv_freq);
        uint16_t* kl = k_cache + size_t(l) * n_ctx * kv_dim;
        uint16_t* vl = v_cache + size_t(l) * n_ctx * kv_dim;
        oracle_f32_to_f16(k.data(), kl + size_t(pos) * kv_dim, kv_dim);
        oracle_f32_to_f16(v.data(), vl + size_t(pos) * kv_dim, kv_dim);
        if (oracle_attn_decode(q.data(), kl, vl, attn.data(), m->n_head, m->n_head_kv, hd, pos + 1, scale,
                               n_threads))
            return -1;
        if (lin(L.wo, attn.data(), x.data(), q_dim, ne, 1)) return -1;
        oracle_rmsnorm(x.data(), L.ffn_norm, h.data(), ne, 1, m->rms_eps);
        if (lin(L.w_gate, h.data(), gate.data(), ne, m->n_ff, 0) ||
            lin(L.w_up, h.data(), up.data(), ne, m->n_ff, 0))
            return -1;
        oracle_silu_mul(gate.data(), up.data(), size_t(m->n_ff));
        if (lin(L.w_down, gate.data(), x.data(), m->n_ff, ne, 1)) return -1;
    }
    oracle_rmsnorm(x.data(), m->output_norm, h.data(), ne, 1, m->rms_eps);
    // logits of one token always take the matvec (f32) path, on the GPU as well
    return oracle_linear(m->output.type, static_cast<const uint8_t*>(m->output.data), h.data(), logits, ne,
                         m->n_vocab, 1, 0, n_threads);
}

}  // extern "C"

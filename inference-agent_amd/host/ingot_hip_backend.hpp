// ingot_hip_backend.hpp — the Llama forward pass of Ingot on MI355X in C++, above the C ABIs
// of include/ingot_attn.h, ingot_linear.h and ingot_model.h (header only; link libingot_attn.so
// and the HIP runtime).
//
// HipBackend has the interface of Ingot's `Backend` (src/backend.h:9-23): forward(token, pos),
// forward_batch(tokens, n, pos) returning the logits of the last token (owned by the backend,
// valid until the next call), n_ctx(), name() == "hip". A maintainer derives it from `Backend`
// and registers it in make_backend (src/engine.cpp:9-13). forward_batch follows
// MetalBackend::forward_batch (src/metal_backend.mm:419-471) step for step:
//   embedding rows; per layer: rmsnorm, q/k/v projections, rope(q) + KV store, attention,
//   x += wo·attn, rmsnorm, gate/up projections, silu(gate)*up, x += down·gate;
//   rmsnorm of the last token and the logits projection.
// For one token (decode) rmsnorm + q/k/v + RoPE + KV store (ingot_proj_rope_kv), rmsnorm +
// gate/up + silu and rmsnorm + logits (ingot_proj) are one launch each (the same results as the
// separate calls, bit for bit).
// The model arrives as HostModel, the reference's Model/Layer/Config (src/model.h:8-28) with each
// gguf::TensorInfo reduced to what the kernels read (type, ne, bytes in the GGUF layout); the
// weights are copied to the device as they are (no dequantization, no repacking).
// Errors throw std::runtime_error with the reference's messages (src/metal_backend.mm:421-424):
// "hip: batch size out of range", "context window exceeded", "token id out of range",
// "hip: <step> failed: <reason>".
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "ingot_attn.h"
#include "ingot_hip_attention.hpp"
#include "ingot_linear.h"
#include "ingot_model.h"

namespace ingot {

struct HostTensor {
    uint32_t type = 0;           // GGUF type id (gguf::TensorType)
    uint64_t ne0 = 0, ne1 = 0;   // gguf::TensorInfo::ne[0], ne[1]
    const void* data = nullptr;  // GGUF-layout bytes (gguf::TensorInfo::data)
};

struct HostLayer {
    std::vector<float> attn_norm, ffn_norm;
    HostTensor wq, wk, wv, wo, w_gate, w_up, w_down;
};

struct HostModel {
    int n_layer = 0, n_embd = 0, n_head = 0, n_head_kv = 0, head_dim = 128, n_ff = 0, n_vocab = 0;
    float rms_eps = 1e-5f;
    HostTensor tok_embd, output;  // output.data == tok_embd.data when the embeddings are tied
    std::vector<float> output_norm, rope_inv_freq;
    std::vector<HostLayer> layers;
};

class HipBackend {
public:
    // Tiles (256 rows x 64 tokens, over q, k and v) from which a chunk's q/k/v run as one batched
    // launch instead of three split-K launches; a test sets 0 to force the one-launch path.
    uint32_t qkv_one_launch_min_tiles = 128;
    // Tiles (128 rows of gate and of up x 64 tokens) from which a chunk's gate/up + silu run as
    // one batched launch; a test sets 0 to force it.
    uint32_t ffn_one_launch_min_tiles = 256;

    // device_weights: the matrices' `data` are device addresses already (gguf::DeviceWeights);
    // otherwise they are host bytes and are copied to the device here.
    HipBackend(const HostModel& m, int n_ctx, int n_batch, hipStream_t stream = nullptr,
               bool device_weights = false)
        : m_(m), n_ctx_(n_ctx), n_batch_(n_batch), stream_(stream), device_weights_(device_weights) {
        if (n_batch < 1) throw std::runtime_error("hip: --batch must be at least 1");
        if (int(m.layers.size()) != m.n_layer) throw std::runtime_error("hip: layer table size mismatch");
        HipAttention::Config ac;
        ac.n_layer = m.n_layer;
        ac.n_head = m.n_head;
        ac.n_head_kv = m.n_head_kv;
        ac.head_dim = m.head_dim;
        ac.n_ctx = n_ctx;
        ac.n_batch = n_batch;
        ac.rope_inv_freq = m.rope_inv_freq;
        attn_ = std::make_unique<HipAttention>(ac, stream);
        q_dim_ = size_t(m.n_head) * m.head_dim;
        kv_dim_ = size_t(m.n_head_kv) * m.head_dim;

        embd_ = upload(m.tok_embd, m.n_embd, m.n_vocab, "token_embd");
        output_ = m.output.data == m.tok_embd.data ? embd_ : upload(m.output, m.n_embd, m.n_vocab, "output");
        output_norm_ = upload_f32(m.output_norm, m.n_embd, "output_norm");
        for (const HostLayer& L : m.layers) {
            DevLayer d;
            d.attn_norm = upload_f32(L.attn_norm, m.n_embd, "attn_norm");
            d.ffn_norm = upload_f32(L.ffn_norm, m.n_embd, "ffn_norm");
            d.wq = upload(L.wq, m.n_embd, q_dim_, "attn_q");
            d.wk = upload(L.wk, m.n_embd, kv_dim_, "attn_k");
            d.wv = upload(L.wv, m.n_embd, kv_dim_, "attn_v");
            d.wo = upload(L.wo, q_dim_, m.n_embd, "attn_output");
            d.w_gate = upload(L.w_gate, m.n_embd, m.n_ff, "ffn_gate");
            d.w_up = upload(L.w_up, m.n_embd, m.n_ff, "ffn_up");
            d.w_down = upload(L.w_down, m.n_ff, m.n_embd, "ffn_down");
            layers_.push_back(d);
        }
        const size_t nb = size_t(n_batch);
        x_ = alloc_f32(nb * m.n_embd);
        h_ = alloc_f32(nb * m.n_embd);
        q_ = alloc_f32(nb * q_dim_);
        k_ = alloc_f32(nb * kv_dim_);
        v_ = alloc_f32(nb * kv_dim_);
        attn_out_ = alloc_f32(nb * q_dim_);
        gate_ = alloc_f32(nb * m.n_ff);
        up_ = alloc_f32(nb * m.n_ff);
        logits_dev_ = alloc_f32(size_t(m.n_vocab));
        tokens_dev_ = static_cast<int32_t*>(alloc_bytes(nb * sizeof(int32_t)));
        logits_.resize(size_t(m.n_vocab));
        // One linear workspace, sized for the largest call of every projection shape over every
        // chunk length (a shorter chunk may split its k ranges over more workgroups).
        for (const Dev& w : {layers_[0].wq, layers_[0].wk, layers_[0].wo, layers_[0].w_gate, layers_[0].w_down})
            for (uint32_t n = 2; n <= uint32_t(n_batch); n++)
                lin_ws_bytes_ = std::max(lin_ws_bytes_, ingot_linear_workspace_size_for(w, n));
        lin_ws_ = alloc_bytes(lin_ws_bytes_);
        check(hipMemset(lin_ws_, 0, lin_ws_bytes_), "linear workspace clear");
    }

    ~HipBackend() {
        for (void* p : owned_) (void)hipFree(p);
    }
    HipBackend(const HipBackend&) = delete;
    HipBackend& operator=(const HipBackend&) = delete;

    const float* forward(int32_t token, int pos) { return forward_batch(&token, 1, pos); }

    const float* forward_batch(const int32_t* tokens, int n, int pos) {
        if (n < 1 || n > n_batch_) throw std::runtime_error("hip: batch size out of range");
        if (pos < 0 || pos + n > n_ctx_) throw std::runtime_error("context window exceeded");
        for (int i = 0; i < n; i++)
            if (tokens[i] < 0 || tokens[i] >= m_.n_vocab) throw std::runtime_error("token id out of range");
        check(hipMemcpyAsync(tokens_dev_, tokens, size_t(n) * sizeof(int32_t), hipMemcpyHostToDevice, stream_),
              "token upload");
        const uint32_t ne = uint32_t(m_.n_embd), nf = uint32_t(m_.n_ff), un = uint32_t(n);
        const uint32_t qd = uint32_t(q_dim_), kvd = uint32_t(kv_dim_);
        abi(ingot_get_rows(embd_.type, embd_.ptr, ne, uint32_t(m_.n_vocab), tokens_dev_, un, x_, stream_),
            "embedding");
        for (int l = 0; l < m_.n_layer; l++) {
            const DevLayer& L = layers_[size_t(l)];
            // One token: rmsnorm + q/k/v + RoPE + KV store in one call (ingot_proj_rope_kv) when
            // the three matrices share a type.
            if (n == 1 && L.wq.type == L.wk.type && L.wq.type == L.wv.type) {
                IngotProjDesc d{};
                d.type = L.wq.type;
                d.n_in = ne;
                d.n_mats = 3;
                d.n_out[0] = qd;
                d.n_out[1] = kvd;
                d.n_out[2] = kvd;
                d.prologue = INGOT_PROJ_RMSNORM;
                d.epilogue = INGOT_PROJ_STORE;
                d.eps = m_.rms_eps;
                const void* w[3] = {L.wq.ptr, L.wk.ptr, L.wv.ptr};
                attn_->proj_kv_store(l, pos, w, x_, L.attn_norm, d, q_, k_, v_);
            } else {
                abi(ingot_rmsnorm(x_, L.attn_norm, h_, ne, un, m_.rms_eps, stream_), "rmsnorm");
                if (n > 1 && L.wq.type == L.wk.type && L.wq.type == L.wv.type && qkv_one_launch(un, qd, kvd)) {
                    const Dev* w[3] = {&L.wq, &L.wk, &L.wv};
                    float* outs[3] = {q_, k_, v_};
                    proj(w, 3, h_, nullptr, outs, INGOT_PROJ_X, INGOT_PROJ_STORE, "q/k/v", un);
                } else {
                    linear(L.wq, h_, q_, ne, qd, un, false);
                    linear(L.wk, h_, k_, ne, kvd, un, false);
                    linear(L.wv, h_, v_, ne, kvd, un, false);
                }
                attn_->kv_store(l, pos, n, q_, k_, v_);
            }
            attn_->attention(l, pos, n, q_, attn_out_);
            linear(L.wo, attn_out_, x_, qd, ne, un, true);
            // One token: rmsnorm + gate/up + silu(gate)*up in one launch.
            if (n == 1 && L.w_gate.type == L.w_up.type) {
                const Dev* w[2] = {&L.w_gate, &L.w_up};
                float* outs[1] = {gate_};
                proj(w, 2, x_, L.ffn_norm, outs, INGOT_PROJ_RMSNORM, INGOT_PROJ_SILU_GATE, "rmsnorm+gate/up");
            } else if (L.w_gate.type == L.w_up.type && ffn_one_launch(un, nf)) {
                // A chunk: rmsnorm, then gate/up + silu(gate)*up in one batched launch.
                abi(ingot_rmsnorm(x_, L.ffn_norm, h_, ne, un, m_.rms_eps, stream_), "rmsnorm");
                const Dev* w[2] = {&L.w_gate, &L.w_up};
                float* outs[1] = {gate_};
                proj(w, 2, h_, nullptr, outs, INGOT_PROJ_X, INGOT_PROJ_SILU_GATE, "gate/up+silu", un);
            } else {
                abi(ingot_rmsnorm(x_, L.ffn_norm, h_, ne, un, m_.rms_eps, stream_), "rmsnorm");
                linear(L.w_gate, h_, gate_, ne, nf, un, false);
                linear(L.w_up, h_, up_, ne, nf, un, false);
                abi(ingot_silu_mul(gate_, up_, uint64_t(n) * nf, stream_), "silu_mul");
            }
            linear(L.w_down, gate_, x_, nf, ne, un, true);
        }
        // Logits only for the last token (src/metal_backend.mm:454-456): rmsnorm + output in one
        // launch.
        {
            const Dev* w[1] = {&output_};
            float* outs[1] = {logits_dev_};
            proj(w, 1, x_ + size_t(n - 1) * ne, output_norm_, outs, INGOT_PROJ_RMSNORM, INGOT_PROJ_STORE,
                 "rmsnorm+logits");
        }
        check(hipMemcpyAsync(logits_.data(), logits_dev_, logits_.size() * sizeof(float), hipMemcpyDeviceToHost,
                             stream_),
              "logits download");
        check(hipStreamSynchronize(stream_), "forward");
        return logits_.data();
    }

    int n_ctx() const { return n_ctx_; }
    const char* name() const { return "hip"; }
    // The f16 KV cache (device), [n_layer][n_ctx][n_head_kv*head_dim].
    const uint16_t* k_cache() const { return attn_->k_cache(); }
    const uint16_t* v_cache() const { return attn_->v_cache(); }

private:
    struct Dev {
        uint32_t type = 0;
        const void* ptr = nullptr;
        uint32_t n_in = 0, n_out = 0;
    };
    struct DevLayer {
        const float *attn_norm = nullptr, *ffn_norm = nullptr;
        Dev wq, wk, wv, wo, w_gate, w_up, w_down;
    };

    static void check(hipError_t e, const char* what) {
        if (e != hipSuccess)
            throw std::runtime_error(std::string("hip: ") + what + " failed: " + hipGetErrorString(e));
    }
    static void abi(int rc, const char* what) {
        if (rc != INGOT_ATTN_OK)
            throw std::runtime_error(std::string("hip: ") + what + " failed: " + ingot_attn_strerror(rc));
    }
    void* alloc_bytes(size_t bytes) {
        void* p = nullptr;
        check(hipMalloc(&p, bytes < 16 ? 16 : bytes), "allocation");
        owned_.push_back(p);
        return p;
    }
    float* alloc_f32(size_t n) { return static_cast<float*>(alloc_bytes(n * sizeof(float))); }
    const float* upload_f32(const std::vector<float>& v, int n, const char* what) {
        if (int(v.size()) != n) throw std::runtime_error(std::string("model: bad size of ") + what);
        float* d = alloc_f32(v.size());
        check(hipMemcpy(d, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice), what);
        return d;
    }
    // A weight matrix of n_out rows of n_in elements, copied in its GGUF layout.
    Dev upload(const HostTensor& t, size_t n_in, size_t n_out, const char* what) {
        if (t.ne0 != n_in || t.ne1 != n_out || !t.data)
            throw std::runtime_error(std::string("model: tensor ") + what + " has the wrong shape");
        IngotLinearDesc d{t.type, uint32_t(n_in), uint32_t(n_out), 1, 0, 0, 0};
        const size_t bytes = ingot_linear_weight_bytes(&d);
        if (bytes == 0)
            throw std::runtime_error(std::string("hip: no kernel for the type of tensor ") + what);
        if (device_weights_) return Dev{t.type, t.data, uint32_t(n_in), uint32_t(n_out)};
        void* p = alloc_bytes(bytes);
        check(hipMemcpy(p, t.data, bytes, hipMemcpyHostToDevice), what);
        return Dev{t.type, p, uint32_t(n_in), uint32_t(n_out)};
    }
    static size_t ingot_linear_workspace_size_for(const Dev& w, uint32_t n_tok) {
        IngotLinearDesc d{w.type, w.n_in, w.n_out, n_tok, 0, 0, 0};
        return ingot_linear_workspace_size(&d);
    }
    // A chunk's q/k/v run as one batched launch (no split-K) rather than three split-K
    // ingot_linear calls when the three matrices' tiles of 256 rows x 64 tokens reach half the
    // CUs together (Llama-3.2-3B at 512 tokens: 160 tiles; at 256 tokens 80).
    bool qkv_one_launch(uint32_t n_tok, uint32_t q_dim, uint32_t kv_dim) const {
        const uint32_t rows = (q_dim + 255) / 256 + 2 * ((kv_dim + 255) / 256);
        return uint64_t(rows) * ((n_tok + 63) / 64) >= qkv_one_launch_min_tiles;
    }
    // A chunk's gate/up + silu run as one batched launch (no split-K) once the paired tiles of
    // 128 + 128 rows x 64 tokens fill the 256 CUs (Llama-3.2-3B: 512 at 512 tokens).
    bool ffn_one_launch(uint32_t n_tok, uint32_t n_ff) const {
        return uint64_t((n_ff + 127) / 128) * ((n_tok + 63) / 64) >= ffn_one_launch_min_tiles;
    }
    // One token (or a chunk of n_tok) through 1..3 matrices sharing x (ingot_proj).
    void proj(const Dev* const* w, uint32_t n_mats, const float* x, const float* norm_w, float* const* outs,
              uint32_t prologue, uint32_t epilogue, const char* what, uint32_t n_tok = 1) {
        IngotProjDesc d{};
        d.n_tok = n_tok;
        d.type = w[0]->type;
        d.n_in = w[0]->n_in;
        d.n_mats = n_mats;
        const void* ptrs[3] = {};
        for (uint32_t m = 0; m < n_mats; m++) {
            d.n_out[m] = w[m]->n_out;
            ptrs[m] = w[m]->ptr;
        }
        d.prologue = prologue;
        d.epilogue = epilogue;
        d.eps = m_.rms_eps;
        abi(ingot_proj(ptrs, x, norm_w, outs, &d, stream_), what);
    }
    void linear(const Dev& w, const float* x, float* out, uint32_t n_in, uint32_t n_out, uint32_t n, bool acc) {
        IngotLinearDesc d{w.type, n_in, n_out, n, 0, acc ? 1u : 0u, 0};
        abi(ingot_linear(w.ptr, x, out, lin_ws_, lin_ws_bytes_, &d, stream_), "linear");
    }

    const HostModel& m_;
    int n_ctx_, n_batch_;
    hipStream_t stream_;
    bool device_weights_;
    std::unique_ptr<HipAttention> attn_;
    size_t q_dim_ = 0, kv_dim_ = 0;
    Dev embd_, output_;
    const float* output_norm_ = nullptr;
    std::vector<DevLayer> layers_;
    float *x_ = nullptr, *h_ = nullptr, *q_ = nullptr, *k_ = nullptr, *v_ = nullptr, *attn_out_ = nullptr;
    float *gate_ = nullptr, *up_ = nullptr, *logits_dev_ = nullptr;
    int32_t* tokens_dev_ = nullptr;
    void* lin_ws_ = nullptr;
    size_t lin_ws_bytes_ = 0;
    std::vector<float> logits_;
    std::vector<void*> owned_;
};

}  // namespace ingot

// ingot_hip_attention.hpp — the C++ host side of Ingot's attention step on MI355X, above the
// C ABI of include/ingot_attn.h (header only; link libingot_attn.so and the HIP runtime).
//
// Ingot's compute boundary is the C++ `Backend` (src/backend.h:9-23). Per layer, its GPU
// backend's forward_batch (src/metal_backend.mm:419-471) encodes, between the projections and
// the output matmul, exactly two attention-path steps:
//   encode_rope(q) + encode_kv_store(slot, pos, n)   (src/metal_backend.mm:443-444, 395-409)
//   encode_attention(layer, pos, n)                   (src/metal_backend.mm:445, 336-383)
// HipAttention owns what those steps own in the reference — the f16 KV cache
// [n_layer][n_ctx][n_head_kv*head_dim] (src/metal_backend.mm:197-198), the partials workspace
// (`part_`, src/metal_backend.mm:201), the rotary frequencies (`inv_freq_`, :202) — and offers
// the two steps as kv_store() and attention(), so a `HipBackend : Backend` only adds the
// matmuls/norms around them. Errors are thrown as std::runtime_error with the reference's
// messages (src/metal_backend.mm:421-424, 462): "context window exceeded", "... batch size out
// of range", "hip: ... failed: <reason>".
//
// Pointers passed to kv_store()/attention() are device pointers; the calls are asynchronous on
// the object's stream (synchronize() waits), like the reference's encoder, which commits and
// waits once per forward (src/metal_backend.mm:458-461).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "ingot_attn.h"
#include "ingot_linear.h"

namespace ingot {

class HipAttention {
public:
    struct Config {
        int n_layer = 0, n_head = 0, n_head_kv = 0, head_dim = 128;
        int n_ctx = 0;    // cache rows per layer
        int n_batch = 1;  // largest chunk kv_store()/attention() accept
        std::vector<float> rope_inv_freq;  // head_dim/2 entries (Model::rope_inv_freq)
    };

    explicit HipAttention(const Config& c, hipStream_t stream = nullptr) : c_(c), stream_(stream) {
        if (c.n_batch < 1) throw std::runtime_error("hip: --batch must be at least 1");
        if (c.n_layer < 1 || c.n_ctx < 1 || c.n_head < 1 || c.n_head_kv < 1)
            throw std::runtime_error("hip: empty model configuration");
        if (c.head_dim <= 0 || c.head_dim > 1024 || c.head_dim % 4 != 0)
            throw std::runtime_error("hip: head_dim must be a multiple of 4 up to 1024");
        if (c.n_head % c.n_head_kv != 0) throw std::runtime_error("hip: n_head must be a multiple of n_head_kv");
        if (int(c.rope_inv_freq.size()) != c.head_dim / 2)
            throw std::runtime_error("hip: rope_inv_freq must have head_dim/2 entries");
        kv_dim_ = size_t(c.n_head_kv) * c.head_dim;
        const size_t cache_bytes = size_t(c.n_layer) * c.n_ctx * kv_dim_ * 2;
        // One workspace serves every call: the largest decode (n_keys = n_ctx) and the bound on
        // every prefill chunk (the most splits of the longest chunk at the end of the context;
        // the split count the library picks is not monotonic in the position).
        ws_bytes_ = ingot_attn_decode_workspace_size_checked(uint32_t(c.n_ctx));
        const int nb = std::min(c.n_batch, c.n_ctx);
        if (nb >= 2)
            ws_bytes_ = std::max(ws_bytes_, prefill_ws(uint32_t(c.n_ctx - nb), uint32_t(nb),
                                                       INGOT_ATTN_MAX_PREFILL_SPLITS));
        alloc(&kcache_, cache_bytes);
        alloc(&vcache_, cache_bytes);
        alloc(&ws_, ws_bytes_);
        alloc(&inv_freq_, c.rope_inv_freq.size() * sizeof(float));
        check(hipMemset(ws_, 0, ws_bytes_), "workspace clear");  // counters start at zero
        check(hipMemcpy(inv_freq_, c.rope_inv_freq.data(), c.rope_inv_freq.size() * sizeof(float),
                        hipMemcpyHostToDevice), "rope frequencies upload");
    }

    ~HipAttention() {
        for (void* p : {kcache_, vcache_, ws_, inv_freq_})
            if (p) (void)hipFree(p);
    }
    HipAttention(const HipAttention&) = delete;
    HipAttention& operator=(const HipAttention&) = delete;

    // encode_rope on q + encode_kv_store: rotates q [n_tok][n_head*head_dim] in place and writes
    // RoPE(k) and v ([n_tok][n_head_kv*head_dim] f32) as f16 into the cache rows pos..pos+n_tok-1
    // of `layer`.
    void kv_store(int layer, int pos, int n_tok, float* q, const float* k, const float* v) {
        check_range(layer, pos, n_tok);
        IngotRopeKvDesc d{uint32_t(c_.n_head), uint32_t(c_.n_head_kv), uint32_t(c_.head_dim),
                          uint32_t(pos), uint32_t(n_tok), slot(layer, pos),
                          uint32_t(c_.n_head * c_.head_dim), uint32_t(kv_dim_)};
        status(ingot_rope_kv_store(q, k, v, static_cast<uint16_t*>(kcache_),
                                   static_cast<uint16_t*>(vcache_), static_cast<float*>(inv_freq_),
                                   &d, stream_),
               "kv store");
    }

    // One decode token's q/k/v step in one call (ingot_proj_rope_kv): the projections of x
    // (after the rmsnorm when p.prologue asks for it) by w = {wq, wk, wv}, RoPE, and K/V into
    // the cache rows of (layer, pos); q receives the rotated queries, k and v are scratch.
    void proj_kv_store(int layer, int pos, const void* const* w, const float* x, const float* norm_w,
                       const IngotProjDesc& p, float* q, float* k, float* v) {
        check_range(layer, pos, 1);
        IngotRopeKvDesc d{uint32_t(c_.n_head), uint32_t(c_.n_head_kv), uint32_t(c_.head_dim),
                          uint32_t(pos), 1u, slot(layer, pos), uint32_t(c_.n_head * c_.head_dim),
                          uint32_t(kv_dim_)};
        status(ingot_proj_rope_kv(w, x, norm_w, q, k, v, static_cast<uint16_t*>(kcache_),
                                  static_cast<uint16_t*>(vcache_), static_cast<float*>(inv_freq_), &p, &d,
                                  stream_),
               "rmsnorm+qkv+kv store");
    }

    // encode_attention: out [n_tok][n_head*head_dim] = causal attention of q (rotated) over the
    // layer's cache rows 0..pos+i for token i (decode when n_tok == 1).
    void attention(int layer, int pos, int n_tok, const float* q, float* out) {
        check_range(layer, pos, n_tok);
        const float scale = 1.0f / std::sqrt(float(c_.head_dim));
        const uint64_t kv_offset = uint64_t(layer) * c_.n_ctx * kv_dim_;
        int rc;
        if (n_tok == 1) {
            IngotAttnDecodeDesc d{uint32_t(c_.n_head), uint32_t(c_.n_head_kv), uint32_t(c_.head_dim),
                                  uint32_t(pos + 1), kv_offset, 0, scale};
            rc = ingot_attn_decode(q, static_cast<uint16_t*>(kcache_), static_cast<uint16_t*>(vcache_),
                                   out, ws_, ws_bytes_, &d, stream_);
        } else {
            IngotAttnPrefillDesc d{uint32_t(c_.n_head), uint32_t(c_.n_head_kv), uint32_t(c_.head_dim),
                                   uint32_t(pos), uint32_t(n_tok), kv_offset,
                                   uint32_t(c_.n_head * c_.head_dim), 0, scale};
            rc = ingot_attn_prefill(q, static_cast<uint16_t*>(kcache_), static_cast<uint16_t*>(vcache_),
                                    out, ws_, ws_bytes_, &d, stream_);
        }
        status(rc, "attention");
    }

    void synchronize() { check(hipStreamSynchronize(stream_), "stream synchronize"); }

    int n_ctx() const { return c_.n_ctx; }
    size_t kv_dim() const { return kv_dim_; }
    const uint16_t* k_cache() const { return static_cast<const uint16_t*>(kcache_); }
    const uint16_t* v_cache() const { return static_cast<const uint16_t*>(vcache_); }

private:
    uint64_t slot(int layer, int pos) const { return (uint64_t(layer) * c_.n_ctx + pos) * kv_dim_; }

    void check_range(int layer, int pos, int n_tok) const {
        if (layer < 0 || layer >= c_.n_layer) throw std::runtime_error("hip: layer out of range");
        if (n_tok < 1 || n_tok > c_.n_batch) throw std::runtime_error("hip: batch size out of range");
        if (pos < 0 || pos + n_tok > c_.n_ctx) throw std::runtime_error("context window exceeded");
    }

    size_t ingot_attn_decode_workspace_size_checked(uint32_t n_keys) const {
        IngotAttnDecodeDesc d{uint32_t(c_.n_head), uint32_t(c_.n_head_kv), uint32_t(c_.head_dim),
                              n_keys, 0, 0, 1.0f};
        const size_t n = ingot_attn_decode_workspace_size(&d);
        if (n == 0) throw std::runtime_error("hip: unsupported attention shape");
        return n;
    }

    size_t prefill_ws(uint32_t pos, uint32_t n_tok, uint32_t n_splits) const {
        IngotAttnPrefillDesc d{uint32_t(c_.n_head), uint32_t(c_.n_head_kv), uint32_t(c_.head_dim),
                               pos, n_tok, 0, uint32_t(c_.n_head * c_.head_dim), n_splits, 1.0f};
        return ingot_attn_prefill_workspace_size(&d);
    }

    static void check(hipError_t e, const char* what) {
        if (e != hipSuccess)
            throw std::runtime_error(std::string("hip: ") + what + " failed: " + hipGetErrorString(e));
    }

    static void status(int rc, const char* what) {
        if (rc != INGOT_ATTN_OK)
            throw std::runtime_error(std::string("hip: ") + what + " failed: " + ingot_attn_strerror(rc));
    }

    static void alloc(void** p, size_t bytes) {
        if (hipMalloc(p, std::max<size_t>(bytes, 16)) != hipSuccess)
            throw std::runtime_error("hip: out of device memory");
    }

    Config c_;
    hipStream_t stream_;
    size_t kv_dim_ = 0, ws_bytes_ = 0;
    void* kcache_ = nullptr;
    void* vcache_ = nullptr;
    void* ws_ = nullptr;
    void* inv_freq_ = nullptr;
};

}  // namespace ingot

// backend_adapter.cpp — the binding a maintainer adds to Ingot to register the MI355X backend:
// `class HipBackendAdapter : public Backend` (src/backend.h:9-23) forwarding to ingot::HipBackend,
// and the "hip" case of make_backend (src/engine.cpp:9-13) that maps Ingot's Model (src/model.h)
// onto ingot::HostModel. Not linked into anything: tests/test_backend_adapter.py compiles it with
// -fsyntax-only against the reference's own headers (-I<reference>/src), so a change to either
// side that breaks the binding fails the CPU suite.
#include <memory>
#include <stdexcept>
#include <string>

#include "backend.h"  // Ingot: class Backend
#include "engine.h"   // Ingot: make_backend(name, gguf::File, Model, n_ctx, n_batch)
#include "model.h"    // Ingot: Model, Layer, Config (gguf::TensorInfo pointers into the mapping)

#include "ingot_hip_backend.hpp"

namespace {

ingot::HostTensor host_tensor(const gguf::TensorInfo* t) {
    if (!t) throw std::runtime_error("hip: missing tensor");
    return ingot::HostTensor{static_cast<uint32_t>(t->type), t->dim(0), t->dim(1), t->data};
}

ingot::HostModel host_model(const Model& m) {
    ingot::HostModel h;
    h.n_layer = m.cfg.n_layer;
    h.n_embd = m.cfg.n_embd;
    h.n_head = m.cfg.n_head;
    h.n_head_kv = m.cfg.n_head_kv;
    h.head_dim = m.cfg.head_dim;
    h.n_ff = m.cfg.n_ff;
    h.n_vocab = m.cfg.n_vocab;
    h.rms_eps = m.cfg.rms_eps;
    h.tok_embd = host_tensor(m.tok_embd);
    h.output = m.output == m.tok_embd ? h.tok_embd : host_tensor(m.output);
    h.output_norm = m.output_norm;
    h.rope_inv_freq = m.rope_inv_freq;
    for (const Layer& L : m.layers) {
        ingot::HostLayer l;
        l.attn_norm = L.attn_norm;
        l.ffn_norm = L.ffn_norm;
        l.wq = host_tensor(L.wq);
        l.wk = host_tensor(L.wk);
        l.wv = host_tensor(L.wv);
        l.wo = host_tensor(L.wo);
        l.w_gate = host_tensor(L.w_gate);
        l.w_up = host_tensor(L.w_up);
        l.w_down = host_tensor(L.w_down);
        h.layers.push_back(std::move(l));
    }
    return h;
}

}  // namespace

class HipBackendAdapter final : public Backend {
public:
    HipBackendAdapter(const Model& model, int n_ctx, int n_batch) : impl_(host_model(model), n_ctx, n_batch) {}
    const float* forward(int32_t token, int pos) override { return impl_.forward(token, pos); }
    const float* forward_batch(const int32_t* tokens, int n, int pos) override {
        return impl_.forward_batch(tokens, n, pos);
    }
    int n_ctx() const override { return impl_.n_ctx(); }
    const char* name() const override { return impl_.name(); }

private:
    ingot::HipBackend impl_;
};

// The case a maintainer adds to make_backend (src/engine.cpp:9-13), before its final throw:
//     if (name == "hip") return make_hip_backend(f, model, n_ctx, n_batch);
std::unique_ptr<Backend> make_hip_backend(const gguf::File& f, const Model& model, int n_ctx, int n_batch) {
    (void)f;  // the weights are read through model's TensorInfo pointers into the mapping
    return std::make_unique<HipBackendAdapter>(model, n_ctx, n_batch);
}

// The drop-in check: the adapter is a Backend and the factory has make_backend's shape.
static_assert(std::is_base_of<Backend, HipBackendAdapter>::value, "HipBackendAdapter is a Backend");
using MakeBackend = std::unique_ptr<Backend> (*)(const std::string&, const gguf::File&, const Model&, int, int);
[[maybe_unused]] static const MakeBackend kIngotFactory = &make_backend;
using MakeHip = std::unique_ptr<Backend> (*)(const gguf::File&, const Model&, int, int);
[[maybe_unused]] static const MakeHip kHipFactory = &make_hip_backend;

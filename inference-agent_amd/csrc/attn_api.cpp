// attn_api.cpp — the extern "C" boundary declared in include/ingot_attn.h.
//
// Validates descriptors the way the reference validates forward_batch's arguments
// (src/metal_backend.mm:421-424, src/cpu_backend.cpp:24-25) but returns error codes instead of
// throwing, resolves the split-KV partition, carves the caller's workspace, and launches the
// kernels on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/ingot_attn.h"
#include "../../include/ingot_linear.h"
#include "../../include/ingot_model.h"
#include "attn_internal.h"

namespace {

using ingot::kCounterBytes;

// The prefill records start right after the counters, where decode calls keep their records:
// every call writes the records it reads (after its own counters say they are there), so the two
// kinds of call can share one workspace, ordered on one stream.
size_t prefill_part_offset(uint32_t) { return kCounterBytes; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_heads(uint32_t n_head, uint32_t n_head_kv, uint32_t head_dim) {
    if (n_head == 0 || n_head_kv == 0 || head_dim == 0) return INGOT_ATTN_EINVAL;
    if (n_head % n_head_kv != 0) return INGOT_ATTN_EINVAL;
    // One epoch word per query head in the workspace.
    if (n_head > kCounterBytes / (ingot::kCounterStride * sizeof(unsigned int))) return INGOT_ATTN_EUNSUPPORTED;
    return INGOT_ATTN_OK;
}

// The head sizes of the MFMA kernels; every other head_dim up to kMaxHeadDim runs the fallback
// kernel of attn_naive.hip (the reference's naive path, src/metal_backend.mm:373-382).
bool mfma_head_dim(uint32_t hd) { return hd == 64 || hd == 128 || hd == 256; }
constexpr uint32_t kMaxHeadDim = 1024;

// Decode: any head_dim up to 1024, any group size.
int check_decode(const IngotAttnDecodeDesc* d) {
    if (!d) return INGOT_ATTN_EINVAL;
    const int rc = check_heads(d->n_head, d->n_head_kv, d->head_dim);
    if (rc) return rc;
    if (d->head_dim > kMaxHeadDim) return INGOT_ATTN_EUNSUPPORTED;
    if (d->n_keys == 0 || d->kv_offset % 8 != 0) return INGOT_ATTN_EINVAL;
    if (!(d->scale > 0.f)) return INGOT_ATTN_EINVAL;
    return INGOT_ATTN_OK;
}

// Prefill: any head_dim up to 1024, any group size.
int check_prefill(const IngotAttnPrefillDesc* d) {
    if (!d) return INGOT_ATTN_EINVAL;
    const int rc = check_heads(d->n_head, d->n_head_kv, d->head_dim);
    if (rc) return rc;
    if (d->head_dim > kMaxHeadDim) return INGOT_ATTN_EUNSUPPORTED;
    if (d->n_tok == 0 || d->kv_offset % 8 != 0) return INGOT_ATTN_EINVAL;
    if (uint64_t(d->pos) + d->n_tok > 0xffffffffull) return INGOT_ATTN_EINVAL;
    if (d->q_stride < d->n_head * d->head_dim) return INGOT_ATTN_EINVAL;
    if (mfma_head_dim(d->head_dim) && d->q_stride % 4 != 0) return INGOT_ATTN_EINVAL;  // 16-byte q rows
    if (!(d->scale > 0.f)) return INGOT_ATTN_EINVAL;
    return INGOT_ATTN_OK;
}

// Elements per block and bytes per block of the GGUF types with a linear kernel
// (src/gguf.cpp's type traits); 0 for the others.
void linear_block(uint32_t type, uint32_t& elems, uint32_t& bytes) {
    switch (type) {
        case 0:  elems = 1;   bytes = 4;   return;  // F32
        case 1:  elems = 1;   bytes = 2;   return;  // F16
        case 30: elems = 1;   bytes = 2;   return;  // BF16
        case 8:  elems = 32;  bytes = 34;  return;  // Q8_0
        case 2:  elems = 32;  bytes = 18;  return;  // Q4_0
        case 3:  elems = 32;  bytes = 20;  return;  // Q4_1
        case 14: elems = 256; bytes = 210; return;  // Q6_K
        default: elems = 0;   bytes = 0;   return;
    }
}

int check_linear(const IngotLinearDesc* d) {
    if (!d || d->n_in == 0 || d->n_out == 0 || d->n_tok == 0) return INGOT_ATTN_EINVAL;
    uint32_t elems, bytes;
    linear_block(d->type, elems, bytes);
    if (elems == 0) return INGOT_ATTN_EUNSUPPORTED;
    if (d->n_in % 32 != 0 || d->n_in % elems != 0) return INGOT_ATTN_EUNSUPPORTED;
    if (uint64_t(d->n_in) / elems * bytes > 0x7fffffffull) return INGOT_ATTN_EUNSUPPORTED;
    if (uint64_t(d->out_offset) + uint64_t(d->n_tok) * d->n_out > 0xffffffffffffull) return INGOT_ATTN_EINVAL;
    if (d->n_splits > 8) return INGOT_ATTN_EINVAL;
    return INGOT_ATTN_OK;
}

// The descriptor and input checks shared by ingot_proj and ingot_proj_rope_kv.
int check_proj(const void* const* w, const float* x, const float* norm_w, const IngotProjDesc* d) {
    if (!d || !w || !x || d->n_in == 0 || d->n_mats < 1 || d->n_mats > 3) return INGOT_ATTN_EINVAL;
    if (d->prologue > INGOT_PROJ_RMSNORM || d->epilogue > INGOT_PROJ_SILU_GATE) return INGOT_ATTN_EINVAL;
    uint32_t elems, bytes;
    linear_block(d->type, elems, bytes);
    if (elems == 0) return INGOT_ATTN_EUNSUPPORTED;
    if (d->n_in % 32 != 0 || d->n_in % elems != 0) return INGOT_ATTN_EUNSUPPORTED;
    if (!aligned16(x)) return INGOT_ATTN_EINVAL;
    if (d->prologue == INGOT_PROJ_RMSNORM && (!norm_w || !aligned16(norm_w) || !(d->eps >= 0.f)))
        return INGOT_ATTN_EINVAL;
    if (d->epilogue == INGOT_PROJ_SILU_GATE && (d->n_mats != 2 || d->n_out[0] != d->n_out[1]))
        return INGOT_ATTN_EINVAL;
    for (uint32_t m = 0; m < d->n_mats; m++)
        if (!w[m] || !aligned16(w[m]) || d->n_out[m] == 0) return INGOT_ATTN_EINVAL;
    if (uint64_t(d->n_in) / elems * bytes > 0x7fffffffull) return INGOT_ATTN_EUNSUPPORTED;
    if (d->n_tok > 1) {  // a chunk: the batched kernel, no prologue
        if (d->prologue != INGOT_PROJ_X) return INGOT_ATTN_EUNSUPPORTED;
        for (uint32_t m = 0; m < d->n_mats; m++)
            if (uint64_t(d->n_tok) * d->n_out[m] > 0xffffffffffffull) return INGOT_ATTN_EINVAL;
    }
    return INGOT_ATTN_OK;
}

}  // namespace

extern "C" {

size_t ingot_linear_weight_bytes(const IngotLinearDesc* d) {
    if (check_linear(d)) return 0;
    uint32_t elems, bytes;
    linear_block(d->type, elems, bytes);
    return size_t(d->n_out) * (d->n_in / elems) * bytes;
}

uint32_t ingot_linear_splits(const IngotLinearDesc* d) {
    if (check_linear(d)) return 0;
    return ingot::linear_splits(d->n_in, d->n_out, d->n_tok, d->n_splits, ~size_t(0));
}

size_t ingot_linear_workspace_size(const IngotLinearDesc* d) {
    if (check_linear(d)) return 0;
    return ingot::linear_workspace_size(d->n_in, d->n_out, d->n_tok, d->n_splits);
}

int ingot_linear(const void* w, const float* x, float* out, void* workspace, size_t workspace_bytes,
                 const IngotLinearDesc* d, void* stream) {
    const int rc = check_linear(d);
    if (rc) return rc;
    if (!w || !x || !out) return INGOT_ATTN_EINVAL;
    if (!aligned16(w) || !aligned16(x) || (reinterpret_cast<uintptr_t>(out) & 3u) != 0)
        return INGOT_ATTN_EINVAL;
    if (workspace && !aligned16(workspace)) return INGOT_ATTN_EINVAL;
    const int lrc = ingot::launch_linear(d->type, w, x, out + d->out_offset, d->n_in, d->n_out,
                                         d->n_tok, d->accumulate ? 1u : 0u, d->n_splits, workspace,
                                         workspace ? workspace_bytes : 0,
                                         static_cast<hipStream_t>(stream));
    return lrc == 0 ? INGOT_ATTN_OK : lrc == -2 ? INGOT_ATTN_EUNSUPPORTED
         : lrc == -1 ? INGOT_ATTN_EINVAL : INGOT_ATTN_EHIP;
}

int ingot_proj(const void* const* w, const float* x, const float* norm_w, float* const* out,
               const IngotProjDesc* d, void* stream) {
    const int rc = check_proj(w, x, norm_w, d);
    if (rc) return rc;
    const uint32_t n_outs = d->epilogue == INGOT_PROJ_SILU_GATE ? 1 : d->n_mats;
    if (!out) return INGOT_ATTN_EINVAL;
    for (uint32_t m = 0; m < n_outs; m++)
        if (!out[m] || (reinterpret_cast<uintptr_t>(out[m]) & 3u) != 0) return INGOT_ATTN_EINVAL;
    const int lrc = ingot::launch_proj(d->type, w, x, norm_w, out, d->n_in, d->n_out, d->n_mats,
                                       int(d->prologue), int(d->epilogue), d->eps,
                                       static_cast<hipStream_t>(stream), nullptr,
                                       d->n_tok > 1 ? d->n_tok : 1u);
    return lrc == 0 ? INGOT_ATTN_OK : lrc == -2 ? INGOT_ATTN_EUNSUPPORTED
         : lrc == -1 ? INGOT_ATTN_EINVAL : INGOT_ATTN_EHIP;
}

int ingot_proj_rope_kv(const void* const* w, const float* x, const float* norm_w, float* q, float* k,
                       float* v, uint16_t* k_cache, uint16_t* v_cache, const float* inv_freq,
                       const IngotProjDesc* p, const IngotRopeKvDesc* r, void* stream) {
    const int rc = check_proj(w, x, norm_w, p);
    if (rc) return rc;
    if (!r || p->n_mats != 3 || p->epilogue != INGOT_PROJ_STORE || r->n_tok != 1 || p->n_tok > 1)
        return INGOT_ATTN_EINVAL;
    if (r->n_head == 0 || r->n_head_kv == 0 || r->head_dim == 0) return INGOT_ATTN_EINVAL;
    if (r->head_dim % 4 != 0) return INGOT_ATTN_EUNSUPPORTED;
    const uint64_t qd = uint64_t(r->n_head) * r->head_dim, kvd = uint64_t(r->n_head_kv) * r->head_dim;
    if (p->n_out[0] != qd || p->n_out[1] != kvd || p->n_out[2] != kvd) return INGOT_ATTN_EINVAL;
    if (!q || !k || !v || !k_cache || !v_cache || !inv_freq) return INGOT_ATTN_EINVAL;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || r->dst_offset % 4 != 0 ||
        (reinterpret_cast<uintptr_t>(k_cache) & 7u) != 0 || (reinterpret_cast<uintptr_t>(v_cache) & 7u) != 0)
        return INGOT_ATTN_EINVAL;
    auto* kc = reinterpret_cast<_Float16*>(k_cache) + r->dst_offset;
    auto* vc = reinterpret_cast<_Float16*>(v_cache) + r->dst_offset;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    // One launch for the streamed weight types; the others take the two-launch sequence
    // through k and v (the same results).
    const ingot::ProjRope rope{inv_freq, kc, vc, r->head_dim, r->pos};
    float* outs[3] = {q, k, v};
    int lrc = ingot::launch_proj(p->type, w, x, norm_w, outs, p->n_in, p->n_out, 3, int(p->prologue),
                                 3 /* rope / KV store */, p->eps, st, &rope);
    if (lrc == -2) {
        lrc = ingot::launch_proj(p->type, w, x, norm_w, outs, p->n_in, p->n_out, 3, int(p->prologue),
                                 INGOT_PROJ_STORE, p->eps, st);
        if (lrc == 0)
            lrc = ingot::launch_rope_kv_store(q, k, v, kc, vc, inv_freq, r->n_head, r->n_head_kv,
                                              r->head_dim, r->pos, 1, uint32_t(qd), uint32_t(kvd), st);
    }
    return lrc == 0 ? INGOT_ATTN_OK : lrc == -2 ? INGOT_ATTN_EUNSUPPORTED
         : lrc == -1 ? INGOT_ATTN_EINVAL : INGOT_ATTN_EHIP;
}

// Decode split count (the fallback kernel chooses its own key slices).
uint32_t decode_split_count(const IngotAttnDecodeDesc* d) {
    return mfma_head_dim(d->head_dim) ? ingot::decode_splits(d->n_keys, d->head_dim, d->n_splits)
                                      : ingot::attn_any_slices(d->n_keys, 1);
}

uint32_t ingot_attn_decode_splits(const IngotAttnDecodeDesc* d) {
    if (check_decode(d)) return 0;
    return decode_split_count(d);
}

// Prefill split count of the MFMA kernel over its workgroup units (1 for the fallback kernel).
uint32_t prefill_split_count(const IngotAttnPrefillDesc* d) {
    if (!mfma_head_dim(d->head_dim)) return 1;
    const uint32_t group = d->n_head / d->n_head_kv;
    const uint32_t units = d->n_head_kv * (group / ingot::prefill_unit_heads(group, d->head_dim));
    return ingot::prefill_splits(d->pos, d->n_tok, units, d->head_dim, d->n_splits);
}

uint32_t ingot_attn_prefill_splits(const IngotAttnPrefillDesc* d) {
    if (check_prefill(d)) return 0;
    return prefill_split_count(d);
}

size_t ingot_attn_decode_workspace_size(const IngotAttnDecodeDesc* d) {
    if (check_decode(d)) return 0;
    const uint32_t splits = decode_split_count(d);
    if (!mfma_head_dim(d->head_dim))  // the fallback kernel's slice records
        return kCounterBytes + (splits > 1 ? size_t(d->n_head) * splits * (d->head_dim + 2) * sizeof(float) : 0);
    return kCounterBytes + (splits > 1 ? size_t(d->n_head) * ingot::kDecodeHeadRecordBytes : 0);
}

size_t ingot_attn_prefill_workspace_size(const IngotAttnPrefillDesc* d) {
    if (check_prefill(d)) return 0;
    const uint32_t splits = prefill_split_count(d);
    const size_t parts = splits > 1 ? size_t(splits) * d->n_tok * d->n_head *
                                          ingot::prefill_record_bytes(d->head_dim) : 0;
    return prefill_part_offset(d->n_head) + parts;
}

int ingot_attn_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                      void* workspace, size_t workspace_bytes, const IngotAttnDecodeDesc* d,
                      void* stream) {
    const int rc = check_decode(d);
    if (rc) return rc;
    if (!q || !k_cache || !v_cache || !out || !workspace) return INGOT_ATTN_EINVAL;
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out) ||
        !aligned16(workspace))
        return INGOT_ATTN_EINVAL;
    if (workspace_bytes < ingot_attn_decode_workspace_size(d)) return INGOT_ATTN_EWORKSPACE;
    const uint32_t splits = decode_split_count(d);
    const auto* k = reinterpret_cast<const _Float16*>(k_cache) + d->kv_offset;
    const auto* v = reinterpret_cast<const _Float16*>(v_cache) + d->kv_offset;
    const int lrc = !mfma_head_dim(d->head_dim)
        ? ingot::launch_attn_any(q, k, v, out, reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes),
                                 d->n_keys - 1, 1, d->n_head * d->head_dim, d->n_head, d->n_head_kv, d->head_dim,
                                 d->scale, static_cast<hipStream_t>(stream))
        : ingot::launch_decode(q, k, v, out, workspace, d->n_keys, splits, d->n_head_kv,
                                         d->n_head / d->n_head_kv, d->head_dim, d->scale,
                                         static_cast<hipStream_t>(stream));
    return lrc == 0 ? INGOT_ATTN_OK : lrc == -2 ? INGOT_ATTN_EUNSUPPORTED
         : lrc == -1 ? INGOT_ATTN_EINVAL : INGOT_ATTN_EHIP;
}

int ingot_attn_prefill(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                       void* workspace, size_t workspace_bytes, const IngotAttnPrefillDesc* d,
                       void* stream) {
    const int rc = check_prefill(d);
    if (rc) return rc;
    if (!q || !k_cache || !v_cache || !out || !workspace) return INGOT_ATTN_EINVAL;
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out) ||
        !aligned16(workspace))
        return INGOT_ATTN_EINVAL;
    if (workspace_bytes < ingot_attn_prefill_workspace_size(d)) return INGOT_ATTN_EWORKSPACE;
    const auto* k = reinterpret_cast<const _Float16*>(k_cache) + d->kv_offset;
    const auto* v = reinterpret_cast<const _Float16*>(v_cache) + d->kv_offset;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const uint32_t splits = prefill_split_count(d);
    char* part = static_cast<char*>(workspace) + prefill_part_offset(d->n_head);
    const int lrc = !mfma_head_dim(d->head_dim)
        ? ingot::launch_attn_any(q, k, v, out, nullptr, d->pos, d->n_tok, d->q_stride, d->n_head, d->n_head_kv,
                                 d->head_dim, d->scale, st)
        : ingot::launch_prefill(q, k, v, out, part, d->pos, d->n_tok, d->q_stride, d->n_head_kv,
                                          d->n_head / d->n_head_kv, d->head_dim, splits, d->scale, st);
    return lrc == 0 ? INGOT_ATTN_OK : lrc == -2 ? INGOT_ATTN_EUNSUPPORTED
         : lrc == -1 ? INGOT_ATTN_EINVAL : INGOT_ATTN_EHIP;
}

int ingot_rmsnorm(const float* x, const float* w, float* out, uint32_t n, uint32_t n_rows, float eps,
                  void* stream) {
    if (!x || !w || !out || n == 0 || n_rows == 0 || n % 4 != 0) return INGOT_ATTN_EINVAL;
    if (!aligned16(x) || !aligned16(w) || !aligned16(out) || !(eps >= 0.f)) return INGOT_ATTN_EINVAL;
    if (n_rows > 0x7fffffffu) return INGOT_ATTN_EINVAL;
    return ingot::launch_rmsnorm(x, w, out, n, n_rows, eps, static_cast<hipStream_t>(stream)) == 0
               ? INGOT_ATTN_OK : INGOT_ATTN_EHIP;
}

int ingot_silu_mul(float* gate, const float* up, uint64_t n, void* stream) {
    if (!gate || !up || n == 0 || n % 4 != 0 || !aligned16(gate) || !aligned16(up)) return INGOT_ATTN_EINVAL;
    const int rc = ingot::launch_silu_mul(gate, up, n, static_cast<hipStream_t>(stream));
    return rc == 0 ? INGOT_ATTN_OK : rc == -1 ? INGOT_ATTN_EINVAL : INGOT_ATTN_EHIP;
}

int ingot_get_rows(uint32_t type, const void* w, uint32_t n, uint32_t n_rows, const int32_t* tokens,
                   uint32_t n_tok, float* out, void* stream) {
    if (!w || !tokens || !out || n == 0 || n_rows == 0 || n_tok == 0 || n_tok > 0x7fffffffu)
        return INGOT_ATTN_EINVAL;
    uint32_t elems, bytes;
    linear_block(type, elems, bytes);
    if (elems == 0 || n % elems != 0) return INGOT_ATTN_EUNSUPPORTED;
    if ((reinterpret_cast<uintptr_t>(w) & 3u) != 0 || (reinterpret_cast<uintptr_t>(out) & 3u) != 0)
        return INGOT_ATTN_EINVAL;
    return ingot::launch_get_rows(type, w, uint64_t(n / elems) * bytes, n, n_rows, tokens, n_tok, out,
                                  static_cast<hipStream_t>(stream)) == 0
               ? INGOT_ATTN_OK : INGOT_ATTN_EHIP;
}

int ingot_rope_kv_store(float* q, const float* k, const float* v, uint16_t* k_cache,
                        uint16_t* v_cache, const float* inv_freq, const IngotRopeKvDesc* d,
                        void* stream) {
    if (!d || !k || !v || !k_cache || !v_cache || !inv_freq) return INGOT_ATTN_EINVAL;
    if (d->n_head_kv == 0 || d->head_dim == 0 || d->n_tok == 0) return INGOT_ATTN_EINVAL;
    if (d->head_dim % 4 != 0) return INGOT_ATTN_EUNSUPPORTED;
    const uint64_t kv_dim = uint64_t(d->n_head_kv) * d->head_dim;
    if (d->kv_stride < kv_dim || d->kv_stride % 4 != 0) return INGOT_ATTN_EINVAL;
    if (d->dst_offset % 4 != 0) return INGOT_ATTN_EINVAL;
    if (uint64_t(d->pos) + d->n_tok > 0xffffffffull) return INGOT_ATTN_EINVAL;
    if (q && (d->n_head == 0 || d->q_stride < uint64_t(d->n_head) * d->head_dim || d->q_stride % 4 != 0 || !aligned16(q)))
        return INGOT_ATTN_EINVAL;
    if (!aligned16(k) || !aligned16(v) || (reinterpret_cast<uintptr_t>(k_cache) & 7u) != 0 ||
        (reinterpret_cast<uintptr_t>(v_cache) & 7u) != 0)
        return INGOT_ATTN_EINVAL;
    auto* kc = reinterpret_cast<_Float16*>(k_cache) + d->dst_offset;
    auto* vc = reinterpret_cast<_Float16*>(v_cache) + d->dst_offset;
    const int lrc = ingot::launch_rope_kv_store(q, k, v, kc, vc, inv_freq, d->n_head, d->n_head_kv,
                                                d->head_dim, d->pos, d->n_tok, d->q_stride,
                                                d->kv_stride, static_cast<hipStream_t>(stream));
    return lrc == 0 ? INGOT_ATTN_OK : lrc == -1 ? INGOT_ATTN_EINVAL : INGOT_ATTN_EHIP;
}

const char* ingot_attn_strerror(int code) {
    switch (code) {
        case INGOT_ATTN_OK: return "ok";
        case INGOT_ATTN_EINVAL: return "invalid argument (null/misaligned pointer, zero size or position out of range)";
        case INGOT_ATTN_EUNSUPPORTED: return "unsupported shape (attention: head_dim above 1024 or n_head above 256; linear: weight type without a kernel or n_in not a multiple of its block)";
        case INGOT_ATTN_EWORKSPACE: return "workspace smaller than the *_workspace_size() figure";
        case INGOT_ATTN_EHIP: return "HIP launch failed";
        default: return "unknown error";
    }
}

const char* ingot_attn_version(void) { return "ingot-attn-gfx950 0.2"; }

}  // extern "C"

// attn_internal.h — launchers shared between the kernel files and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <cstdlib>

namespace ingot {

// Upper bounds on split counts; they size the workspace.
constexpr uint32_t kMaxDecodeSplits = 32;
constexpr uint32_t kMaxPrefillSplits = 16;  // INGOT_ATTN_MAX_PREFILL_SPLITS (include/ingot_attn.h)
// Decode hand-off counters (decode_merge.h): one per workgroup unit (at most one per query head),
// each on its own 256-byte line (no false sharing of the device-scope atomics between units).
constexpr uint32_t kCounterStride = 64;  // uint32 words
constexpr size_t kCounterBytes = 65536;  // up to 256 heads

// Decode: split count for n_keys (requested 0 = choose), the most splits a head_dim allows, and
// the query heads one workgroup serves for a group size (a divisor of it, at most 8).
uint32_t decode_splits(uint32_t n_keys, uint32_t head_dim, uint32_t requested);
uint32_t decode_max_splits(uint32_t head_dim);
uint32_t decode_unit_heads(uint32_t group);
// Bytes of one decode split record: o[head_dim] as f32 and one 16-byte chunk holding {m, l}; and
// the fixed region per query head that holds all records of a call (the largest of max splits x
// record bytes over head_dim 64 / 128 / 256: 32 x 528). Both decode kernels use this layout.
constexpr uint32_t decode_record_bytes(uint32_t head_dim) { return head_dim * 4 + 16; }
constexpr size_t kDecodeHeadRecordBytes = 32 * 528;
static_assert(kDecodeHeadRecordBytes >= 32 * decode_record_bytes(64) &&
              kDecodeHeadRecordBytes >= 32 * decode_record_bytes(128) &&
              kDecodeHeadRecordBytes >= 16 * decode_record_bytes(256), "decode record region");
// Prefill: split count (n_units = workgroup units: KV heads x group / prefill_unit_heads) and
// the query heads one MFMA-prefill unit serves (a divisor of the group: at most 3, 1 for
// head_dim 256). A split record is o[head_dim] normalized (o / l) as f16, then {m, l} as f32 in a
// 16-byte chunk.
uint32_t prefill_splits(uint32_t pos, uint32_t n_tok, uint32_t n_units, uint32_t head_dim,
                        uint32_t requested);
uint32_t prefill_unit_heads(uint32_t group, uint32_t head_dim);
constexpr size_t prefill_record_bytes(uint32_t head_dim) { return head_dim * 2 + 16; }

// Decode attention, dispatched by launch_decode: head_dim 128 with groups 1..4 (or multiples of
// 3 or 4) take the tuned kernel (attn_decode.hip), every other shape the generic one
// (attn_decode_any.hip). Both keep their hand-off counters in the workspace's first
// kCounterBytes and the records after them. Return 0, -1 (grid too large), -2 (shape without a
// kernel) or -4 (launch failed).
int launch_decode(const float* q, const _Float16* k, const _Float16* v, float* out, void* workspace,
                  uint32_t n_keys, uint32_t n_splits, uint32_t n_head_kv, uint32_t group,
                  uint32_t head_dim, float scale, hipStream_t stream);
int launch_decode_g128(const float* q, const _Float16* k, const _Float16* v, float* out, char* recs,
                       unsigned int* counters, uint32_t n_keys, uint32_t n_splits, uint32_t n_head_kv,
                       uint32_t group, float scale, hipStream_t stream);
int launch_decode_any(const float* q, const _Float16* k, const _Float16* v, float* out, void* recs,
                      unsigned int* counters,
                      uint32_t n_keys, uint32_t n_splits, uint32_t n_head_kv, uint32_t group,
                      uint32_t head_dim, float scale, hipStream_t stream);
// The MFMA prefill kernel (attn_prefill.hip), head_dim 64, 128 or 256.
int launch_prefill(const float* q, const _Float16* k, const _Float16* v, float* out, char* part,
                   uint32_t pos, uint32_t n_tok, uint32_t q_stride, uint32_t n_head_kv,
                   uint32_t group, uint32_t head_dim, uint32_t n_splits, float scale,
                   hipStream_t stream);

// Attention for head sizes without an MFMA kernel (attn_naive.hip): head_dim 1..1024, decode
// (pos = n_keys - 1, n_tok = 1) and causal prefill. Decode splits the keys into
// attn_any_slices(n_keys, 1) slices whose records (head_dim + 2 floats each, per head) go to
// `part` and are merged by a second launch. Returns 0, -1 (grid too large), -2 (head_dim above
// 1024) or -4 (launch failed).
constexpr uint32_t kMinSliceKeys = 256;
constexpr uint32_t kMaxAnySlices = 64;
uint32_t attn_any_slices(uint32_t n_keys, uint32_t n_tok);
int launch_attn_any(const float* q, const _Float16* k, const _Float16* v, float* out, float* part, uint32_t pos,
                    uint32_t n_tok, uint32_t q_stride, uint32_t n_head, uint32_t n_head_kv, uint32_t head_dim,
                    float scale, hipStream_t stream);

// RoPE on q (in place, skipped when q is null) and k; K and V as f16 into the cache rows.
// Returns 0, -1 (grid too large) or -4 (launch failed).
int launch_rope_kv_store(float* q, const float* k, const float* v, _Float16* k_cache,
                         _Float16* v_cache, const float* inv_freq, uint32_t n_head,
                         uint32_t n_head_kv, uint32_t head_dim, uint32_t pos, uint32_t n_tok,
                         uint32_t q_stride, uint32_t kv_stride, hipStream_t stream);

// Linear layer workspace: split-K completion counters (one 64-byte line per output tile, for up
// to kLinearMaxTiles tiles), then the partial tiles.
constexpr size_t kLinearCounterBytes = 16384;
constexpr uint32_t kLinearMaxTiles = 256;

// out (+)= W·x over a GGUF weight layout (type id as in ggml). With a workspace (zero-filled
// once) the batched path may split K across workgroups; without one it never does.
// Returns 0, -1 (grid too large), -2 (type without a kernel) or -4 (launch failed).
int launch_linear(uint32_t type, const void* W, const float* x, float* out, uint32_t n_in,
                  uint32_t n_out, uint32_t n_tok, uint32_t accumulate, uint32_t n_splits,
                  void* workspace, size_t workspace_bytes, hipStream_t stream);
// The rope / KV-store epilogue's arguments: the cache rows of the token (K and V, f16), the
// rotary inverse frequencies, head_dim and the position.
struct ProjRope {
    const float* inv_freq;
    _Float16* k_row;
    _Float16* v_row;
    uint32_t head_dim, pos;
};

// One token through n_mats (1..3) matrices of one type sharing x, with the rmsnorm prologue
// (pro 1, norm weights aux) and the store / accumulate / silu-gate / rope-KV epilogue
// (epi 0 / 1 / 2 / 3; 3 takes q, k, v and `rope`, and only the streamed types).
// Returns 0, -2 (type without a kernel, rows too long to stage) or -4 (launch failed).
int launch_proj(uint32_t type, const void* const* W, const float* x, const float* aux,
                float* const* out, uint32_t n_in, const uint32_t* n_out, uint32_t n_mats,
                int pro, int epi, float eps, hipStream_t stream, const ProjRope* rope = nullptr,
                uint32_t n_tok = 1);
// Split count for the batched path (requested: 0 = choose); `workspace_bytes` bounds it.
uint32_t linear_splits(uint32_t n_in, uint32_t n_out, uint32_t n_tok, uint32_t requested,
                       size_t workspace_bytes);
size_t linear_workspace_size(uint32_t n_in, uint32_t n_out, uint32_t n_tok, uint32_t requested);

// Per-layer model ops (model_ops.hip). Return 0, -1 (grid too large) or -4 (launch failed).
int launch_rmsnorm(const float* x, const float* w, float* out, uint32_t n, uint32_t n_rows, float eps,
                   hipStream_t stream);
int launch_silu_mul(float* gate, const float* up, uint64_t n, hipStream_t stream);
int launch_get_rows(uint32_t type, const void* w, uint64_t row_bytes, uint32_t n, uint32_t n_rows,
                    const int32_t* tokens, uint32_t n_tok, float* out, hipStream_t stream);

}  // namespace ingot

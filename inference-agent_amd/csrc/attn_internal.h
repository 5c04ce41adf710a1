// attn_internal.h — launchers shared between the kernel files and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ingot {

// Upper bounds on split counts; they size the workspace.
constexpr uint32_t kMaxDecodeSplits = 1024;
constexpr uint32_t kMaxPrefillSplits = 16;

uint32_t decode_splits(uint32_t n_keys, uint32_t n_head_kv, uint32_t requested);
uint32_t prefill_splits(uint32_t pos, uint32_t n_tok, uint32_t n_head, uint32_t requested);

// Return 0, -2 (unsupported group) or -4 (launch failed).
int launch_decode(const float* q, const _Float16* k, const _Float16* v, float* out, float* part,
                  unsigned int* counters, uint32_t n_keys, uint32_t n_splits, uint32_t n_head_kv,
                  uint32_t group, float scale, hipStream_t stream);
int launch_prefill(const float* q, const _Float16* k, const _Float16* v, float* out, float* part,
                   uint32_t pos, uint32_t n_tok, uint32_t q_stride, uint32_t n_head_kv,
                   uint32_t group, uint32_t n_splits, float scale, hipStream_t stream);

}  // namespace ingot

// attn_oracle.h — CPU restatement of Ingot's attention (TEST INFRASTRUCTURE ONLY; see
// attn_oracle.cpp for the reference lines each function follows). Not part of the product.
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void oracle_f32_to_f16(const float* in, uint16_t* out, size_t n);
void oracle_f16_to_f32(const uint16_t* in, float* out, size_t n);
void oracle_softmax(float* x, size_t n);

// Decode: q [n_head*head_dim]; k_cache/v_cache: layer slice, rows [n_keys][n_head_kv*head_dim];
// out [n_head*head_dim]. Returns 0, or -1 on a bad argument.
int oracle_attn_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                       int n_head, int n_head_kv, int head_dim, int n_keys, float scale,
                       int n_threads);

// Causal prefill: q/out [n_tok][q_stride]; cache rows 0..pos+n_tok-1. Returns 0 or -1.
int oracle_attn_prefill(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                        int n_head, int n_head_kv, int head_dim, int pos, int n_tok, int q_stride,
                        float scale, int n_threads);

#ifdef __cplusplus
}
#endif

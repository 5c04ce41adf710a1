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

// Rotary frequencies (head_dim/2 entries); factors may be NULL.
void oracle_rope_inv_freq(float theta, int head_dim, const float* factors, float* out);

// ops::rope in place on x [n_tok][row_stride], token t at position pos + t.
void oracle_rope(float* x, int n_tok, int row_stride, int n_heads, int head_dim, int pos,
                 const float* inv_freq);

// RoPE on q (in place; q may be NULL) and k, then K and V rounded to f16 into the cache rows
// dst_offset + t*kv_dim (kv_dim = n_head_kv*head_dim). Returns 0 or -1.
int oracle_rope_kv_store(float* q, int q_stride, int n_head, const float* k, const float* v,
                         int kv_stride, uint16_t* k_cache, uint16_t* v_cache, size_t dst_offset,
                         int n_head_kv, int head_dim, int pos, int n_tok, const float* inv_freq);

// Linear layer over a GGUF weight layout (linear_oracle.cpp). type = GGUF type id (F32 0,
// F16 1, Q4_0 2, Q4_1 3, Q8_0 8, Q6_K 14, BF16 30). out[t*n_out + r] (+)= W[r]·x[t].
// oracle_linear follows ops::matvec (f32); oracle_linear_f16 the Metal batched path (x and
// weights rounded to f16). Return 0 or -1.
int oracle_dequant_row(int type, const uint8_t* row, float* out, int n);
int oracle_linear(int type, const uint8_t* w, const float* x, float* out, int n_in, int n_out,
                  int n_tok, int accumulate, int n_threads);
int oracle_linear_f16(int type, const uint8_t* w, const float* x, float* out, int n_in, int n_out,
                      int n_tok, int accumulate, int n_threads);

// Model-level pieces (model_oracle.cpp).
void oracle_rmsnorm(const float* x, const float* w, float* out, int n, int n_rows, float eps);
void oracle_silu_mul(float* gate, const float* up, size_t n);

typedef struct OracleTensor {
    int type;          // GGUF type id
    const void* data;  // the tensor's bytes (GGUF layout)
} OracleTensor;

typedef struct OracleLayer {
    const float* attn_norm;
    const float* ffn_norm;
    OracleTensor wq, wk, wv, wo, w_gate, w_up, w_down;
} OracleLayer;

typedef struct OracleModel {
    int n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab;
    float rms_eps;
    const float* rope_inv_freq;  // head_dim/2
    OracleTensor tok_embd, output;
    const float* output_norm;
    const OracleLayer* layers;   // n_layer
} OracleModel;

// CpuBackend::forward for one token at pos (0 <= pos < n_ctx): writes K/V (f16) into the cache
// rows of pos and the logits [n_vocab]. f16_linear selects the Metal batched linear numerics.
int oracle_forward(const OracleModel* m, uint16_t* k_cache, uint16_t* v_cache, int n_ctx, int token,
                   int pos, float* logits, int f16_linear, int n_threads);

#ifdef __cplusplus
}
#endif

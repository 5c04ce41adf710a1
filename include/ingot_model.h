/*
 * ingot_model.h — C ABI of the small per-layer ops of the MI355X Llama forward pass: the steps
 * of `MetalBackend::forward_batch` (src/metal_backend.mm:419-471) around attention
 * (ingot_attn.h) and the linear layers (ingot_linear.h).
 *
 * Same conventions as ingot_attn.h: device pointers owned by the caller, stream-ordered, 0 or a
 * negative INGOT_ATTN_E* code, no workspace.
 */
#ifndef INGOT_MODEL_H
#define INGOT_MODEL_H

#include "ingot_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* out[r][i] = x[r][i] * (1 / sqrt(mean_i(x[r][i]^2) + eps)) * w[i] for r < n_rows, i < n.
 * Replaces encode_rmsnorm (src/metal_backend.mm:312-322; NormParams {n, eps}); the CPU path is
 * ops::rmsnorm (src/ops.cpp:226-231). n a multiple of 4; x, w, out 16-byte aligned; out may
 * equal x. */
int ingot_rmsnorm(const float* x, const float* w, float* out, uint32_t n, uint32_t n_rows, float eps,
                  void* stream);

/* gate[i] = silu(gate[i]) * up[i], silu(g) = g / (1 + exp(-g)), for i < n (a multiple of 4).
 * Replaces encode_silu_mul (src/metal_backend.mm:411-417); the CPU path is
 * src/cpu_backend.cpp:77 with ops::silu (src/ops.h:35). gate and up 16-byte aligned. */
int ingot_silu_mul(float* gate, const float* up, uint64_t n, void* stream);

/* out[t][0..n) = row tokens[t] of the GGUF embedding table w (type, n = ne[0], n_rows = ne[1]),
 * dequantized to f32, for t < n_tok. tokens is a device array. An id outside [0, n_rows) gives
 * a zero row: validate ids on the host first, as forward_batch does (src/metal_backend.mm:
 * 423-424, "token id out of range"). The reference dequantizes on the CPU
 * (ops::dequant_row, src/ops.cpp:196-198, at src/metal_backend.mm:428); with tied embeddings
 * the table is on the device anyway for the logits. Types as ingot_linear; n a multiple of the
 * type's block. */
int ingot_get_rows(uint32_t type, const void* w, uint32_t n, uint32_t n_rows, const int32_t* tokens,
                   uint32_t n_tok, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INGOT_MODEL_H */

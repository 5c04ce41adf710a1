/*
 * ingot_linear.h — C ABI of the MI355X (gfx950) linear layer over GGUF weight layouts.
 *
 * Replaces `encode_linear` of the Metal backend (src/metal_backend.mm:282-310), used by the
 * attention output projection with its residual accumulate (`encode_linear(enc, *L.wo, in, x_,
 * 0, true, n)`, src/metal_backend.mm:446-447) and every other projection of the forward pass;
 * the CPU path is `ops::matvec` + `x += tmp` (src/ops.cpp:218-225, src/cpu_backend.cpp:71-72).
 *
 * Same conventions as ingot_attn.h (device pointers owned by the caller, stream-ordered,
 * 0 or a negative INGOT_ATTN_E* code). The library is the same libingot_attn.so.
 *
 * W keeps the GGUF on-disk layout: ne = [n_in, n_out], row r is n_in elements stored as
 * n_in / block_size blocks of the tensor type (src/gguf.h:30-33, src/ops.cpp:33-87):
 *   F32 (0), F16 (1), BF16 (30): plain rows;
 *   Q8_0 (8): 34-byte blocks of 32; Q4_0 (2): 18-byte blocks of 32; Q4_1 (3): 20-byte blocks
 *   of 32; Q6_K (14): 210-byte blocks of 256.
 * These are the types the reference's GPU path has kernels for (src/metal_backend.mm:61-83)
 * plus BF16, which its CPU path also reads (src/ops.cpp:89-99). Others return
 * INGOT_ATTN_EUNSUPPORTED, as the reference throws "no matvec kernel for type".
 *
 * Numerics: n_tok == 1 computes in f32 from the exact dequantized weights (as ops::matvec and
 * the Metal matvec kernels); n_tok > 1 rounds x and the dequantized weights to f16 and
 * accumulates in f32 (as the Metal to_half + matmul path, src/metal_backend.mm:385-392).
 */
#ifndef INGOT_LINEAR_H
#define INGOT_LINEAR_H

#include "ingot_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Mirrors MatvecParams / MatmulParams (shaders/kernels.metal:19, 716: n_in, n_out, n_tok,
 * out_offset, accumulate) plus the weight type (gguf::TensorInfo::type) and, as in the
 * attention descriptors, a requested split count for the batched path. */
typedef struct IngotLinearDesc {
    uint32_t type;        /* GGUF tensor type id */
    uint32_t n_in;        /* W.ne[0]; a multiple of 32 (of 256 for Q6_K) */
    uint32_t n_out;       /* W.ne[1] */
    uint32_t n_tok;       /* rows of x and of out */
    uint32_t out_offset;  /* elements added to out */
    uint32_t accumulate;  /* 0: out = W·x; 1: out += W·x (the residual add after wo) */
    uint32_t n_splits;    /* n_tok > 1: ways to split n_in across workgroups; 0 = library's
                             choice, 1 = never; at most 8 */
} IngotLinearDesc;

/* Bytes of W for this descriptor (n_out rows of the type's row size), 0 if the descriptor is
 * invalid or the type unsupported. */
size_t ingot_linear_weight_bytes(const IngotLinearDesc* d);

/* Split count the call with this descriptor and a large enough workspace would use (1 for
 * n_tok == 1 or no split), 0 for an invalid descriptor. */
uint32_t ingot_linear_splits(const IngotLinearDesc* d);

/* Bytes of device workspace that lets the batched path (n_tok > 1) split the reduction over
 * n_in across workgroups when the output alone has too few tiles to fill the GPU. The
 * workspace must be zero-filled once when it is allocated (it holds completion counters that
 * every call leaves at zero again); one workspace of the largest size serves every smaller
 * call. Returns 0 for an invalid descriptor. */
size_t ingot_linear_workspace_size(const IngotLinearDesc* d);

/* out[out_offset + t*n_out + r] (+)= sum_k W[r][k] * x[t*n_in + k] for t < n_tok, r < n_out.
 *   w          weight bytes, 16-byte aligned (GGUF data is 32-byte aligned)
 *   x          [n_tok][n_in] f32, 16-byte aligned
 *   out        f32, 4-byte aligned, must not overlap x or w
 *   workspace  NULL (n_in is never split) or 16-byte aligned device memory of workspace_bytes;
 *              with less than ingot_linear_workspace_size() bytes the call splits less or not
 *              at all.
 * Deterministic: the split partials are summed in a fixed order, so equal inputs and equal
 * workspace sizes give bit-identical results; calls with and without a split differ by f32
 * rounding only. Not thread-safe per workspace (calls sharing one must be ordered on a
 * stream). */
int ingot_linear(const void* w, const float* x, float* out, void* workspace, size_t workspace_bytes,
                 const IngotLinearDesc* d, void* stream);

/* One decode token through up to three projections that read the same input, in one launch,
 * with the per-layer step before and after fused in (ingot_proj):
 *   prologue INGOT_PROJ_X        x' = x
 *            INGOT_PROJ_RMSNORM  x' = x * (1 / sqrt(mean(x^2) + eps)) * norm_w — the rmsnorm
 *                                before q/k/v and before gate/up (src/metal_backend.mm:
 *                                433-437, 448-449; ops::rmsnorm, src/ops.cpp:226-231)
 *   epilogue INGOT_PROJ_STORE      out[m] = W[m]·x'
 *            INGOT_PROJ_ACCUMULATE out[m] += W[m]·x' (the residual adds after wo and w_down)
 *            INGOT_PROJ_SILU_GATE  n_mats == 2 (gate, up), equal n_out:
 *                                  out[0] = silu(W[0]·x') * (W[1]·x'), silu(g) = g/(1+exp(-g))
 *                                  (encode_silu_mul, src/metal_backend.mm:411-417;
 *                                  src/cpu_backend.cpp:77, ops::silu src/ops.h:35)
 * The reference encodes these as separate dispatches (encode_rmsnorm, three or two
 * encode_linear calls, encode_silu_mul: src/metal_backend.mm:433-452); the results equal those
 * of ingot_rmsnorm, ingot_linear (n_tok == 1) and ingot_silu_mul run in sequence, bit for bit.
 * Every matrix has the same type and n_in. */
enum {
    INGOT_PROJ_X = 0,
    INGOT_PROJ_RMSNORM = 1
};
enum {
    INGOT_PROJ_STORE = 0,
    INGOT_PROJ_ACCUMULATE = 1,
    INGOT_PROJ_SILU_GATE = 2
};

typedef struct IngotProjDesc {
    uint32_t type;       /* GGUF tensor type id, shared by the matrices */
    uint32_t n_in;       /* as IngotLinearDesc.n_in */
    uint32_t n_mats;     /* 1..3 */
    uint32_t n_out[3];   /* rows of each matrix (entries past n_mats ignored) */
    uint32_t prologue;   /* INGOT_PROJ_X or INGOT_PROJ_RMSNORM */
    uint32_t epilogue;   /* INGOT_PROJ_STORE, INGOT_PROJ_ACCUMULATE or INGOT_PROJ_SILU_GATE */
    float eps;           /* rmsnorm epsilon (prologue INGOT_PROJ_RMSNORM) */
    uint32_t n_tok;      /* tokens: 0 or 1 = one decode token; > 1 = a chunk (see below) */
} IngotProjDesc;

/* A chunk (n_tok > 1) runs the batched linear-layer kernel over the rows of every matrix in one
 * launch, without split-K: x is [n_tok][n_in], out[m] is [n_tok][n_out[m]], prologue
 * INGOT_PROJ_X (else INGOT_ATTN_EUNSUPPORTED). With INGOT_PROJ_STORE or INGOT_PROJ_ACCUMULATE
 * each out[m] equals that of ingot_linear (n_tok, n_splits = 1) on matrix m, bit for bit. It
 * replaces the q/k/v encode_linear calls of a chunk (src/metal_backend.mm:440-442) where the
 * three matrices' row tiles together fill the GPU better than each alone (Llama-3.2-3B at 512
 * tokens: 160 tiles of 256 rows x 64 tokens against 96 + 32 + 32 in three launches). With
 * INGOT_PROJ_SILU_GATE (two matrices of equal n_out) out[0] = silu(W[0]·x) * (W[1]·x) per
 * element, equal bit for bit to ingot_linear on each matrix (n_splits = 1) followed by
 * ingot_silu_mul; it replaces the gate and up encode_linear calls and encode_silu_mul of a chunk
 * (src/metal_backend.mm:448-451) with one launch whose tiles hold 128 rows of each matrix.
 *   w       host array of n_mats device pointers to the weight bytes, each 16-byte aligned
 *   x       [n_in] f32 ([n_tok][n_in] for a chunk), 16-byte aligned
 *   norm_w  [n_in] f32 rmsnorm weights, 16-byte aligned (INGOT_PROJ_RMSNORM; else ignored)
 *   out     host array of n_mats device pointers, f32 [n_out[m]], 4-byte aligned, not
 *           overlapping x or w (one pointer for INGOT_PROJ_SILU_GATE)
 * Returns INGOT_ATTN_EUNSUPPORTED for a type without a kernel or rows too long to stage
 * (n_in * 8 + 8 rows' bytes beyond 160 KB). */
int ingot_proj(const void* const* w, const float* x, const float* norm_w, float* const* out,
               const IngotProjDesc* d, void* stream);

/* One decode token's q/k/v step, end to end: ingot_proj with matrices (wq, wk, wv), the
 * descriptor's prologue and INGOT_PROJ_STORE, followed by ingot_rope_kv_store for that token
 * (r->n_tok == 1): q rotated in place, K rotated and V rounded to f16 into the cache rows at
 * r->dst_offset. For Q4_0, Q4_1, Q8_0, F16 and BF16 weights this is one launch and k, v are not
 * written; for the other types it is the two launches through k and v. Either way q and the
 * cache rows equal those of the two calls in sequence, bit for bit. Replaces, for one token,
 * the encode_rmsnorm + q/k/v encode_linear + rope + rope_k_to_cache + to_half sequence of
 * src/metal_backend.mm:433-444 (CpuBackend: src/cpu_backend.cpp:36-49).
 *   q, k, v   f32 [n_head*head_dim], [n_head_kv*head_dim] x2, 16-byte aligned (k, v scratch)
 *   p         n_mats 3, n_out = {n_head*head_dim, n_head_kv*head_dim, n_head_kv*head_dim}
 *   r         as for ingot_rope_kv_store (q_stride / kv_stride ignored: rows are dense) */
int ingot_proj_rope_kv(const void* const* w, const float* x, const float* norm_w, float* q, float* k,
                       float* v, uint16_t* k_cache, uint16_t* v_cache, const float* inv_freq,
                       const IngotProjDesc* p, const IngotRopeKvDesc* r, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INGOT_LINEAR_H */

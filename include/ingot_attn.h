/*
 * ingot_attn.h — C ABI of the MI355X (gfx950) attention hot path of Ingot.
 *
 * This is the drop-in boundary below Ingot's `Backend` interface (src/backend.h:9-23). It
 * replaces the attention step that the Metal backend encodes per layer:
 *   - `encode_attention` (src/metal_backend.mm:336-383) with its two flash paths
 *       decode  (n_tok == 1): attn_decode_g3 + attn_combine (shaders/kernels.metal:428-516)
 *       prefill (n_tok  > 1): attn_prefill                  (shaders/kernels.metal:518-633)
 *   - `encode_kv_store` (src/metal_backend.mm:395-409), the writer of the f16 KV cache
 *       (rope_k_to_cache + to_half, shaders/kernels.metal:270-282, 779-782), together with the
 *       rope on q before it (src/metal_backend.mm:443): ingot_rope_kv_store.
 * The numerics follow Ingot's CPU attention (src/cpu_backend.cpp:46-69, src/ops.cpp:234-241)
 * on K/V rounded to f16 (round-to-nearest-even).
 *
 * Conventions (every entry point):
 *   - All buffers are device pointers owned by the caller; their lifetime is the caller's.
 *   - Q and the output are f32, row-major [n_tok][q_stride] with head h at columns h*head_dim.
 *   - The KV cache is f16 (IEEE binary16 bits in uint16_t), row-major
 *     [layer][n_ctx][n_head_kv*head_dim]; `kv_offset` (elements) selects the layer slice, as
 *     `layer * n_ctx * kv_dim` does at src/metal_backend.mm:345 and :437.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream). Launches are
 *     stream-ordered and asynchronous; nothing here synchronizes the device.
 *   - Return value: 0 on success or a negative INGOT_ATTN_E* code. No exception crosses the ABI.
 *     The reference throws std::runtime_error for the same conditions
 *     (src/cpu_backend.cpp:24-25, src/metal_backend.mm:421-424, 462).
 *   - Not thread-safe per workspace: two calls that share a workspace must be ordered on one
 *     stream.
 *
 * Supported shapes: every head_dim from 1 to 1024 and any group size n_head / n_head_kv, for
 * decode and prefill, as the reference serves them (its flash kernels cover head_dim 128 —
 * decode with groups up to 4, src/metal_backend.mm:339, prefill any group, :360 — and its naive
 * kernel every other shape, src/metal_backend.mm:373-382, shaders/kernels.metal:639-702, with
 * one thread per head dimension, so up to 1024). Here head_dim 128 decode with groups 1..4 (and
 * groups that are multiples of 3 or 4, as units of 3 or 4 heads) runs
 * the tuned kernel (attn_decode.hip), other head_dim 64/256/128 decode shapes the generic split
 * kernel, prefill at 64/128/256 the MFMA kernel (units of up to 3 heads, 1 at head_dim 256), and
 * every other head_dim the fallback kernel (attn_naive.hip, never split). At most 256 query
 * heads (one workspace counter each). Llama-3.2-3B is 24 Q heads / 8 KV heads (group 3);
 * Llama-3.2-1B 32 / 8 with head_dim 64.
 */
#ifndef INGOT_ATTN_H
#define INGOT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define INGOT_ATTN_OK 0
#define INGOT_ATTN_EINVAL (-1)      /* null pointer, zero size, pos/n out of range */
#define INGOT_ATTN_EUNSUPPORTED (-2) /* head_dim above 1024; n_head > 256;
                                       linear: weight type or n_in the kernels do not cover */
#define INGOT_ATTN_EWORKSPACE (-3)  /* workspace smaller than *_workspace_size() */
#define INGOT_ATTN_EHIP (-4)        /* a HIP runtime call or launch failed */

/* Decode descriptor. Mirrors AttnDecParams (src/metal_backend.mm:32): n_head, n_head_kv,
 * head_dim, n_keys, kv_offset, n_splits, scale. n_keys = pos + 1 (src/metal_backend.mm:342).
 * n_splits = 0 lets the library choose the split-KV partition (the reference uses
 * max(1, min(8, n_keys/64)), src/metal_backend.mm:343; this build sizes it for 256 CUs). */
typedef struct IngotAttnDecodeDesc {
    uint32_t n_head;
    uint32_t n_head_kv;
    uint32_t head_dim;
    uint32_t n_keys;
    uint64_t kv_offset;
    uint32_t n_splits;
    float scale;
} IngotAttnDecodeDesc;

/* Prefill descriptor. Mirrors AttnPrefillParams (src/metal_backend.mm:33): n_head, n_head_kv,
 * head_dim, pos, n_tok, kv_offset, q_stride, scale. Query i (0 <= i < n_tok) sits at absolute
 * position pos+i and attends to cache rows 0..pos+i (src/backend.h:16-20; mask `key <= pos+tok`
 * at shaders/kernels.metal:578). n_splits = 0 lets the library split the key range. */
typedef struct IngotAttnPrefillDesc {
    uint32_t n_head;
    uint32_t n_head_kv;
    uint32_t head_dim;
    uint32_t pos;
    uint32_t n_tok;
    uint64_t kv_offset;
    uint32_t q_stride;
    uint32_t n_splits;
    float scale;
} IngotAttnPrefillDesc;

/* KV-store descriptor. Mirrors RopeKParams (src/metal_backend.mm:31: n_heads, head_dim, pos,
 * dst_offset, row_stride) plus what the fused launch also covers: the query heads rotated in
 * place (the reference's separate `rope` dispatch on q, src/metal_backend.mm:443) and the token
 * count. dst_offset is the cache element offset of token 0's row,
 * (layer*n_ctx + pos) * n_head_kv*head_dim (`slot`, src/metal_backend.mm:437). */
typedef struct IngotRopeKvDesc {
    uint32_t n_head;     /* query heads (used when q != NULL) */
    uint32_t n_head_kv;
    uint32_t head_dim;   /* even; a multiple of 4 here */
    uint32_t pos;        /* position of token 0 */
    uint32_t n_tok;
    uint64_t dst_offset;
    uint32_t q_stride;   /* elements between q rows, >= n_head*head_dim */
    uint32_t kv_stride;  /* elements between k (and v) rows, >= n_head_kv*head_dim */
} IngotRopeKvDesc;

/* Bytes of device workspace the call with this descriptor needs. The workspace must be
 * zero-filled once when it is allocated (it holds completion counters that every call leaves
 * at zero again). One workspace of the largest size serves every smaller call. Returns 0 for an
 * invalid descriptor. (The reference preallocates its partials buffer `part_`,
 * src/metal_backend.mm:201.) */
size_t ingot_attn_decode_workspace_size(const IngotAttnDecodeDesc* d);
size_t ingot_attn_prefill_workspace_size(const IngotAttnPrefillDesc* d);

/* The most key splits a prefill call uses (n_splits = 0 chooses at most this many). The split
 * count chosen for a chunk depends on its position, not monotonically, so the prefill workspace
 * that serves every chunk of up to n_batch tokens in a context of n_ctx is
 * ingot_attn_prefill_workspace_size() of the descriptor with pos = n_ctx - n_batch,
 * n_tok = n_batch and n_splits = INGOT_ATTN_MAX_PREFILL_SPLITS. The decode workspace grows with
 * n_keys: n_keys = n_ctx gives the largest. */
#define INGOT_ATTN_MAX_PREFILL_SPLITS 16

/* Split count the library would use for this descriptor (after n_splits = 0 resolution). */
uint32_t ingot_attn_decode_splits(const IngotAttnDecodeDesc* d);
uint32_t ingot_attn_prefill_splits(const IngotAttnPrefillDesc* d);

/* GQA decode attention for one query token.
 *   q        [n_head*head_dim] f32
 *   k_cache, v_cache: f16 cache bases; rows kv_offset/kv_dim .. + n_keys-1 are read
 *   out      [n_head*head_dim] f32
 * Replaces encode_attention's n_tok == 1 branch (src/metal_backend.mm:339-359) and computes
 * what src/cpu_backend.cpp:51-69 computes for one token. */
int ingot_attn_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                      void* workspace, size_t workspace_bytes, const IngotAttnDecodeDesc* d,
                      void* stream);

/* Causal prefill attention for a chunk of n_tok query tokens at positions pos..pos+n_tok-1.
 *   q   [n_tok][q_stride] f32; out [n_tok][q_stride] f32
 *   The cache must already hold rows 0..pos+n_tok-1 of the layer (the reference stores the
 *   chunk's K/V before attention, src/metal_backend.mm:444-445).
 * Replaces encode_attention's n_tok > 1 branch (src/metal_backend.mm:360-371); equal to
 * n_tok successive decode steps (src/backend.h:16-20). */
int ingot_attn_prefill(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                       void* workspace, size_t workspace_bytes, const IngotAttnPrefillDesc* d,
                       void* stream);

/* Decode without a caller-provided workspace and without any allocation: the library uses a
 * device-resident scratch array of INGOT_ATTN_NOALLOC_SCRATCH_BYTES per GPU (enough for up to 64
 * query heads), resolved and zero-filled on the first call on a device (with a fill kernel on
 * `stream`). This entry point has no counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, results and errors as ingot_attn_decode, plus INGOT_ATTN_EWORKSPACE when the
 * call needs more than the scratch holds (more than 64 query heads). Every call on one GPU shares
 * that GPU's scratch: calls that overlap on one GPU race, so order them on one stream. */
#define INGOT_ATTN_NOALLOC_SCRATCH_BYTES (65536u + 64u * 16896u)
int ingot_attn_decode_noalloc(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                              float* out, const IngotAttnDecodeDesc* d, void* stream);

/* RoPE and KV-cache store for n_tok tokens at positions pos..pos+n_tok-1, in one launch:
 *   q        [n_tok][q_stride] f32, rotated in place (NULL: only K and V are handled)
 *   k, v     [n_tok][kv_stride] f32 projections
 *   k_cache, v_cache: f16 cache bases; rows dst_offset/kv_dim .. + n_tok-1 are written
 *   inv_freq [head_dim/2] f32 rotary frequencies (Model::rope_inv_freq, src/model.cpp:59-68)
 * Pair (2i, 2i+1) of each q/k head is rotated by angle float(pos + t) * inv_freq[i]
 * (ops::rope, src/ops.cpp:243-255); K and V are rounded to f16, round to nearest even.
 * Replaces encode_rope on q plus encode_kv_store (src/metal_backend.mm:395-409, 443-444) and
 * does what src/cpu_backend.cpp:43-49 does per token. No workspace. */
int ingot_rope_kv_store(float* q, const float* k, const float* v, uint16_t* k_cache,
                        uint16_t* v_cache, const float* inv_freq, const IngotRopeKvDesc* d,
                        void* stream);

/* Static description of an error code (never NULL). */
const char* ingot_attn_strerror(int code);

/* Library version string, e.g. "ingot-attn-gfx950 0.1". */
const char* ingot_attn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* INGOT_ATTN_H */

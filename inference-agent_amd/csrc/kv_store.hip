// kv_store.hip — RoPE and the f16 KV-cache store for gfx950, fused into one launch.
//
// The step right before attention: q and k of n_tok tokens at positions pos..pos+n_tok-1 are
// rotated by RoPE (pairs (2i, 2i+1) of each head by angle float(pos + t) * inv_freq[i], as
// ops::rope, src/ops.cpp:243-255), and K and V are rounded to f16 (round to nearest even) into
// the cache rows of those positions (src/cpu_backend.cpp:43-49). The Metal backend does this in
// three dispatches — rope on q (shaders/kernels.metal:255-266), rope_k_to_cache (270-282) and
// to_half for V (779-782), encoded by src/metal_backend.mm:395-409 and 443-444 — here it is one,
// because on this GPU every launch costs ~1.8 us before it does anything.
//
// The work is HBM-bound elementwise: thread u of token t owns 4 consecutive elements (two
// rotary pairs) of one of the token's q, k or v rows: one 16-byte load, one 16-byte (q) or
// 8-byte (K, V as f16) store. cos/sin come from the HIP math library's sincosf (full-range
// argument reduction; the angle can reach ~pos radians).
#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

// (x0, x1) -> (x0 c - x1 s, x0 s + x1 c), each product rounded separately (no fused
// multiply-add), as the fused projection epilogue computes it too.
__device__ __forceinline__ float4v rotate2(float4v x, float c0, float s0, float c1, float s1) {
    return float4v{rope_even(x[0], x[1], c0, s0), rope_odd(x[0], x[1], c0, s0),
                   rope_even(x[2], x[3], c1, s1), rope_odd(x[2], x[3], c1, s1)};
}

__global__ __launch_bounds__(256) void rope_kv_store_kernel(
    float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    _Float16* __restrict__ k_cache, _Float16* __restrict__ v_cache,
    const float* __restrict__ inv_freq, uint32_t head_dim, uint32_t pos, uint32_t n_tok,
    uint32_t q_stride, uint32_t kv_stride, uint32_t kv_dim, uint32_t units_q,
    uint32_t units_kv) {
    const uint32_t per_tok = units_q + 2 * units_kv;
    const uint64_t gid = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= uint64_t(n_tok) * per_tok) return;
    const uint32_t t = uint32_t(gid / per_tok), u = uint32_t(gid % per_tok);
    if (u >= units_q + units_kv) {  // V: f32 -> f16
        const uint32_t e = 4 * (u - units_q - units_kv);
        const float4v x = *reinterpret_cast<const float4v*>(v + size_t(t) * kv_stride + e);
        *reinterpret_cast<half4*>(v_cache + size_t(t) * kv_dim + e) =
            half4{_Float16(x[0]), _Float16(x[1]), _Float16(x[2]), _Float16(x[3])};
        return;
    }
    const bool is_q = u < units_q;
    const uint32_t e = 4 * (is_q ? u : u - units_q);
    const uint32_t i = (e % head_dim) / 2;  // first of the two rotary pairs
    const float p = float(pos + t);
    float s0, c0, s1, c1;
    sincosf(p * inv_freq[i], &s0, &c0);
    sincosf(p * inv_freq[i + 1], &s1, &c1);
    if (is_q) {
        float4v* row = reinterpret_cast<float4v*>(q + size_t(t) * q_stride + e);
        *row = rotate2(*row, c0, s0, c1, s1);
    } else {
        const float4v x = rotate2(*reinterpret_cast<const float4v*>(k + size_t(t) * kv_stride + e),
                                  c0, s0, c1, s1);
        *reinterpret_cast<half4*>(k_cache + size_t(t) * kv_dim + e) =
            half4{_Float16(x[0]), _Float16(x[1]), _Float16(x[2]), _Float16(x[3])};
    }
}

}  // namespace

int launch_rope_kv_store(float* q, const float* k, const float* v, _Float16* k_cache,
                         _Float16* v_cache, const float* inv_freq, uint32_t n_head,
                         uint32_t n_head_kv, uint32_t head_dim, uint32_t pos, uint32_t n_tok,
                         uint32_t q_stride, uint32_t kv_stride, hipStream_t stream) {
    const uint32_t kv_dim = n_head_kv * head_dim;
    const uint32_t units_q = q ? n_head * head_dim / 4 : 0;
    const uint32_t units_kv = kv_dim / 4;
    const uint64_t threads = uint64_t(n_tok) * (units_q + 2 * units_kv);
    const uint64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffffu) return -1;
    hipLaunchKernelGGL(rope_kv_store_kernel, dim3(uint32_t(blocks)), dim3(256), 0, stream, q, k, v,
                       k_cache, v_cache, inv_freq, head_dim, pos, n_tok, q_stride, kv_stride,
                       kv_dim, units_q, units_kv);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace ingot

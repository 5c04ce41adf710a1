// attn_common.h — device helpers shared by the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ingot {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kHeadDim = 128;
// log2(e): scores are kept in the base-2 domain (q is pre-multiplied by scale*log2(e)), so the
// softmax uses the hardware exp2 (v_exp_f32). exp(x*s) == exp2(x*s*log2(e)).
constexpr float kLog2e = 1.4426950408889634f;
// Finite "no key seen yet" running maximum, so exp2(m_old - m_new) never evaluates inf - inf.
constexpr float kNoMax = -1e30f;
// Per-(split, head) partial record: o[128] (unnormalized), m (base-2), l, 2 pad words.
constexpr int kPartStride = 132;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// DPP lane permutes inside a row of 16 lanes. Control codes (GCN/CDNA DPP):
//   0xB1 quad_perm [1,0,3,2]  (lane ^ 1)
//   0x4E quad_perm [2,3,0,1]  (lane ^ 2)
//   0x141 row_half_mirror     (lane i <- 7-i within each half-row; after the quad steps this
//                              brings the other quad's value)
//   0x140 row_mirror          (lane i <- 15-i; brings the other half-row's value)
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    x += dpp<0x141>(x);
    x += dpp<0x140>(x);
    return x;
}

// One RoPE pair (x0, x1) rotated by (c, s) = (cos, sin) of the angle: the first and second
// element of the result, with every product rounded on its own (no fused multiply-add), so the
// separate rope kernel and the fused projection epilogue agree bit for bit.
__device__ __forceinline__ float rope_even(float x0, float x1, float c, float s) {
    return __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
}
__device__ __forceinline__ float rope_odd(float x0, float x1, float c, float s) {
    return __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
}

__device__ __forceinline__ half8 load_half8(const _Float16* p) {
    return *reinterpret_cast<const half8*>(p);
}

__device__ __forceinline__ half8 load_half8_nt(const _Float16* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const half8*>(p));
}

}  // namespace ingot

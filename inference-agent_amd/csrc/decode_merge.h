// decode_merge.h — the split-KV hand-off shared by the two decode kernels (attn_decode.hip,
// attn_decode_any.hip): the per-split records and their merge by the last key slice to finish
// (the log-sum-exp rule of attn_combine, shaders/kernels.metal:501-516).
//
// Protocol, per query head of a call with n_splits > 1:
//   1. Each key slice stores the head's record (o[HD], m, l) with device-scope (sc1,
//      write-through) stores and waits until memory has acknowledged them.
//   2. It then increments the head's counter (relaxed, device scope) and reads the old value.
//   3. The slice that read n_splits - 1 arrived last: every other record was acknowledged before
//      its counter increment, so it is in memory. The last slice loads all records with
//      device-scope loads (which do not return stale lines from its L1 or its XCD's L2), merges
//      them in split order (bitwise independent of which slice merges) and resets the counter.
// Nothing waits for another workgroup, so no dispatch order or residency is assumed, and nothing
// depends on which XCD a workgroup runs on: measured on this GPU, relaxed device-scope atomics
// on one counter from workgroups on all 8 XCDs return distinct values, and this store / wait /
// count / load hand-off sees every record wherever the last arriver runs. The counters start at
// zero (the workspace is zero-filled once) and every call leaves them at zero.
//
// Why not a release/acquire pair: an agent-scope acq_rel increment also writes back and
// invalidates the whole L2 around the atomic (measured: C3 decode 8.0 -> 17.9 us). The order is
// kept by hand: sc1 stores, a wait for their acknowledgement, the relaxed increment, sc1 loads.
// Compiler-only fences on both sides of the wait keep the optimizer from moving the stores or
// the atomic across it (the hardware order comes from the wait itself).
#pragma once

#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace handoff {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBufferFlags = 0x00020000;  // buffer descriptor word 3 (raw, 32-bit format)
constexpr int kScDevice = 16;             // buffer cache-policy bits: sc1 = device scope

__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    x = fmaxf(x, dpp<0x141>(x));
    x = fmaxf(x, dpp<0x140>(x));
    return x;
}
// With both operands equal to x, v_permlane16_swap yields {x_l, x_(l^16)} and
// v_permlane32_swap {x_l, x_(l^32)} (gfx950 lane-swap instructions).
__device__ __forceinline__ float add_x16(float x) {
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_x32(float x) {
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_x16(float x) {
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_x32(float x) {
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_max(float x) { return max_x32(max_x16(row16_max(x))); }
__device__ __forceinline__ float wave_sum(float x) { return add_x32(add_x16(row16_sum(x))); }

// Buffer descriptor of one query head's record region (split s at s * decode_record_bytes(HD):
// o[HD], then {m, l, 0, 0}).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_region(char* recs, uint32_t head) {
    return __builtin_amdgcn_make_buffer_rsrc(recs + size_t(head) * kDecodeHeadRecordBytes, 0,
                                             uint32_t(kDecodeHeadRecordBytes), kBufferFlags);
}

// 16 bytes of output at byte offset `off` of `row` with a write-through (sc1) store: the output
// then leaves no dirty line in the L2 for the end-of-dispatch write-back (measured: C3 decode
// 8.04 -> 7.92 us, 8192 keys 10.60 -> 10.46; a nontemporal store gained nothing).
// `bytes` (wave-uniform) is the row's size: the buffer descriptor covers the row.
__device__ __forceinline__ void store_out(float* row, int bytes, int off, float4v v) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(row, 0, bytes, kBufferFlags);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, off, 0, kScDevice);
}

// Steps 1 and 2 for one head, called by a whole wave: lane l holds dims 4c..4c+3 of o,
// c = l % (HD/4) (lanes with the same c hold the same values); (m, l) are wave-uniform. Returns
// the counter's old value (wave-uniform).
template <int HD>
__device__ __forceinline__ unsigned store_and_arrive(__amdgpu_buffer_rsrc_t rs, unsigned int* counter,
                                                     uint32_t split, float4v o, float m, float l, int lane) {
    constexpr int CPR = HD / 4;
    const int rec = int(split * decode_record_bytes(HD));
    // One store instruction per record where the wave has a lane left over: lanes 0..CPR-1 write
    // o and lane CPR the {m, l} chunk right after it. (Two stores under separate lane tests let
    // the compiler merge the (m, l) store into the atomic's branch below, which made the wave wait
    // for acknowledgements twice, once per side of the branch.)
    const u32x4 ml4 = u32x4{__float_as_uint(m), __float_as_uint(l), 0u, 0u};
    if constexpr (CPR < 64) {
        if (lane <= CPR)
            __builtin_amdgcn_raw_buffer_store_b128(lane < CPR ? __builtin_bit_cast(u32x4, o) : ml4, rs, rec + 16 * lane,
                                                   0, kScDevice);
    } else {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), rs, rec + 16 * lane, 0, kScDevice);
        __builtin_amdgcn_raw_buffer_store_b128(ml4, rs, rec + HD * 4, 0, kScDevice);  // same chunk from every lane
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // the record has reached device scope
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    unsigned prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_amdgcn_readfirstlane(prev);
}

// Step 3 for one head, called by a whole wave of the last arriver; `lds_w` is 64 floats of LDS
// private to the wave. Lane (sg, c) loads chunk c of the records of splits sg, sg + SG, ...
// (all loads in flight at once, from clamped split indices; splits past n_splits get weight 0),
// lane t loads (m, l) of split t. Writes out[0..HD) and leaves the counter at zero.
template <int HD, int MAXS>
__device__ __forceinline__ void merge_records(__amdgpu_buffer_rsrc_t rs, unsigned int* counter, uint32_t n_splits,
                                              int lane, float* lds_w, float* out) {
    constexpr int CPR = HD / 4;          // 16-byte o chunks per record
    constexpr int SG = 64 / CPR;         // split groups
    constexpr int NS = MAXS / SG;        // o loads per lane
    constexpr uint32_t rec = decode_record_bytes(HD);
    static_assert(CPR * SG == 64 && NS * SG == MAXS && MAXS <= 64, "merge lane layout");
    const int c = lane % CPR, sg = lane / CPR;

    float4v os[NS];
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const uint32_t sp = min(uint32_t(sg + SG * i), n_splits - 1);
        os[i] = __builtin_bit_cast(float4v,
                                   __builtin_amdgcn_raw_buffer_load_b128(rs, int(sp * rec) + 16 * c, 0, kScDevice));
    }
    const u32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(
        rs, int(min(uint32_t(lane), n_splits - 1) * rec) + HD * 4, 0, kScDevice);
    const bool have = uint32_t(lane) < n_splits;
    const float m_s = have ? __uint_as_float(ml[0]) : kNoMax;
    const float Mt = wave_max(m_s);
    const float w = fast_exp2(m_s - Mt);  // 0 for lanes past n_splits
    const float Lt = wave_sum(have ? w * __uint_as_float(ml[1]) : 0.f);
    lds_w[lane] = w;
    __builtin_amdgcn_wave_barrier();
    float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NS; i++) acc += os[i] * lds_w[sg + SG * i];
    // Sum over the split groups (lanes c + CPR*k) in a fixed order.
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float a = acc[e];
        if constexpr (SG >= 4) a = add_x16(a);
        if constexpr (SG >= 2) a = add_x32(a);
        acc[e] = a;
    }
    __builtin_amdgcn_wave_barrier();
    if (sg == 0) store_out(out, HD * 4, 16 * c, acc * (Lt > 0.f ? 1.f / Lt : 0.f));
    if (lane == 0)  // leave the workspace ready for the next call
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace handoff

}  // namespace ingot

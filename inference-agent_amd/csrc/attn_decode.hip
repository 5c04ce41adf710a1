// attn_decode.hip — split-KV (flash-decoding) GQA decode attention for gfx950: the tuned kernel
// for head_dim 128 and groups 1..4 (Llama-3.2-3B: group 3), and for larger groups that are
// multiples of 3 or 4 as n_sub units of 3 or 4 heads per KV head (group 8: 64/8 heads, KV 1024
// 8.50 -> 7.08 us, 4096 10.40 -> 10.11; each unit streams the KV head's slice, the second read
// served by the caches); attn_decode_any.hip serves the other
// shapes.
//
// Computes, for one query token and every Q head h, out_h = softmax(q_h K^T * scale) V over cache
// rows 0..n_keys-1 of KV head h / G — the attention block of src/cpu_backend.cpp:51-69 and the
// decode flash path of src/metal_backend.mm:339-359 (attn_decode_g3 + attn_combine,
// shaders/kernels.metal:428-516), re-designed for CDNA4.
//
// Grid: one dimension of n_splits * n_units workgroups (n_units = n_head_kv * n_sub), workgroup
// b serving unit b % n_units (query heads unit*G.., KV head unit / n_sub) and key slice
// b / n_units. The hardware hands workgroups to the 8 XCDs round robin (b % 8), so with 8 KV
// heads and one unit each every slice of one KV head runs on the same XCD. Each workgroup has NW wave64s; a wave step covers 16 keys and serves all
// G query heads of the group from each K/V row it reads:
//   - Scores on the matrix cores: S (16 rows x 16 keys) = A (16 x 256) * B (256 x 16) with
//     v_mfma_f32_16x16x32_f16 x 8. Rows 0..G-1 of A hold the G query heads; the 256-long
//     contraction is q_hi (128 dims) followed by q_lo (128 dims), where q*scale*log2(e) =
//     q_hi + q_lo with both parts f16, and B is the K tile repeated twice (same registers). The
//     score is thus exact to ~2^-22 relative although K and the MFMA inputs are f16; the
//     accumulation is f32. Lane l loads 4 x 16 bytes of key row l%16.
//   - Online softmax per head with a wave-uniform running max (base 2), 16-lane DPP max.
//   - P*V on the vector ALUs (v_fma_mix: f16 V, f32 P and accumulators). Lane l owns dims
//     8*(l%16)..+7 of key rows l/16 + 4u (u = 0..3); p reaches it through LDS.
//   - The K and V loads of the next step are issued before the current step is computed.
//
// The tail is latency, not bandwidth: after the last K/V row arrives, what is left is a chain of
// device-memory round trips, so it is cut per query head. Each wave publishes its four lane-group
// partials of o (no cross-lane reduction) and its (m, l) in LDS; after one barrier, wave h (h < G)
// alone merges head h of the workgroup, stores the head's record (o[128], m, l) with 16-byte
// device-scope stores, waits for them, and bumps the head's completion counter. The last slice to
// arrive for a head merges that head's n_splits records (decode_merge.h): lane (half, j) loads
// 16-byte chunk j of the records of splits half, half + 2, ...; lane t loads (m, l) of split t,
// the wave reduces the maximum, each lane computes its split's weight once, and the weights reach
// the chunk owners through LDS. The three heads of a group thus merge in parallel, in three
// different waves, with no workgroup barrier after the counter. The hand-off is correct whatever
// the workgroup placement (device-scope accesses throughout).
//
// MFMA 16x16x32 f16 register layouts (wave64, lane l, i = l%16, g = l/16):
//   A (16 x 32): lane holds A[i][8g + e], e = 0..7;  B (32 x 16): lane holds B[8g + e][i];
//   D (16 x 16): lane holds D[4g + j][i], j = 0..3.
//
// Record layout (workspace, after the counters): one region of kDecodeHeadRecordBytes per query
// head, [split][528 bytes]: o[128] (unnormalized, relative to m), then m (base 2) and l — the
// reference's part[...][130] record (AD_STRIDE, shaders/kernels.metal:291).
#include <type_traits>

#include "attn_common.h"
#include "attn_internal.h"
#include "decode_merge.h"

namespace ingot {

namespace {

using handoff::max_x16;
using handoff::max_x32;
using handoff::row16_max;

__device__ __forceinline__ float lane0(float x) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
}

template <int G, int NW, bool ROT, bool SUB>
__global__ __launch_bounds__(64 * NW) void attn_decode_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ K, const _Float16* __restrict__ V,
    float* __restrict__ out, char* __restrict__ recs, unsigned int* __restrict__ counters,
    uint32_t n_keys, uint32_t keys_per_split, uint32_t n_splits, uint32_t n_units, uint32_t n_sub,
    float qscale) {
    static_assert(G <= NW, "one tail wave per query head of the group");
    static_assert(kMaxDecodeSplits <= 64, "one lane per split in the merge");
    constexpr int KW = 16;  // keys per wave step
    __shared__ __attribute__((aligned(16))) float lds_o[NW][4][G][kHeadDim];  // per lane group r
    __shared__ float lds_ml[NW][G][2];
    __shared__ __attribute__((aligned(16))) float lds_p[NW][KW][4];  // p[key][head] per wave
    __shared__ float lds_w[G][64];                                   // split weights per head

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane >> 4, c = lane & 15;
    // unit = query heads unit*G .. unit*G+G-1 of KV head unit / n_sub (n_sub units share a KV
    // head when the group is larger than G)
    const uint32_t unit = blockIdx.x % n_units, split = blockIdx.x / n_units, kvh = SUB ? unit / n_sub : unit;
    const size_t kv_dim = size_t(n_units / n_sub) * kHeadDim;
    const uint32_t k0 = split * keys_per_split;
    const uint32_t k1 = min(n_keys, k0 + keys_per_split);

    // K: lane reads key row (base + c), 16 bytes at dims 32m + 8r. V: key rows base + 4u + r,
    // 16 bytes at dims 8c. Loads are unconditional: rows past the slice are clamped to its last
    // row (already in cache), so the number of loads in flight is the same on every path and
    // the compiler's wait counts never stall the current step on the prefetch of the next.
    const _Float16* Kb = K + size_t(kvh) * kHeadDim + 8 * r;
    const _Float16* Vb = V + size_t(kvh) * kHeadDim + 8 * c;
    auto load_step = [&](uint32_t b, half8 (&kx)[4], half8 (&vx)[4]) {
        const uint32_t kk = min(b + c, k1 - 1);
#pragma unroll
        for (int m = 0; m < 4; m++) kx[m] = load_half8(Kb + size_t(kk) * kv_dim + 32 * m);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t kv = min(b + 4 * u + r, k1 - 1);
            vx[u] = load_half8(Vb + size_t(kv) * kv_dim);
        }
    };

    // A operand: lane holds A[row c][k = 8r + e] of MFMA m (m < 4: q_hi of dims 32m+8r+e,
    // m >= 4: q_lo of the same dims). Rows >= G are zero.
    half8 qa[8];
    {
        const bool live = c < G;
        const float* qrow = q + (size_t(unit) * G + (live ? c : 0)) * kHeadDim;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const float4v* src = reinterpret_cast<const float4v*>(qrow + 32 * m + 8 * r);
            const float4v a = src[0], b = src[1];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = (e < 4 ? a[e] : b[e - 4]) * qscale;
                const _Float16 hi = _Float16(x);
                const _Float16 lo = _Float16(x - float(hi));
                qa[m][e] = live ? hi : _Float16(0.f);
                qa[4 + m][e] = live ? lo : _Float16(0.f);
            }
        }
    }

    float o[G][8], m_run[G], l_run[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m_run[h] = kNoMax;
        l_run[h] = 0.f;  // lane-local partial sum (lanes 0..15 only)
#pragma unroll
        for (int i = 0; i < 8; i++) o[h][i] = 0.f;
    }

    auto compute_step = [&](uint32_t b, const half8 (&kx)[4], const half8 (&vx)[4]) {
        // S[row][key]: lane holds rows 4r..4r+3 of key c; rows 0..G-1 (lanes 0..15) are real.
        float4v S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 8; m++) S = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[m], kx[m & 3], S, 0, 0, 0);
        const bool valid = b + c < k1;
        float alpha[G];
        float4v pp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float s = valid ? S[h] : -__builtin_inff();
            const float m_new = fmaxf(m_run[h], lane0(row16_max(s)));  // wave-uniform
            alpha[h] = fast_exp2(m_run[h] - m_new);
            m_run[h] = m_new;
            const float p = fast_exp2(s - m_new);
            l_run[h] = l_run[h] * alpha[h] + p;
            pp[h] = p;
        }
        if (r == 0) *reinterpret_cast<float4v*>(&lds_p[wave][c][0]) = pp;
        __builtin_amdgcn_wave_barrier();
        float4v pv[4];
#pragma unroll
        for (int u = 0; u < 4; u++) pv[u] = *reinterpret_cast<const float4v*>(&lds_p[wave][4 * u + r][0]);
#pragma unroll
        for (int h = 0; h < G; h++) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float acc = o[h][i] * alpha[h];
#pragma unroll
                for (int u = 0; u < 4; u++) acc = __builtin_fmaf(pv[u][h], float(vx[u][i]), acc);
                o[h][i] = acc;
            }
        }
        __builtin_amdgcn_wave_barrier();
    };

    // Two register buffers alternate (ping-pong), so a prefetch never waits for the step it
    // follows. ROT: the slice's nst workgroup steps (kStride keys each) are walked starting at
    // step split % nst and wrapping: the slices lie a power-of-two distance apart in the cache
    // (e.g. 256 keys = 512 KB at 8192 keys and 32 splits), and walked in lockstep from their
    // starts their concurrent loads pile onto the same memory channels (a load-only probe of
    // this grid at 8192 keys: 8.54 us in order, 7.39 us rotated). Steps whose keys all lie past
    // k1 (a wave's part of a short last step) are masked in compute_step, as the partial ones
    // are. The host launches the in-order walk for slices of fewer than three steps (C3: two),
    // where rotation gains nothing and its index arithmetic measured ~0.1 us slower.
    constexpr uint32_t kStride = NW * KW;
    const uint32_t nst = (k1 - k0 + kStride - 1) / kStride;
    half8 ka[4], va[4], kb[4], vb[4];
    if constexpr (ROT) {
        const uint32_t rot = split % nst;
        auto at = [&](uint32_t j) {  // first key of this wave in walk step j (clamped to the last)
            uint32_t p = min(j, nst - 1) + rot;
            p = p >= nst ? p - nst : p;
            return k0 + p * kStride + wave * KW;
        };
        load_step(at(0), ka, va);
        for (uint32_t j = 0; j < nst; j += 2) {
            load_step(at(j + 1), kb, vb);
            __builtin_amdgcn_sched_barrier(0);  // issue the prefetch before any of this step's math
            compute_step(at(j), ka, va);
            if (j + 1 >= nst) break;
            load_step(at(j + 2), ka, va);
            __builtin_amdgcn_sched_barrier(0);
            compute_step(at(j + 1), kb, vb);
        }
    } else {  // in order
        uint32_t base = k0 + wave * KW;
        load_step(base, ka, va);
        while (base < k1) {
            load_step(base + kStride, kb, vb);
            __builtin_amdgcn_sched_barrier(0);
            compute_step(base, ka, va);
            base += kStride;
            if (base >= k1) break;
            load_step(base + kStride, ka, va);
            __builtin_amdgcn_sched_barrier(0);
            compute_step(base, kb, vb);
            base += kStride;
        }
    }

    // Publish the wave's partials: lane group r holds dims 8c..8c+7 of its key rows; all four
    // groups share the wave-uniform m, so the reader sums them without weights.
#pragma unroll
    for (int h = 0; h < G; h++) {
        float* dst = &lds_o[wave][r][h][8 * c];
        *reinterpret_cast<float4v*>(dst) = float4v{o[h][0], o[h][1], o[h][2], o[h][3]};
        *reinterpret_cast<float4v*>(dst + 4) = float4v{o[h][4], o[h][5], o[h][6], o[h][7]};
        const float l = row16_sum(r == 0 ? l_run[h] : 0.f);
        if (lane == 0) {
            lds_ml[wave][h][0] = m_run[h];
            lds_ml[wave][h][1] = l;
        }
    }
    __syncthreads();
    if (wave >= G) return;

    // Wave h merges head h of this workgroup; lane j < 32 owns dims 4j..4j+3.
    const int h = wave, j = lane & 31;
    float M = kNoMax;
#pragma unroll
    for (int w = 0; w < NW; w++) M = fmaxf(M, lds_ml[w][h][0]);
    float L = 0.f;
    float4v O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; w++) {
        const float wt = fast_exp2(lds_ml[w][h][0] - M);
        L += lds_ml[w][h][1] * wt;
        float4v s4 = *reinterpret_cast<const float4v*>(&lds_o[w][0][h][4 * j]);
#pragma unroll
        for (int g = 1; g < 4; g++) s4 += *reinterpret_cast<const float4v*>(&lds_o[w][g][h][4 * j]);
        O += s4 * wt;
    }
    const size_t head = size_t(unit) * G + h;
    if (n_splits == 1) {
        if (lane < 32) handoff::store_out(out + head * kHeadDim, kHeadDim * 4, 16 * j, O * (L > 0.f ? 1.f / L : 0.f));
        return;
    }

    // The split hand-off (decode_merge.h): store this head's record, count it in, and the last
    // slice to arrive merges the head's records.
    const __amdgpu_buffer_rsrc_t rs = handoff::head_region(recs, uint32_t(head));
    unsigned int* counter = counters + head * kCounterStride;
    if (handoff::store_and_arrive<kHeadDim>(rs, counter, split, O, M, L, lane) != n_splits - 1) return;
    handoff::merge_records<kHeadDim, int(kMaxDecodeSplits)>(rs, counter, n_splits, lane, lds_w[h],
                                                           out + head * kHeadDim);
}

template <int G, int NW>
void launch_g(uint32_t n_blocks, hipStream_t stream, const float* q, const _Float16* k,
              const _Float16* v, float* out, char* recs, unsigned int* counters, uint32_t n_keys,
              uint32_t per, uint32_t n_splits, uint32_t n_units, uint32_t n_sub, float qscale) {
    // (SUB: several units per KV head, which costs the one-split-per-head case an integer
    // division before its first loads; instantiated for the unit sizes that large groups use)
    auto go = [&](auto rot, auto sub) {
        hipLaunchKernelGGL((attn_decode_kernel<G, NW, decltype(rot)::value, decltype(sub)::value>), dim3(n_blocks),
                           dim3(64 * NW), 0, stream, q, k, v, out, recs, counters, n_keys, per, n_splits, n_units,
                           n_sub, qscale);
    };
    const bool rot = n_splits > 1 && (per + 16 * NW - 1) / (16 * NW) >= 3;  // several slices of 3+ steps
    using T = std::true_type;
    using F = std::false_type;
    if constexpr (G >= 3) {
        if (n_sub > 1) {
            if (rot) go(T{}, T{});
            else go(F{}, T{});
            return;
        }
    }
    if (rot) go(T{}, F{});
    else go(F{}, F{});
}

constexpr int kNW = 4;

}  // namespace

int launch_decode_g128(const float* q, const _Float16* k, const _Float16* v, float* out, char* recs,
                       unsigned int* counters, uint32_t n_keys, uint32_t n_splits, uint32_t n_head_kv,
                       uint32_t group, float scale, hipStream_t stream) {
    const uint32_t per = (n_keys + n_splits - 1) / n_splits;
    // Groups above 4 run as units of gs heads (the largest divisor of the group up to 4), n_sub
    // units per KV head, each streaming that KV head's slice.
    uint32_t gs = group;
    if (group > 4) {
        gs = 1;
        for (uint32_t g = 4; g > 1; g--)
            if (group % g == 0) { gs = g; break; }
    }
    const uint32_t n_sub = group / gs, n_units = n_head_kv * n_sub;
    const uint32_t blocks = n_splits * n_units;
    const float qscale = scale * kLog2e;
    switch (gs) {
        case 1: launch_g<1, kNW>(blocks, stream, q, k, v, out, recs, counters, n_keys, per, n_splits, n_units, n_sub, qscale); break;
        case 2: launch_g<2, kNW>(blocks, stream, q, k, v, out, recs, counters, n_keys, per, n_splits, n_units, n_sub, qscale); break;
        case 3: launch_g<3, kNW>(blocks, stream, q, k, v, out, recs, counters, n_keys, per, n_splits, n_units, n_sub, qscale); break;
        case 4: launch_g<4, kNW>(blocks, stream, q, k, v, out, recs, counters, n_keys, per, n_splits, n_units, n_sub, qscale); break;
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace ingot

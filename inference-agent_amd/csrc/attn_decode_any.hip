// attn_decode_any.hip — split-KV GQA decode attention for any head_dim in {64, 128, 256} and any
// group size (gfx950); attn_decode.hip holds the tuned kernel for head_dim 128 and groups 1..4
// (and multiples of 3 or 4).
//
// Computes, for one query token and every Q head h, out_h = softmax(q_h K^T * scale) V over cache
// rows 0..n_keys-1 of KV head h / group — the attention block of src/cpu_backend.cpp:51-69 and
// the decode flash path of src/metal_backend.mm:339-359 (attn_decode_g3 + attn_combine,
// shaders/kernels.metal:428-516), re-designed for CDNA4. Head dimension HD is 64, 128 or 256;
// a workgroup serves G query heads of one KV head (a "unit"); groups larger than the
// instantiated G are served by several units per KV head (each streams the KV head once).
//
// Grid: one dimension of n_splits * n_units workgroups: workgroup b serves unit b % n_units and
// key slice b / n_units.
//
// Key walkers (4 wave64s; a wave step covers 16 keys and serves all G query heads from each K/V
// row it reads):
//   - Scores on the matrix cores: S (16 rows x 16 keys) = A (16 x 2HD) * B (2HD x 16) with
//     v_mfma_f32_16x16x32_f16. Row r of A is query head r (rows >= G are zero); the contraction
//     is q_hi (HD dims) followed by q_lo (HD dims), where q*scale*log2(e) = q_hi + q_lo with both
//     parts f16, and B is the K tile repeated twice (same registers). The score is exact to
//     ~2^-22 relative although K and the MFMA inputs are f16; the accumulation is f32.
//   - Online softmax per head with a wave-uniform running max (base 2), 16-lane DPP max.
//   - P*V on the vector ALUs (v_fma_mix: f16 V, f32 P and accumulators). p reaches the V lanes
//     through LDS.
//   - K/V come through buffer loads whose descriptors cover exactly the slice (rows past its end
//     read as zero and are masked), two register buffers alternating: the next step's loads are
//     in flight while a step is computed.
//   - The 4 waves merge through LDS; with one slice wave h writes head h's output. With several,
//     wave w handles heads w, w + 4 of the unit: it stores the head's record, waits for it to
//     reach device scope and counts it in on the head's counter; the slice that arrives last
//     merges the head's records (decode_merge.h). Nothing waits for another workgroup, and
//     nothing depends on which XCD a workgroup runs on or on the order of dispatch.
//
// MFMA 16x16x32 f16 register layouts (wave64, lane l, i = l%16, g = l/16):
//   A (16 x 32): lane holds A[i][8g + e], e = 0..7;  B (32 x 16): lane holds B[8g + e][i];
//   D (16 x 16): lane holds D[4g + j][i], j = 0..3.
//
// Workspace: the first kCounterBytes hold one counter per query head (kCounterStride words apart);
// then one region of kDecodeHeadRecordBytes per query head holding the records
// [split][HD*4 + 16 B]: o[HD], then {m, l} — the reference's part[...][130] record (o, m, l;
// AD_STRIDE at shaders/kernels.metal:291).
#include "attn_common.h"
#include "attn_internal.h"
#include "decode_merge.h"

namespace ingot {

namespace {

constexpr int kBufferFlags = 0x00020000;  // buffer descriptor word 3 (raw, 32-bit format)
constexpr int kNW = 4;                    // waves per workgroup
constexpr int kKW = 16;                   // keys per wave step

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

using handoff::row16_max;

__device__ __forceinline__ float readlane_f(float x, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

template <int HD, int G>
__global__ __launch_bounds__(64 * kNW) void attn_decode_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ K, const _Float16* __restrict__ V,
    float* __restrict__ out, char* __restrict__ recs, unsigned int* __restrict__ counters, uint32_t n_keys,
    uint32_t keys_per_split, uint32_t n_splits, uint32_t n_units, uint32_t n_sub, uint32_t kv_dim,
    uint32_t group, float qscale) {
    static_assert(HD == 64 || HD == 128 || HD == 256, "head_dim 64, 128 or 256");
    static_assert(G >= 1 && G <= 8, "up to 8 query heads per unit (two MFMA row groups)");
    constexpr int NKC = HD / 32;          // K loads (16 B) per lane per step
    constexpr int CPR = HD / 8;           // 16-byte chunks per K/V row
    constexpr int KPL = 64 / CPR;         // keys per V load instruction
    constexpr int NV = kKW / KPL;         // V loads per lane per step
    constexpr int GQ = (G + 3) / 4;       // MFMA row groups holding real heads
    constexpr int GP = 4 * GQ;
    constexpr int OL = HD / 4;            // lanes owning 4 output dims after the workgroup merge

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    __shared__ __attribute__((aligned(16))) float lds_o[kNW][KPL][G][HD];
    __shared__ float lds_ml[kNW][G][2];
    __shared__ __attribute__((aligned(16))) float lds_p[kNW][kKW][GP];
    __shared__ float lds_w[kNW][64];  // split weights of the head a wave merges

    const int ki = lane & 15, kg = lane >> 4;         // MFMA lane coordinates
    const int vc = lane % CPR, vr = lane / CPR;       // V chunk and key sub-row of the lane
    const uint32_t unit = blockIdx.x % n_units, split = blockIdx.x / n_units;
    const uint32_t kvh = unit / n_sub, sub = unit % n_sub;
    const uint32_t head0 = kvh * group + sub * G;     // first query head of the unit
    const uint32_t k0 = split * keys_per_split;
    const uint32_t k1 = min(n_keys, k0 + keys_per_split);
    const bool multi = n_splits > 1;

    // A operand: lane holds A[row ki][k = 8 kg + e] of MFMA m (m < NKC: q_hi of dims
    // 32m + 8kg + e, m >= NKC: q_lo of the same dims). Rows >= G are zero. q is loaded first.
    float4v qf[2 * NKC];
    const bool live = ki < G;
    {
        const float* qrow = q + size_t(head0 + (live ? ki : 0)) * HD;
#pragma unroll
        for (int m = 0; m < NKC; m++) {
            const float4v* src = reinterpret_cast<const float4v*>(qrow + 32 * m + 8 * kg);
            qf[2 * m] = src[0];
            qf[2 * m + 1] = src[1];
        }
    }

    // K/V buffer descriptors covering exactly this split's rows of the KV head (the last row ends
    // at its head's last byte): a row past k1 is out of range and reads as zero (its score is
    // masked below). Offsets are 32-bit, one add per load group.
    const uint32_t row_bytes = kv_dim * 2;
    const uint32_t span = (k1 - k0 - 1) * row_bytes + HD * 2;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(K + size_t(k0) * kv_dim + size_t(kvh) * HD), 0, span, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(V + size_t(k0) * kv_dim + size_t(kvh) * HD), 0, span, kBufferFlags);
    const uint32_t k_lane = ki * row_bytes + 16 * kg;   // key row ki, dims 8kg (+32m)
    const uint32_t v_lane = vr * row_bytes + 16 * vc;   // key row vr, dims 8vc
    // The register buffers hold raw dwords (u32x4); they become f16 vectors only where they are
    // used, so the loop-carried buffers are plain 32-bit registers that the allocator keeps in
    // place (as f16 vectors they were copied element-wise at the back edge, which waited for the
    // loads in flight).
    auto load_step = [&](uint32_t b, u32x4 (&kx)[NKC], u32x4 (&vx)[NV]) {
        const uint32_t step = (b - k0) * row_bytes;
        const int ko = int(k_lane + step);
#pragma unroll
        for (int m = 0; m < NKC; m++) kx[m] = __builtin_amdgcn_raw_buffer_load_b128(krs, ko + 64 * m, 0, 0);
#pragma unroll
        for (int u = 0; u < NV; u++)
            vx[u] = __builtin_amdgcn_raw_buffer_load_b128(vrs, int(v_lane + step + u * KPL * row_bytes), 0, 0);
    };
    constexpr uint32_t kStride = kNW * kKW;
    uint32_t base = k0 + wave * kKW;
    u32x4 ka[NKC], va[NV], kb[NKC], vb[NV];
    load_step(base, ka, va);

    half8 qa[2 * NKC];
#pragma unroll
    for (int m = 0; m < NKC; m++) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float x = qf[2 * m + e / 4][e % 4] * qscale;
            const _Float16 hi = _Float16(x);
            const _Float16 lo = _Float16(x - float(hi));
            qa[m][e] = live ? hi : _Float16(0.f);
            qa[NKC + m][e] = live ? lo : _Float16(0.f);
        }
    }

    float o[G][8], m_run[G], l_lane[4];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m_run[h] = kNoMax;
#pragma unroll
        for (int i = 0; i < 8; i++) o[h][i] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; j++) l_lane[j] = 0.f;  // head 4*kg + j of this lane's row group

    auto compute_step = [&](uint32_t b, const u32x4 (&kx)[NKC], const u32x4 (&vx)[NV]) {
        // S[row][key]: lane holds rows 4kg..4kg+3 of key ki.
        float4v S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 2 * NKC; m++)
            S = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[m], __builtin_bit_cast(half8, kx[m % NKC]), S, 0, 0, 0);
        const bool valid = b + ki < k1;
        float rm[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            S[j] = valid ? S[j] : -__builtin_inff();
            rm[j] = row16_max(S[j]);
        }
        float alpha[G];
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float m_new = fmaxf(m_run[h], readlane_f(rm[h & 3], 16 * (h >> 2)));  // uniform
            alpha[h] = fast_exp2(m_run[h] - m_new);
            m_run[h] = m_new;
        }
        float4v pp;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // this lane's row group kg holds head 4kg + j
            float mh = m_run[j < G ? j : 0], ah = alpha[j < G ? j : 0];
            if constexpr (GQ > 1) {
                if (kg == 1 && 4 + j < G) { mh = m_run[4 + j]; ah = alpha[4 + j]; }
            }
            const float p = fast_exp2(S[j] - mh);
            l_lane[j] = l_lane[j] * ah + p;
            pp[j] = p;
        }
        if (kg < GQ) *reinterpret_cast<float4v*>(&lds_p[wave][ki][4 * kg]) = pp;
        __builtin_amdgcn_wave_barrier();
        float4v pv[NV][GQ];
#pragma unroll
        for (int u = 0; u < NV; u++)
#pragma unroll
            for (int t = 0; t < GQ; t++)
                pv[u][t] = *reinterpret_cast<const float4v*>(&lds_p[wave][vr + KPL * u][4 * t]);
#pragma unroll
        for (int h = 0; h < G; h++) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float acc = o[h][i] * alpha[h];
#pragma unroll
                for (int u = 0; u < NV; u++)
                    acc = __builtin_fmaf(pv[u][h >> 2][h & 3], float(__builtin_bit_cast(half8, vx[u])[i]), acc);
                o[h][i] = acc;
            }
        }
        __builtin_amdgcn_wave_barrier();
    };

    // Two register buffers alternate (ping-pong): the next step's loads are in flight while a
    // step is computed.
    while (base < k1) {
        load_step(base + kStride, kb, vb);
        __builtin_amdgcn_sched_barrier(0);  // issue the prefetch before any of this step's math
        compute_step(base, ka, va);
        base += kStride;
        if (base >= k1) break;
        load_step(base + kStride, ka, va);
        __builtin_amdgcn_sched_barrier(0);
        compute_step(base, kb, vb);
        base += kStride;
    }

    // Publish the wave's partials: lane (vc, vr) holds dims 8vc..8vc+7 over its key sub-rows; all
    // share the wave-uniform m, so the reader sums the sub-rows without weights.
#pragma unroll
    for (int h = 0; h < G; h++) {
        float* dst = &lds_o[wave][vr][h][8 * vc];
        *reinterpret_cast<float4v*>(dst) = float4v{o[h][0], o[h][1], o[h][2], o[h][3]};
        *reinterpret_cast<float4v*>(dst + 4) = float4v{o[h][4], o[h][5], o[h][6], o[h][7]};
        const float l = readlane_f(row16_sum(l_lane[h & 3]), 16 * (h >> 2));
        if (lane == 0) {
            lds_ml[wave][h][0] = m_run[h];
            lds_ml[wave][h][1] = l;
        }
    }
    __syncthreads();

    for (int h = wave; h < G; h += kNW) {
        // Merge the workgroup's waves for head h; lane l owns dims 4c..4c+3, c = l % OL (the lane
        // layout of the hand-off; lanes with the same c compute the same values).
        const int d0 = 4 * (lane % OL);
        float M = kNoMax;
#pragma unroll
        for (int w = 0; w < kNW; w++) M = fmaxf(M, lds_ml[w][h][0]);
        float L = 0.f;
        float4v O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < kNW; w++) {
            const float wt = fast_exp2(lds_ml[w][h][0] - M);
            L += lds_ml[w][h][1] * wt;
            float4v s4 = *reinterpret_cast<const float4v*>(&lds_o[w][0][h][d0]);
#pragma unroll
            for (int r = 1; r < KPL; r++) s4 += *reinterpret_cast<const float4v*>(&lds_o[w][r][h][d0]);
            O += s4 * wt;
        }
        const uint32_t head = head0 + h;
        float* dst = out + size_t(head) * HD;
        if (!multi) {
            if (lane < OL) handoff::store_out(dst, HD * 4, 4 * d0, O * (L > 0.f ? 1.f / L : 0.f));
            continue;
        }
        // The split hand-off (decode_merge.h): store this head's record, count it in, and the
        // last slice to arrive merges the head's records.
        const __amdgpu_buffer_rsrc_t rs = handoff::head_region(recs, head);
        unsigned int* counter = counters + head * kCounterStride;
        if (handoff::store_and_arrive<HD>(rs, counter, split, O, M, L, lane) != n_splits - 1) continue;
        constexpr int MAXS = HD > 128 ? int(kMaxDecodeSplits) / 2 : int(kMaxDecodeSplits);
        handoff::merge_records<HD, MAXS>(rs, counter, n_splits, lane, lds_w[wave], dst);
    }
}

template <int HD, int G>
void launch_g(uint32_t n_blocks, hipStream_t stream, const float* q, const _Float16* k,
              const _Float16* v, float* out, char* recs, unsigned int* counters, uint32_t n_keys,
              uint32_t per, uint32_t n_splits, uint32_t n_units, uint32_t n_sub,
              uint32_t kv_dim, uint32_t group, float qscale) {
    hipLaunchKernelGGL((attn_decode_kernel<HD, G>), dim3(n_blocks), dim3(64 * kNW), 0, stream, q, k, v,
                       out, recs, counters, n_keys, per, n_splits, n_units, n_sub, kv_dim, group,
                       qscale);
}

template <int HD>
int launch_hd(uint32_t gs, uint32_t n_blocks, hipStream_t stream, const float* q, const _Float16* k,
              const _Float16* v, float* out, char* recs, unsigned int* counters, uint32_t n_keys,
              uint32_t per, uint32_t n_splits, uint32_t n_units, uint32_t n_sub,
              uint32_t kv_dim, uint32_t group, float qscale) {
#define INGOT_DECODE_G(GG)                                                                         \
    case GG:                                                                                       \
        launch_g<HD, GG>(n_blocks, stream, q, k, v, out, recs, counters, n_keys, per,                       \
                         n_splits, n_units, n_sub, kv_dim, group, qscale);                        \
        return 0;
    switch (gs) {
        INGOT_DECODE_G(1)
        INGOT_DECODE_G(2)
        INGOT_DECODE_G(3)
        INGOT_DECODE_G(4)
        INGOT_DECODE_G(5)
        INGOT_DECODE_G(6)
        INGOT_DECODE_G(7)
        INGOT_DECODE_G(8)
        default: return -2;
    }
#undef INGOT_DECODE_G
}

constexpr uint32_t kMinKeysPerSplit = 32;  // two wave steps: the tail costs more than the loads
constexpr uint32_t kOneSplitKeys = 192;
constexpr uint32_t kMinSplits = 16;  // for caches above kOneSplitKeys

}  // namespace

uint32_t decode_unit_heads(uint32_t group) {
    // Largest divisor of the group that one workgroup serves (at most 8 heads: two MFMA row
    // groups); the rest of the group is covered by further units over the same KV head.
    for (uint32_t g = group < 8 ? group : 8; g > 1; g--)
        if (group % g == 0) return g;
    return 1;
}

uint32_t decode_max_splits(uint32_t head_dim) {
    // A merging wave loads one 16-byte chunk per lane and split group; head_dim 256 records are
    // twice as long.
    return head_dim > 128 ? kMaxDecodeSplits / 2 : kMaxDecodeSplits;
}

uint32_t decode_splits(uint32_t n_keys, uint32_t head_dim, uint32_t requested) {
    uint32_t splits = requested;
    // Short caches take one workgroup per unit: below ~192 keys the split records and merge cost
    // more than the parallel key walk saves. Above that at least 16 splits (measured, head_dim
    // 128, 24/8 heads: 256 keys 4.77 us at 8 splits, 4.66 at 16; 384 keys 5.12 at 12, 5.13 at
    // 16), then one per 32 keys.
    if (splits == 0)
        splits = n_keys <= kOneSplitKeys ? 1 : max(kMinSplits, (n_keys + kMinKeysPerSplit - 1) / kMinKeysPerSplit);
    splits = max(1u, min(splits, min(n_keys, decode_max_splits(head_dim))));
    // No empty splits: recompute from the per-split key count.
    const uint32_t per = (n_keys + splits - 1) / splits;
    return (n_keys + per - 1) / per;
}

namespace {

}  // namespace

int launch_decode_any(const float* q, const _Float16* k, const _Float16* v, float* out, void* recs,
                      unsigned int* counters,
                      uint32_t n_keys, uint32_t n_splits, uint32_t n_head_kv, uint32_t group,
                      uint32_t head_dim, float scale, hipStream_t stream) {
    const uint32_t per = (n_keys + n_splits - 1) / n_splits;
    const uint32_t gs = decode_unit_heads(group);
    const uint32_t n_sub = group / gs, n_units = n_head_kv * n_sub;
    const uint64_t blocks = uint64_t(n_splits) * n_units;
    if (blocks > 0x7fffffffu) return -1;
    const uint32_t kv_dim = n_head_kv * head_dim;
    const float qscale = scale * kLog2e;
    char* r = static_cast<char*>(recs);
    const uint32_t nb = uint32_t(blocks);
    int rc;
    switch (head_dim) {
        case 64: rc = launch_hd<64>(gs, nb, stream, q, k, v, out, r, counters, n_keys, per, n_splits, n_units, n_sub, kv_dim, group, qscale); break;
        case 128: rc = launch_hd<128>(gs, nb, stream, q, k, v, out, r, counters, n_keys, per, n_splits, n_units, n_sub, kv_dim, group, qscale); break;
        case 256: rc = launch_hd<256>(gs, nb, stream, q, k, v, out, r, counters, n_keys, per, n_splits, n_units, n_sub, kv_dim, group, qscale); break;
        default: return -2;
    }
    if (rc) return rc;
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_decode(const float* q, const _Float16* k, const _Float16* v, float* out, void* workspace,
                  uint32_t n_keys, uint32_t n_splits, uint32_t n_head_kv, uint32_t group,
                  uint32_t head_dim, float scale, hipStream_t stream) {
    char* ws = static_cast<char*>(workspace);
    if (head_dim == 128 && (group <= 4 || group % 4 == 0 || group % 3 == 0))
        return launch_decode_g128(q, k, v, out, ws + kCounterBytes,
                                  reinterpret_cast<unsigned int*>(ws), n_keys, n_splits, n_head_kv, group,
                                  scale, stream);
    return launch_decode_any(q, k, v, out, ws + kCounterBytes, reinterpret_cast<unsigned int*>(ws), n_keys, n_splits, n_head_kv, group, head_dim,
                             scale, stream);
}

}  // namespace ingot

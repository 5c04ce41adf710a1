// attn_prefill.hip — causal tiled (flash) prefill attention on f16 MFMA for gfx950.
//
// For a chunk of n_tok queries at absolute positions pos..pos+n_tok-1, query i of head h
// attends to cache rows 0..pos+i of KV head h / G: the semantics of n_tok successive decode
// steps (src/backend.h:16-20, src/cpu_backend.cpp:51-69) and of the reference's attn_prefill
// (shaders/kernels.metal:518-633, mask `key <= pos+tok`, line 578), re-designed for CDNA4:
//
//   - One workgroup = G waves (one per query head of a GQA group) x NQB query blocks of 32.
//     Every K/V tile (64 keys) is staged once in LDS and read by all G heads' waves.
//   - Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_f16 (A = K rows from LDS,
//     B = Q^T held in registers), so a lane owns one query column: the row max and row sum of
//     the online softmax are lane-local plus one exchange with lane^32.
//   - O^T += V^T P^T with the same MFMA. P^T comes straight out of the S^T accumulator layout
//     (no shuffle); V is stored transposed in LDS with the key order permuted to match, so the
//     A operand is one 16-byte LDS read.
//   - Q is pre-scaled by scale*log2(e) and rounded to f16 (the reference rounds Q*scale to
//     half, shaders/kernels.metal:543); P is rounded to f16 for the PV product (line 588);
//     S, O, m and l stay f32.
//   - Causal tile skipping: a wave stops at the last key its last query may see; tiles that
//     straddle the diagonal are masked per element.
//   - Split-KV: with n_splits > 1 each workgroup covers a slice of its key tiles and writes
//     (o, m, l) partials; attn_prefill_combine merges them (log-sum-exp rule of attn_combine,
//     shaders/kernels.metal:501-516).
//
// MFMA 32x32x16 f16 register layouts (wave64, lane l, i = l%32, hb = l/32):
//   A (32 x 16): lane holds A[i][8*hb + e], e = 0..7
//   B (16 x 32): lane holds B[8*hb + e][i]
//   D (32 x 32): lane holds D[8*(r/4) + 4*hb + r%4][i], r = 0..15
#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace {

constexpr int kBN = 64;            // keys per tile
constexpr int kKS = kHeadDim + 8;  // LDS row stride of K (halves): 272 B
constexpr int kVS = kBN + 8;       // LDS row stride of V^T (halves): 144 B

// Position of key j (0..15 inside a 16-key group) in a V^T row: swap bits 2 and 3, so that the
// 8 keys a lane feeds to one PV MFMA ({0-3, 8-11} or {4-7, 12-15}) are contiguous.
__device__ __forceinline__ int vt_pos(int j) {
    return (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1);
}

__device__ __forceinline__ uint32_t pack_halves(_Float16 lo, _Float16 hi) {
    const uint32_t a = __builtin_bit_cast(uint16_t, lo), b = __builtin_bit_cast(uint16_t, hi);
    return a | (b << 16);
}

template <int G, int NQB>
__global__ __launch_bounds__(64 * G * NQB) void attn_prefill_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ K, const _Float16* __restrict__ V,
    float* __restrict__ out, float* __restrict__ part, uint32_t pos, uint32_t n_tok,
    uint32_t q_stride, uint32_t n_head_kv, uint32_t n_splits, float qscale) {
    constexpr int NT = 64 * G * NQB;
    __shared__ __attribute__((aligned(16))) _Float16 Ks[kBN * kKS];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[kHeadDim * kVS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hh = wave % G, qsb = wave / G;
    const int li = lane & 31, hb = lane >> 5;
    const uint32_t kvh = blockIdx.y, split = blockIdx.z;
    const uint32_t h = kvh * G + hh;
    const size_t kv_dim = size_t(n_head_kv) * kHeadDim;
    const uint32_t qblk0 = blockIdx.x * 32 * NQB;
    const uint32_t q0 = qblk0 + qsb * 32;

    // Keys [0, kend) are visible to some query of this workgroup.
    const uint32_t qlast_wg = min(n_tok, qblk0 + 32 * NQB) - 1;
    const uint32_t kend = pos + qlast_wg + 1;
    const uint32_t ntiles = (kend + kBN - 1) / kBN;
    const uint32_t t_begin = uint32_t((uint64_t(split) * ntiles) / n_splits);
    const uint32_t t_end = uint32_t((uint64_t(split + 1) * ntiles) / n_splits);
    // Keys [0, kend_w) are visible to some query of this wave; 0 if the wave has no queries.
    const uint32_t kend_w = q0 < n_tok ? pos + min(n_tok, q0 + 32) : 0;
    const uint32_t qpos = pos + q0 + li;  // this lane's query position

    const _Float16* Kg = K + size_t(kvh) * kHeadDim;
    const _Float16* Vg = V + size_t(kvh) * kHeadDim;

    // B operand Q^T: lane holds Q[q0 + li][16*ks + 8*hb + e] * scale*log2(e), as f16.
    half8 qb[8];
    {
        const uint32_t row = q0 + li;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            if (row < n_tok) {
                const float4v* src = reinterpret_cast<const float4v*>(
                    q + size_t(row) * q_stride + size_t(h) * kHeadDim + 16 * ks + 8 * hb);
                const float4v a = src[0], b = src[1];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    qb[ks][e] = _Float16(a[e] * qscale);
                    qb[ks][4 + e] = _Float16(b[e] * qscale);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) qb[ks][e] = _Float16(0.f);
            }
        }
    }

    float16v O[4];
#pragma unroll
    for (int d = 0; d < 4; d++) O[d] = float16v{};
    float m = kNoMax, l = 0.f;

    for (uint32_t t = t_begin; t < t_end; t++) {
        const uint32_t kb = t * kBN;
        __syncthreads();  // the previous tile has been consumed
        // K tile: Ks[key][dim], 16 chunks of 16 B per key; rows past kend are zero.
        for (int i = tid; i < kBN * 16; i += NT) {
            const int key = i >> 4, ch = i & 15;
            const uint32_t kk = kb + key;
            half8 val = {};
            if (kk < kend) val = load_half8(Kg + size_t(kk) * kv_dim + 8 * ch);
            *reinterpret_cast<half8*>(&Ks[key * kKS + 8 * ch]) = val;
        }
        // V tile, transposed: Vt[dim][vt_pos(key)], two keys packed per 32-bit LDS write.
        for (int i = tid; i < (kBN / 2) * 16; i += NT) {
            const int pr = i >> 4, ch = i & 15;
            const uint32_t ka = kb + 2 * pr;
            half8 va = {}, vb = {};
            if (ka < kend) va = load_half8(Vg + size_t(ka) * kv_dim + 8 * ch);
            if (ka + 1 < kend) vb = load_half8(Vg + size_t(ka + 1) * kv_dim + 8 * ch);
            const int j = (2 * pr) & 15;
            const int col = ((2 * pr) & ~15) + vt_pos(j);
#pragma unroll
            for (int e = 0; e < 8; e++)
                *reinterpret_cast<uint32_t*>(&Vt[(8 * ch + e) * kVS + col]) = pack_halves(va[e], vb[e]);
        }
        __syncthreads();
        if (kb >= kend_w) continue;  // every key of this tile is in this wave's future

        // S^T (64 keys x 32 queries) as two 32x32 tiles.
        float16v S[2];
#pragma unroll
        for (int T = 0; T < 2; T++) {
            S[T] = float16v{};
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                const half8 a = *reinterpret_cast<const half8*>(&Ks[(32 * T + li) * kKS + 16 * ks + 8 * hb]);
                S[T] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[ks], S[T], 0, 0, 0);
            }
        }
        // Causal mask where the tile reaches past the wave's first query position.
        if (kb + kBN - 1 > pos + q0) {
#pragma unroll
            for (int T = 0; T < 2; T++)
#pragma unroll
                for (int rr = 0; rr < 16; rr++) {
                    const uint32_t key = kb + 32 * T + 8 * (rr >> 2) + 4 * hb + (rr & 3);
                    if (key > qpos) S[T][rr] = -__builtin_inff();
                }
        }
        float mx = S[0][0];
#pragma unroll
        for (int T = 0; T < 2; T++)
#pragma unroll
            for (int rr = 0; rr < 16; rr++) mx = fmaxf(mx, S[T][rr]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m, mx);
        const float alpha = fast_exp2(m - m_new);
        m = m_new;

        half8 P[4];
        float ls = 0.f;
#pragma unroll
        for (int T = 0; T < 2; T++)
#pragma unroll
            for (int rr = 0; rr < 16; rr++) {
                const float p = fast_exp2(S[T][rr] - m_new);
                ls += p;
                P[2 * T + (rr >> 3)][rr & 7] = _Float16(p);
            }
        l = l * alpha + ls;
#pragma unroll
        for (int d = 0; d < 4; d++) O[d] *= alpha;

        // O^T (128 dims x 32 queries) += V^T (128 x 64) P^T (64 x 32).
#pragma unroll
        for (int d = 0; d < 4; d++)
#pragma unroll
            for (int k4 = 0; k4 < 4; k4++) {
                const half8 a = *reinterpret_cast<const half8*>(&Vt[(32 * d + li) * kVS + 16 * k4 + 8 * hb]);
                O[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, P[k4], O[d], 0, 0, 0);
            }
    }

    // Both half-waves hold partial sums of the same rows (same m): add them.
    l += __shfl_xor(l, 32);
    const uint32_t row = q0 + li;
    if (row >= n_tok) return;
    if (n_splits == 1) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        float* dst = out + size_t(row) * q_stride + size_t(h) * kHeadDim;
#pragma unroll
        for (int d = 0; d < 4; d++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                float4v v = {O[d][4 * g], O[d][4 * g + 1], O[d][4 * g + 2], O[d][4 * g + 3]};
                *reinterpret_cast<float4v*>(dst + 32 * d + 8 * g + 4 * hb) = v * inv;
            }
    } else {
        const uint32_t n_head = n_head_kv * G;
        float* dst = part + ((size_t(split) * n_tok + row) * n_head + h) * kPartStride;
#pragma unroll
        for (int d = 0; d < 4; d++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                float4v v = {O[d][4 * g], O[d][4 * g + 1], O[d][4 * g + 2], O[d][4 * g + 3]};
                *reinterpret_cast<float4v*>(dst + 32 * d + 8 * g + 4 * hb) = v;
            }
        if (hb == 0) {
            dst[128] = m;
            dst[129] = l;
        }
    }
}

// out[tok][h][d] = sum_s o_s[d] 2^(m_s - M) / sum_s l_s 2^(m_s - M); 0 if the sum is 0.
// One 64-thread block per (token, head); thread t owns dims 2t, 2t+1.
__global__ __launch_bounds__(64) void attn_prefill_combine(const float* __restrict__ part,
                                                           float* __restrict__ out, uint32_t n_tok,
                                                           uint32_t n_head, uint32_t q_stride,
                                                           uint32_t n_splits) {
    const uint32_t row = blockIdx.x / n_head, h = blockIdx.x % n_head;
    const int d = threadIdx.x * 2;
    const size_t sstride = size_t(n_tok) * n_head * kPartStride;
    const float* src = part + (size_t(row) * n_head + h) * kPartStride;
    float M = kNoMax;
    for (uint32_t s = 0; s < n_splits; s++) M = fmaxf(M, src[s * sstride + 128]);
    float L = 0.f, O0 = 0.f, O1 = 0.f;
    for (uint32_t s = 0; s < n_splits; s++) {
        const float* ps = src + s * sstride;
        const float wt = fast_exp2(ps[128] - M);
        L += ps[129] * wt;
        O0 += ps[d] * wt;
        O1 += ps[d + 1] * wt;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    float* dst = out + size_t(row) * q_stride + size_t(h) * kHeadDim + d;
    dst[0] = O0 * inv;
    dst[1] = O1 * inv;
}

template <int G>
int launch_prefill_g(const float* q, const _Float16* k, const _Float16* v, float* out, float* part,
                     uint32_t pos, uint32_t n_tok, uint32_t q_stride, uint32_t n_head_kv,
                     uint32_t n_splits, float qscale, hipStream_t stream) {
    constexpr int NQB = 1;
    const dim3 grid((n_tok + 32 * NQB - 1) / (32 * NQB), n_head_kv, n_splits);
    hipLaunchKernelGGL((attn_prefill_kernel<G, NQB>), grid, dim3(64 * G * NQB), 0, stream, q, k, v,
                       out, part, pos, n_tok, q_stride, n_head_kv, n_splits, qscale);
    if (hipGetLastError() != hipSuccess) return -4;
    if (n_splits > 1) {
        const uint32_t n_head = n_head_kv * G;
        hipLaunchKernelGGL(attn_prefill_combine, dim3(n_tok * n_head), dim3(64), 0, stream, part,
                           out, n_tok, n_head, q_stride, n_splits);
        if (hipGetLastError() != hipSuccess) return -4;
    }
    return 0;
}

}  // namespace

uint32_t prefill_splits(uint32_t pos, uint32_t n_tok, uint32_t n_head, uint32_t requested) {
    const uint32_t max_tiles = (pos + n_tok + kBN - 1) / kBN;
    uint32_t splits = requested;
    if (splits == 0) {
        // Aim for >= 2048 waves (2 per SIMD on 256 CUs), keeping >= 2 key tiles per split.
        const uint32_t waves = ((n_tok + 31) / 32) * n_head;
        splits = (2048 + waves - 1) / waves;
        splits = min(splits, max(1u, max_tiles / 2));
    }
    return max(1u, min(splits, min(max_tiles, kMaxPrefillSplits)));
}

int launch_prefill(const float* q, const _Float16* k, const _Float16* v, float* out, float* part,
                   uint32_t pos, uint32_t n_tok, uint32_t q_stride, uint32_t n_head_kv,
                   uint32_t group, uint32_t n_splits, float scale, hipStream_t stream) {
    const float qscale = scale * kLog2e;
    switch (group) {
        case 1: return launch_prefill_g<1>(q, k, v, out, part, pos, n_tok, q_stride, n_head_kv, n_splits, qscale, stream);
        case 2: return launch_prefill_g<2>(q, k, v, out, part, pos, n_tok, q_stride, n_head_kv, n_splits, qscale, stream);
        case 3: return launch_prefill_g<3>(q, k, v, out, part, pos, n_tok, q_stride, n_head_kv, n_splits, qscale, stream);
        case 4: return launch_prefill_g<4>(q, k, v, out, part, pos, n_tok, q_stride, n_head_kv, n_splits, qscale, stream);
        default: return -2;
    }
}

}  // namespace ingot

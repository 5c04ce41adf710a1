// attn_decode.hip — split-KV (flash-decoding) GQA decode attention for gfx950.
//
// Computes, for one query token and every Q head h, out_h = softmax(q_h K^T * scale) V over cache
// rows 0..n_keys-1 of KV head h / G — the attention block of src/cpu_backend.cpp:51-69 and the
// decode flash path of src/metal_backend.mm:339-359 (attn_decode_g3 + attn_combine,
// shaders/kernels.metal:428-516), re-designed for CDNA4:
//
//   grid (n_splits, n_head_kv), 256 threads = 4 wave64. A workgroup owns one KV head and one
//   contiguous key slice, and serves all G query heads of the group from each K/V row it reads.
//   Within a wave, lane l owns dims 8*(l%16)..+7 (one 16-byte load) of key row (l/16), so one
//   load instruction covers 4 full 256-byte K rows; each wave keeps 4 keys x (K,V) = 8 loads in
//   flight per step. Scores are reduced across the 16 lanes of a row with 4 DPP adds.
//   Every 16-lane row runs its own online softmax (running max m, sum l, o[G][8]) in base 2;
//   rows merge with 2 xor-shuffles, waves merge through LDS, and splits merge in the last
//   workgroup to finish for that KV head (a completion counter, so no second launch is needed;
//   the reference launches attn_combine separately).
//
// Partial record (per KV head, split, group head): o[128] (unnormalized), m, l — as the
// reference's part[...][130] (AD_STRIDE, shaders/kernels.metal:291), stride 132 here.
#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace {

constexpr int kDecThreads = 256;
constexpr int kDecWaves = kDecThreads / 64;
constexpr int kKeysPerWaveStep = 16;                           // 4 rows x 4 unrolled loads
constexpr int kKeysPerBlockStep = kKeysPerWaveStep * kDecWaves;  // 64

template <int G>
__global__ __launch_bounds__(kDecThreads) void attn_decode_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ K, const _Float16* __restrict__ V,
    float* __restrict__ out, float* __restrict__ part, unsigned int* __restrict__ counters,
    uint32_t n_keys, uint32_t keys_per_split, uint32_t n_splits, uint32_t n_head_kv,
    float qscale) {
    __shared__ float red[kDecWaves][G][kPartStride];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int r = lane >> 4, c = lane & 15;
    const uint32_t split = blockIdx.x, kvh = blockIdx.y;
    const size_t kv_dim = size_t(n_head_kv) * kHeadDim;
    const uint32_t k0 = split * keys_per_split;
    const uint32_t k1 = min(n_keys, k0 + keys_per_split);

    // q pre-scaled by scale*log2(e): scores come out in base 2.
    float qf[G][8];
#pragma unroll
    for (int h = 0; h < G; h++) {
        const float4v* qp = reinterpret_cast<const float4v*>(q + (size_t(kvh) * G + h) * kHeadDim + 8 * c);
        const float4v a = qp[0], b = qp[1];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            qf[h][i] = a[i] * qscale;
            qf[h][4 + i] = b[i] * qscale;
        }
    }

    float o[G][8], m[G], l[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m[h] = kNoMax;
        l[h] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) o[h][i] = 0.f;
    }

    const _Float16* Kb = K + size_t(kvh) * kHeadDim + 8 * c;
    const _Float16* Vb = V + size_t(kvh) * kHeadDim + 8 * c;

    for (uint32_t base = k0 + wave * kKeysPerWaveStep; base < k1; base += kKeysPerBlockStep) {
        half8 kr[4], vr[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t key = min(base + 4 * u + r, k1 - 1);
            kr[u] = load_half8_nt(Kb + size_t(key) * kv_dim);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t key = min(base + 4 * u + r, k1 - 1);
            vr[u] = load_half8_nt(Vb + size_t(key) * kv_dim);
        }
        float s[G][4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const bool valid = base + 4 * u + r < k1;
#pragma unroll
            for (int h = 0; h < G; h++) {
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) acc = __builtin_fmaf(qf[h][i], float(kr[u][i]), acc);
                acc = row16_sum(acc);
                s[h][u] = valid ? acc : -__builtin_inff();
            }
        }
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float mt = fmaxf(fmaxf(s[h][0], s[h][1]), fmaxf(s[h][2], s[h][3]));
            const float m_new = fmaxf(m[h], mt);
            const float alpha = fast_exp2(m[h] - m_new);
            m[h] = m_new;
            float p[4];
#pragma unroll
            for (int u = 0; u < 4; u++) p[u] = fast_exp2(s[h][u] - m_new);
            l[h] = l[h] * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float acc = o[h][i] * alpha;
#pragma unroll
                for (int u = 0; u < 4; u++) acc = __builtin_fmaf(p[u], float(vr[u][i]), acc);
                o[h][i] = acc;
            }
        }
    }

    // Merge the 4 row streams of the wave (rows differ in lane bits 4 and 5).
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float m_o = __shfl_xor(m[h], off);
            const float l_o = __shfl_xor(l[h], off);
            const float M = fmaxf(m[h], m_o);
            const float a = fast_exp2(m[h] - M), b = fast_exp2(m_o - M);
            l[h] = l[h] * a + l_o * b;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float oo = __shfl_xor(o[h][i], off);
                o[h][i] = o[h][i] * a + oo * b;
            }
            m[h] = M;
        }
    }
    if (r == 0) {
#pragma unroll
        for (int h = 0; h < G; h++) {
#pragma unroll
            for (int i = 0; i < 8; i++) red[wave][h][8 * c + i] = o[h][i];
            if (c == 0) {
                red[wave][h][128] = m[h];
                red[wave][h][129] = l[h];
            }
        }
    }
    __syncthreads();

    // Merge the waves: thread t < G*32 owns head t/32, dims 4*(t%32)..+3.
    if (tid < G * 32) {
        const int h = tid >> 5, d = (tid & 31) * 4;
        float M = kNoMax;
#pragma unroll
        for (int w = 0; w < kDecWaves; w++) M = fmaxf(M, red[w][h][128]);
        float L = 0.f;
        float4v O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < kDecWaves; w++) {
            const float wt = fast_exp2(red[w][h][128] - M);
            L += red[w][h][129] * wt;
#pragma unroll
            for (int i = 0; i < 4; i++) O[i] += red[w][h][d + i] * wt;
        }
        const size_t head = size_t(kvh) * G + h;
        if (n_splits == 1) {
            const float inv = L > 0.f ? 1.f / L : 0.f;
            *reinterpret_cast<float4v*>(out + head * kHeadDim + d) = O * inv;
        } else {
            float* dst = part + ((size_t(kvh) * n_splits + split) * G + h) * kPartStride;
            *reinterpret_cast<float4v*>(dst + d) = O;
            if (d == 0) {
                dst[128] = M;
                dst[129] = L;
            }
        }
    }
    if (n_splits == 1) return;

    // Last workgroup to finish for this KV head merges the n_splits partials.
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = atomicAdd(&counters[kvh], 1u);
        s_last = (prev == n_splits - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    if (tid < G * 64) {
        const int h = tid >> 6, d = (tid & 63) * 2;
        const float* src = part + (size_t(kvh) * n_splits * G + h) * kPartStride;
        const size_t sstride = size_t(G) * kPartStride;
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
        float* dst = out + (size_t(kvh) * G + h) * kHeadDim + d;
        dst[0] = O0 * inv;
        dst[1] = O1 * inv;
    }
    if (tid == 0) counters[kvh] = 0u;  // leave the workspace ready for the next call
}

}  // namespace

uint32_t decode_splits(uint32_t n_keys, uint32_t n_head_kv, uint32_t requested) {
    uint32_t splits = requested;
    if (splits == 0) {
        // Aim for ~1024 workgroups over the chip (256 CUs) with at least one 64-key block step
        // per workgroup.
        const uint32_t target = max(1u, 1024u / max(1u, n_head_kv));
        splits = min(target, (n_keys + kKeysPerBlockStep - 1) / kKeysPerBlockStep);
    }
    splits = max(1u, min(splits, min(n_keys, kMaxDecodeSplits)));
    // No empty splits: recompute from the per-split key count.
    const uint32_t per = (n_keys + splits - 1) / splits;
    return (n_keys + per - 1) / per;
}

int launch_decode(const float* q, const _Float16* k, const _Float16* v, float* out, float* part,
                  unsigned int* counters, uint32_t n_keys, uint32_t n_splits, uint32_t n_head_kv,
                  uint32_t group, float scale, hipStream_t stream) {
    const uint32_t per = (n_keys + n_splits - 1) / n_splits;
    const dim3 grid(n_splits, n_head_kv), block(kDecThreads);
    const float qscale = scale * kLog2e;
    switch (group) {
        case 1: hipLaunchKernelGGL(attn_decode_kernel<1>, grid, block, 0, stream, q, k, v, out, part, counters, n_keys, per, n_splits, n_head_kv, qscale); break;
        case 2: hipLaunchKernelGGL(attn_decode_kernel<2>, grid, block, 0, stream, q, k, v, out, part, counters, n_keys, per, n_splits, n_head_kv, qscale); break;
        case 3: hipLaunchKernelGGL(attn_decode_kernel<3>, grid, block, 0, stream, q, k, v, out, part, counters, n_keys, per, n_splits, n_head_kv, qscale); break;
        case 4: hipLaunchKernelGGL(attn_decode_kernel<4>, grid, block, 0, stream, q, k, v, out, part, counters, n_keys, per, n_splits, n_head_kv, qscale); break;
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace ingot

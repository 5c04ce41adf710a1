// attn_decode.hip — split-KV (flash-decoding) GQA decode attention for gfx950.
//
// Computes, for one query token and every Q head h, out_h = softmax(q_h K^T * scale) V over cache
// rows 0..n_keys-1 of KV head h / G — the attention block of src/cpu_backend.cpp:51-69 and the
// decode flash path of src/metal_backend.mm:339-359 (attn_decode_g3 + attn_combine,
// shaders/kernels.metal:428-516), re-designed for CDNA4:
//
//   grid (n_splits, n_head_kv), NW wave64s per workgroup. A workgroup owns one KV head and one
//   contiguous key slice and serves all G query heads of the group from each K/V row it reads.
//   A wave step covers 16 keys:
//   - Scores on the matrix cores: S (16 rows x 16 keys) = A (16 x 256) * B (256 x 16) with
//     v_mfma_f32_16x16x32_f16 x 8. Rows 0..G-1 of A hold the G query heads; the 256-long
//     contraction is q_hi (128 dims) followed by q_lo (128 dims), where q*scale*log2(e) =
//     q_hi + q_lo with both parts f16, and B is the K tile repeated twice (same registers). The
//     score is thus exact to ~2^-22 relative even though K and the MFMA inputs are f16; the
//     accumulation is f32. Lane l loads 4 x 16 bytes of key row l%16.
//   - Online softmax per head with a wave-uniform running max (base 2), 16-lane DPP max.
//   - P*V on the vector ALUs (v_fma_mix: f16 V, f32 P and accumulators). For this, lane l owns
//     dims 8*(l%16)..+7 of key rows l/16 + 4u (u = 0..3); p reaches it through LDS.
//   - The K and V loads of the next step are issued before the current step is computed.
//   Waves merge through LDS. Splits merge in the last workgroup to finish for a KV head (a
//   completion counter, so no second launch; the reference launches attn_combine separately).
//   Partial records are written and read with device-scope (sc1) accesses, so neither an L2
//   writeback nor an L2 invalidate is needed; the merging workgroup issues all its loads in
//   one batch and spreads the splits over all of its threads.
//
// MFMA 16x16x32 f16 register layouts (wave64, lane l, i = l%16, g = l/16):
//   A (16 x 32): lane holds A[i][8g + e], e = 0..7;  B (32 x 16): lane holds B[8g + e][i];
//   D (16 x 16): lane holds D[4g + j][i], j = 0..3.
//
// Partial record (per KV head, split, group head): o[128] (unnormalized), m, l — as the
// reference's part[...][130] (AD_STRIDE, shaders/kernels.metal:291), stride 132 here.
#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace {

__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    x = fmaxf(x, dpp<0x141>(x));
    x = fmaxf(x, dpp<0x140>(x));
    return x;
}

__device__ __forceinline__ float lane0(float x) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
}

template <int G, int NW>
__global__ __launch_bounds__(64 * NW) void attn_decode_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ K, const _Float16* __restrict__ V,
    float* __restrict__ out, float* __restrict__ part, unsigned int* __restrict__ counters,
    uint32_t n_keys, uint32_t keys_per_split, uint32_t n_splits, uint32_t n_head_kv,
    float qscale) {
    constexpr int NT = 64 * NW;
    constexpr int KW = 16;  // keys per wave step
    // LDS: per-wave records during the workgroup merge, then per-thread partial merges in the
    // cross-split merge (the two uses do not overlap in time).
    constexpr int kRedFloats = NW * G * kPartStride;
    constexpr int kMrgFloats = NT * 6;
    __shared__ __attribute__((aligned(16))) float lds[kRedFloats > kMrgFloats ? kRedFloats : kMrgFloats];
    __shared__ __attribute__((aligned(16))) float lds_p[NW][KW][4];  // p[key][head] per wave
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int r = lane >> 4, c = lane & 15;
    const uint32_t split = blockIdx.x, kvh = blockIdx.y;
    const size_t kv_dim = size_t(n_head_kv) * kHeadDim;
    const uint32_t k0 = split * keys_per_split;
    const uint32_t k1 = min(n_keys, k0 + keys_per_split);

    // A operand: lane holds A[row c][k = 8r + e] of MFMA m (m < 4: q_hi of dims 32m+8r+e,
    // m >= 4: q_lo of the same dims). Rows >= G are zero.
    half8 qa[8];
    {
        const bool live = c < G;
        const float* qrow = q + (size_t(kvh) * G + (live ? c : 0)) * kHeadDim;
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

    // K: lane reads key row (base + c), 16 bytes at dims 32m + 8r. V: key rows base + 4u + r,
    // 16 bytes at dims 8c.
    const _Float16* Kb = K + size_t(kvh) * kHeadDim + 8 * r;
    const _Float16* Vb = V + size_t(kvh) * kHeadDim + 8 * c;

    // Loads are unconditional: rows past the slice are clamped to its last row (already in
    // cache), so the number of loads in flight is the same on every path and the compiler's
    // wait counts never stall the current step on the prefetch of the next. Two register
    // buffers alternate (ping-pong), so a prefetch never waits for the step it follows.
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

    constexpr uint32_t kStride = NW * KW;
    uint32_t base = k0 + wave * KW;
    half8 ka[4], va[4], kb[4], vb[4];
    load_step(base, ka, va);
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

    // Wave totals: o summed over the 4 lane rows (same dims, same wave-uniform max); l summed
    // over lanes 0..15.
#pragma unroll
    for (int h = 0; h < G; h++) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float x = o[h][i];
            x += __shfl_xor(x, 16);
            x += __shfl_xor(x, 32);
            o[h][i] = x;
        }
        l_run[h] = row16_sum(r == 0 ? l_run[h] : 0.f);
    }
    if (r == 0) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            float* rec = lds + (wave * G + h) * kPartStride;
            *reinterpret_cast<float4v*>(rec + 8 * c) = float4v{o[h][0], o[h][1], o[h][2], o[h][3]};
            *reinterpret_cast<float4v*>(rec + 8 * c + 4) = float4v{o[h][4], o[h][5], o[h][6], o[h][7]};
            if (c == 0) {
                rec[128] = m_run[h];
                rec[129] = l_run[h];
            }
        }
    }
    __syncthreads();

    // Merge the waves: thread t < G*32 owns head t/32, dims 4*(t%32)..+3.
    if (tid < G * 32) {
        const int h = tid >> 5, d = (tid & 31) * 4;
        float M = kNoMax;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, lds[(w * G + h) * kPartStride + 128]);
        float L = 0.f;
        float4v O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float* rec = lds + (w * G + h) * kPartStride;
            const float wt = fast_exp2(rec[128] - M);
            L += rec[129] * wt;
            O += *reinterpret_cast<const float4v*>(rec + d) * wt;
        }
        const size_t head = size_t(kvh) * G + h;
        if (n_splits == 1) {
            const float inv = L > 0.f ? 1.f / L : 0.f;
            *reinterpret_cast<float4v*>(out + head * kHeadDim + d) = O * inv;
        } else {
            // Device-scope (sc1) stores, all issued before one wait for their completion, so
            // the record is visible to a workgroup on another XCD without an L2 writeback.
            float* dst = part + ((size_t(kvh) * n_splits + split) * G + h) * kPartStride;
#pragma unroll
            for (int i = 0; i < 4; i++)
                __hip_atomic_store(dst + d + i, O[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d == 0) {
                __hip_atomic_store(dst + 128, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(dst + 129, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __builtin_amdgcn_s_waitcnt(0);  // the device-scope stores have completed
        }
    }
    if (n_splits == 1) return;

    // The last workgroup to finish for this KV head merges the n_splits partials. The records
    // were stored device-scope and awaited before the barrier, so a relaxed device-scope
    // counter increment orders them; only the merging workgroup invalidates its L2 (acquire).
    unsigned int* counter = counters + size_t(kvh) * kCounterStride;
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == n_splits - 1);
    }
    __syncthreads();
    if (!s_last) return;

    // Merge: thread t < P*COLS owns column (head, 4 dims) t % COLS and the splits s = t / COLS
    // (mod P). All of its record words are loaded device-scope (sc1, coherent across XCDs
    // without an L2 invalidate) in one unrolled batch, merged with the log-sum-exp rule, and
    // the P partial merges per column are combined through LDS.
    {
        constexpr int COLS = G * 32;
        constexpr int P = NT / COLS;
        constexpr int ITER = (int(kMaxDecodeSplits) + P - 1) / P;
        float M = kNoMax, L = 0.f;
        float4v O = {0.f, 0.f, 0.f, 0.f};
        const int col = tid % COLS, grp = tid / COLS;
        const int h = col >> 5, d = (col & 31) * 4;
        if (grp < P) {
            const float* base_rec = part + (size_t(kvh) * n_splits * G + h) * kPartStride;
            float ms[ITER], ls[ITER];
            float4v os[ITER];
            // Unconditional loads from clamped indices (no branches between them, so they
            // are all in flight at once); out-of-range splits are masked afterwards.
#pragma unroll
            for (int it = 0; it < ITER; it++) {
                const uint32_t sp = min(uint32_t(grp + it * P), n_splits - 1);
                const float* rec = base_rec + size_t(sp) * G * kPartStride;
                ms[it] = __hip_atomic_load(rec + 128, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ls[it] = __hip_atomic_load(rec + 129, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                for (int i = 0; i < 4; i++)
                    os[it][i] = __hip_atomic_load(rec + d + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int it = 0; it < ITER; it++) {
                const bool ok = uint32_t(grp + it * P) < n_splits;
                ms[it] = ok ? ms[it] : kNoMax;
                ls[it] = ok ? ls[it] : 0.f;
                os[it] = ok ? os[it] : float4v{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int it = 0; it < ITER; it++) M = fmaxf(M, ms[it]);
#pragma unroll
            for (int it = 0; it < ITER; it++) {
                const float wt = fast_exp2(ms[it] - M);
                L += ls[it] * wt;
                O += os[it] * wt;
            }
        }
        __syncthreads();  // the workgroup-merge records in LDS are no longer needed
        float* red = lds;  // [P][COLS][6]: o[4], m, l
        if (grp < P) {
            float* e = red + (grp * COLS + col) * 6;
            e[0] = O[0]; e[1] = O[1]; e[2] = O[2]; e[3] = O[3]; e[4] = M; e[5] = L;
        }
        __syncthreads();
        if (tid < COLS) {
            float Mt = kNoMax;
#pragma unroll
            for (int g = 0; g < P; g++) Mt = fmaxf(Mt, red[(g * COLS + tid) * 6 + 4]);
            float Lt = 0.f;
            float4v Ot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int g = 0; g < P; g++) {
                const float* e = red + (g * COLS + tid) * 6;
                const float wt = fast_exp2(e[4] - Mt);
                Lt += e[5] * wt;
                Ot += float4v{e[0], e[1], e[2], e[3]} * wt;
            }
            const float inv = Lt > 0.f ? 1.f / Lt : 0.f;
            *reinterpret_cast<float4v*>(out + (size_t(kvh) * G + h) * kHeadDim + d) = Ot * inv;
        }
    }
    if (tid == 0)  // leave the workspace ready for the next call
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int G, int NW>
void launch_g(dim3 grid, hipStream_t stream, const float* q, const _Float16* k, const _Float16* v,
              float* out, float* part, unsigned int* counters, uint32_t n_keys, uint32_t per,
              uint32_t n_splits, uint32_t n_head_kv, float qscale) {
    hipLaunchKernelGGL((attn_decode_kernel<G, NW>), grid, dim3(64 * NW), 0, stream, q, k, v, out,
                       part, counters, n_keys, per, n_splits, n_head_kv, qscale);
}

constexpr int kNW = 4;
constexpr uint32_t kKeysPerBlockStep = uint32_t(kNW) * 16;

}  // namespace

uint32_t decode_splits(uint32_t n_keys, uint32_t n_head_kv, uint32_t requested) {
    (void)n_head_kv;
    uint32_t splits = requested;
    if (splits == 0) {
        // One block step (kKeysPerBlockStep keys) or more per workgroup.
        splits = (n_keys + kKeysPerBlockStep - 1) / kKeysPerBlockStep;
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
    const dim3 grid(n_splits, n_head_kv);
    const float qscale = scale * kLog2e;
    switch (group) {
        case 1: launch_g<1, kNW>(grid, stream, q, k, v, out, part, counters, n_keys, per, n_splits, n_head_kv, qscale); break;
        case 2: launch_g<2, kNW>(grid, stream, q, k, v, out, part, counters, n_keys, per, n_splits, n_head_kv, qscale); break;
        case 3: launch_g<3, kNW>(grid, stream, q, k, v, out, part, counters, n_keys, per, n_splits, n_head_kv, qscale); break;
        case 4: launch_g<4, kNW>(grid, stream, q, k, v, out, part, counters, n_keys, per, n_splits, n_head_kv, qscale); break;
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace ingot

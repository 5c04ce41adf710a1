// attn_naive.hip — attention for head sizes the MFMA kernels do not cover (anything but 64,
// 128 and 256, up to 1024): decode and causal prefill.
//
// The counterpart of the reference's naive `attention` kernel (shaders/kernels.metal:639-702),
// which src/metal_backend.mm:373-382 runs for every shape outside its flash paths: query i of
// head h at absolute position pos + i attends to cache rows 0..pos+i of KV head h / group, with
// the semantics of src/cpu_backend.cpp:51-69 (scores q.k * scale, softmax, weighted sum of V).
// The reference keeps all pos+i+1 scores in threadgroup memory; here a workgroup walks its keys
// in chunks of 256 with an online softmax (running max and sum, rescaled per chunk), so the
// context length is not bounded by LDS.
//
// Workgroup = one query head, TQ consecutive tokens (8 for prefill, 1 for decode) and a key
// slice, 256 threads. Per chunk: thread t scores key c0 + t against the TQ queries (f32 dot
// products, q staged in LDS, the f16 K row read once, 16, 4 or 2 bytes at a time as the row
// alignment allows), the workgroup reduces each query's chunk max and sum through LDS, and the
// threads then accumulate the TQ outputs over the chunk's keys: the head's dims are cut into
// groups of VW, thread t takes one dim group and every KGp-th key of the chunk (KGp key phases),
// each V load feeding all TQ queries. Prefill runs one slice per (head, token block); decode
// splits the keys into slices of at least kMinSliceKeys so that a long cache spreads over the
// CUs, each slice writes (o, m, l) to the workspace, and a second launch merges them with the
// log-sum-exp rule of attn_combine (shaders/kernels.metal:501-516).
// Bytes per unit (one key row of one KV head, read once per query head and token block):
// 4 * head_dim.
#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxDims = 1024;
constexpr int kPrefillTokens = 8;  // TQ of a prefill workgroup

__device__ __forceinline__ float wave_max64(float x) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}
__device__ __forceinline__ float wave_sum64(float x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// VW: K and V read width (halves; divides hd and the row alignment). NG: dim groups a thread
// owns in the V phase (more than one only when hd / VW > 256; then KGp = 1). Workgroup b: slice
// b % n_slices of the (token block, head) pair b / n_slices. With one slice the outputs are
// written directly; with several (decode, TQ = 1), the slice's record (o[hd] unnormalized, m, l)
// goes to part[((pair) * n_slices + slice) * (hd + 2)].
template <int TQ, int NG, int VW>
__global__ __launch_bounds__(kThreads) void attn_any_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ K, const _Float16* __restrict__ V,
    float* __restrict__ out, float* __restrict__ part, uint32_t pos, uint32_t n_tok, uint32_t n_head,
    uint32_t group, uint32_t hd, uint32_t kv_dim, uint32_t q_stride, uint32_t n_slices, uint32_t slice_keys,
    float scale) {
    typedef _Float16 hv __attribute__((ext_vector_type(VW)));
    __shared__ float qs[TQ][kMaxDims];
    __shared__ float ps[TQ][kThreads];
    __shared__ float red[2][TQ][kWaves];
    __shared__ float osum[kThreads * VW > kMaxDims ? kThreads * VW : kMaxDims];  // [phase][hd]

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t pair = blockIdx.x / n_slices, slice = blockIdx.x % n_slices;
    const uint32_t h = pair % n_head, tok0 = (pair / n_head) * TQ;
    const uint32_t nq = min(uint32_t(TQ), n_tok - tok0);  // live queries of the block
    const uint32_t qp0 = pos + tok0;                        // position of query 0
    const uint32_t n = qp0 + nq;                            // keys 0..n-1 are visible to some query
    const uint32_t kb = slice * slice_keys, ke = min(n, kb + slice_keys);
    const _Float16* Kh = K + size_t(h / group) * hd;
    const _Float16* Vh = V + size_t(h / group) * hd;
#pragma unroll
    for (int j = 0; j < TQ; j++) {
        if (uint32_t(j) < nq) {
            const float* qh = q + size_t(tok0 + j) * q_stride + size_t(h) * hd;
            for (uint32_t i = tid; i < hd; i += kThreads) qs[j][i] = qh[i];
        } else {
            for (uint32_t i = tid; i < hd; i += kThreads) qs[j][i] = 0.f;
        }
    }
    __syncthreads();

    const uint32_t DG = hd / VW;
    const uint32_t KGp = DG <= kThreads ? kThreads / DG : 1;  // key phases
    const uint32_t dg = DG <= kThreads ? tid % DG : tid, kq = DG <= kThreads ? tid / DG : 0;
    const bool vlive = kq < KGp;
    float m_run[TQ], l_run[TQ];
    float o[TQ][NG][VW];
#pragma unroll
    for (int j = 0; j < TQ; j++) {
        m_run[j] = kNoMax;
        l_run[j] = 0.f;
#pragma unroll
        for (int g = 0; g < NG; g++)
#pragma unroll
            for (int e = 0; e < VW; e++) o[j][g][e] = 0.f;
    }

    for (uint32_t c0 = kb; c0 < ke; c0 += kThreads) {
        const uint32_t t = c0 + tid;
        // Scores of key t against the TQ queries; query j sees keys up to qp0 + j.
        float s[TQ];
        {
            float acc[TQ];
#pragma unroll
            for (int j = 0; j < TQ; j++) acc[j] = 0.f;
            if (t < ke) {
                const _Float16* kt = Kh + size_t(t) * kv_dim;
                for (uint32_t i = 0; i < hd; i += VW) {
                    const hv k = *reinterpret_cast<const hv*>(kt + i);
#pragma unroll
                    for (int j = 0; j < TQ; j++)
#pragma unroll
                        for (int e = 0; e < VW; e++) acc[j] += qs[j][i + e] * float(k[e]);
                }
            }
#pragma unroll
            for (int j = 0; j < TQ; j++) s[j] = t < ke && t <= qp0 + j ? acc[j] * scale : kNoMax;
        }
        // chunk max per query
#pragma unroll
        for (int j = 0; j < TQ; j++) {
            const float x = wave_max64(s[j]);
            if (lane == 0) red[0][j][wave] = x;
        }
        __syncthreads();
        float alpha[TQ];
#pragma unroll
        for (int j = 0; j < TQ; j++) {
            float cmax = red[0][j][0];
#pragma unroll
            for (int w = 1; w < kWaves; w++) cmax = fmaxf(cmax, red[0][j][w]);
            const float m_new = fmaxf(m_run[j], cmax);
            alpha[j] = expf(m_run[j] - m_new);
            const float p = t < ke && t <= qp0 + j ? expf(s[j] - m_new) : 0.f;
            ps[j][tid] = p;
            const float x = wave_sum64(p);
            if (lane == 0) red[1][j][wave] = x;
            m_run[j] = m_new;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < TQ; j++) {
            float csum = red[1][j][0];
#pragma unroll
            for (int w = 1; w < kWaves; w++) csum += red[1][j][w];
            l_run[j] = l_run[j] * alpha[j] + csum;
        }
        const uint32_t nk = min(uint32_t(kThreads), ke - c0);
        if (vlive) {
#pragma unroll
            for (int g = 0; g < NG; g++) {
                const uint32_t gi = dg + kThreads * g;
                if (gi >= DG) break;
                const _Float16* vt = Vh + size_t(c0) * kv_dim + gi * VW;
#pragma unroll
                for (int j = 0; j < TQ; j++)
#pragma unroll
                    for (int e = 0; e < VW; e++) o[j][g][e] *= alpha[j];
                uint32_t k = kq;
                // four keys' loads in flight
                for (; k + 3 * KGp < nk; k += 4 * KGp) {
                    hv vv[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) vv[u] = *reinterpret_cast<const hv*>(vt + size_t(k + u * KGp) * kv_dim);
#pragma unroll
                    for (int u = 0; u < 4; u++)
#pragma unroll
                        for (int j = 0; j < TQ; j++) {
                            const float pu = ps[j][k + u * KGp];
#pragma unroll
                            for (int e = 0; e < VW; e++) o[j][g][e] += pu * float(vv[u][e]);
                        }
                }
                for (; k < nk; k += KGp) {
                    const hv vv = *reinterpret_cast<const hv*>(vt + size_t(k) * kv_dim);
#pragma unroll
                    for (int j = 0; j < TQ; j++) {
                        const float pu = ps[j][k];
#pragma unroll
                        for (int e = 0; e < VW; e++) o[j][g][e] += pu * float(vv[e]);
                    }
                }
            }
        }
        __syncthreads();  // ps and red are rewritten by the next chunk
    }
    // Per query: the key phases' partial sums, added in phase order through osum[kq * hd + d].
#pragma unroll
    for (int j = 0; j < TQ; j++) {
        if (uint32_t(j) >= nq) break;
        if (j > 0) __syncthreads();  // the previous query's sums have been read
        if (vlive) {
#pragma unroll
            for (int g = 0; g < NG; g++) {
                const uint32_t gi = dg + kThreads * g;
                if (gi >= DG) break;
#pragma unroll
                for (int e = 0; e < VW; e++) osum[kq * hd + gi * VW + e] = o[j][g][e];
            }
        }
        __syncthreads();
        const float inv = l_run[j] > 0.f ? 1.f / l_run[j] : 0.f;
        float* rec = part + (size_t(pair) * n_slices + slice) * (hd + 2);
        float* oh = out + size_t(tok0 + j) * q_stride + size_t(h) * hd;
        for (uint32_t d = tid; d < hd; d += kThreads) {
            float od = osum[d];
            for (uint32_t k = 1; k < KGp; k++) od += osum[k * hd + d];
            if (n_slices == 1) oh[d] = od * inv;
            else rec[d] = od;
        }
        if (n_slices > 1 && tid == 0) {
            rec[hd] = m_run[j];
            rec[hd + 1] = l_run[j];
        }
    }
}

// Merge of the decode slices' records (the log-sum-exp rule of attn_combine,
// shaders/kernels.metal:501-516): workgroup = one head. Thread s < n_slices loads slice s's
// (m, l); the weights e^(m_s - M) go through LDS; then thread d sums o_s[d] * w_s over the slices
// in order, eight slices' loads in flight.
__global__ __launch_bounds__(kThreads) void attn_any_combine(const float* __restrict__ part, float* __restrict__ out,
                                                             uint32_t hd, uint32_t n_slices) {
    __shared__ float w[kMaxAnySlices];
    __shared__ float Ls;
    const uint32_t h = blockIdx.x, tid = threadIdx.x;
    const float* recs = part + size_t(h) * n_slices * (hd + 2);
    if (tid < 64) {  // one wave: n_slices <= kMaxAnySlices = 64
        const bool have = tid < n_slices;
        const float m = have ? recs[tid * (hd + 2) + hd] : kNoMax;
        const float l = have ? recs[tid * (hd + 2) + hd + 1] : 0.f;
        const float M = wave_max64(m);
        const float ws = have ? expf(m - M) : 0.f;
        const float L = wave_sum64(l * ws);
        w[tid] = ws;
        if (tid == 0) Ls = L;
    }
    __syncthreads();
    const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
    for (uint32_t d = tid; d < hd; d += kThreads) {
        float acc = 0.f;
        uint32_t s = 0;
        for (; s + 8 <= n_slices; s += 8) {
            float x[8];
#pragma unroll
            for (int u = 0; u < 8; u++) x[u] = recs[(s + u) * (hd + 2) + d];
#pragma unroll
            for (int u = 0; u < 8; u++) acc += x[u] * w[s + u];
        }
        for (; s < n_slices; s++) acc += recs[s * (hd + 2) + d] * w[s];
        out[size_t(h) * hd + d] = acc * inv;
    }
}

template <int TQ, int NG>
void launch_ng(uint32_t vw, dim3 grid, hipStream_t stream, const float* q, const _Float16* k, const _Float16* v,
               float* out, float* part, uint32_t pos, uint32_t n_tok, uint32_t n_head, uint32_t group, uint32_t hd,
               uint32_t kv_dim, uint32_t q_stride, uint32_t n_slices, uint32_t slice_keys, float scale) {
    const dim3 block{uint32_t(kThreads)};
    if constexpr (NG == 1) {
        if (vw == 8) {
            hipLaunchKernelGGL((attn_any_kernel<TQ, 1, 8>), grid, block, 0, stream, q, k, v, out, part, pos, n_tok,
                               n_head, group, hd, kv_dim, q_stride, n_slices, slice_keys, scale);
            return;
        }
    }
    if constexpr (NG <= 2) {
        if (vw == 2) {
            hipLaunchKernelGGL((attn_any_kernel<TQ, NG, 2>), grid, block, 0, stream, q, k, v, out, part, pos, n_tok,
                               n_head, group, hd, kv_dim, q_stride, n_slices, slice_keys, scale);
            return;
        }
    }
    hipLaunchKernelGGL((attn_any_kernel<TQ, NG, 1>), grid, block, 0, stream, q, k, v, out, part, pos, n_tok,
                       n_head, group, hd, kv_dim, q_stride, n_slices, slice_keys, scale);
}

template <int TQ>
void launch_tq(uint32_t vw, dim3 grid, hipStream_t stream, const float* q, const _Float16* k, const _Float16* v,
               float* out, float* part, uint32_t pos, uint32_t n_tok, uint32_t n_head, uint32_t group, uint32_t hd,
               uint32_t kv_dim, uint32_t q_stride, uint32_t n_slices, uint32_t slice_keys, float scale) {
    // dim groups of vw per thread in the V phase: at most 1024 / 8 = 128 for vw 8, 512 for vw 2
    const uint32_t groups = hd / vw;
    if (groups <= 256)
        launch_ng<TQ, 1>(vw, grid, stream, q, k, v, out, part, pos, n_tok, n_head, group, hd, kv_dim, q_stride,
                         n_slices, slice_keys, scale);
    else if (groups <= 512)
        launch_ng<TQ, 2>(vw, grid, stream, q, k, v, out, part, pos, n_tok, n_head, group, hd, kv_dim, q_stride,
                         n_slices, slice_keys, scale);
    else
        launch_ng<TQ, 4>(vw, grid, stream, q, k, v, out, part, pos, n_tok, n_head, group, hd, kv_dim, q_stride,
                         n_slices, slice_keys, scale);
}

}  // namespace

uint32_t attn_any_slices(uint32_t n_keys, uint32_t n_tok) {
    // Decode only: slices of at least kMinSliceKeys keys, at most kMaxAnySlices of them.
    if (n_tok != 1) return 1;
    const uint32_t s = (n_keys + kMinSliceKeys - 1) / kMinSliceKeys;
    return s < kMaxAnySlices ? s : kMaxAnySlices;
}

int launch_attn_any(const float* q, const _Float16* k, const _Float16* v, float* out, float* part, uint32_t pos,
                    uint32_t n_tok, uint32_t q_stride, uint32_t n_head, uint32_t n_head_kv, uint32_t head_dim,
                    float scale, hipStream_t stream) {
    if (head_dim == 0 || head_dim > uint32_t(kMaxDims)) return -2;
    const uint32_t n_slices = part != nullptr ? attn_any_slices(pos + 1, n_tok) : 1u;  // no records: one slice
    const uint32_t slice_keys = (pos + n_tok + n_slices - 1) / n_slices;
    // Token blocks: TQ = 8 tokens per workgroup for a prefill whose keys span more than one
    // chunk, so each K/V row read serves 8 queries (head_dim 96, 24/8 heads, 128 tokens at 384:
    // 75.1 -> 46.5 us); one token per workgroup for decode and for short prefills, where the
    // 8x larger grid is worth more than the shared reads (128 tokens at 0: 14.4 us against 26.0).
    const uint32_t tq = n_tok > 1 && pos + n_tok > uint32_t(kThreads) ? kPrefillTokens : 1;
    const uint64_t blocks = uint64_t(n_head) * ((n_tok + tq - 1) / tq) * n_slices;
    if (blocks > 0x7fffffffu) return -1;
    const uint32_t group = n_head / n_head_kv, kv_dim = n_head_kv * head_dim;
    // K rows start at element t * kv_dim + kvh * head_dim: 16-byte aligned when head_dim is a
    // multiple of 8 (the cache base and kv_offset are 16-byte aligned), 4-byte when it is even.
    const uint32_t vw = head_dim % 8 == 0 ? 8 : head_dim % 2 == 0 ? 2 : 1;
    const dim3 grid{uint32_t(blocks)};
    if (tq == 1)
        launch_tq<1>(vw, grid, stream, q, k, v, out, part, pos, n_tok, n_head, group, head_dim, kv_dim, q_stride,
                     n_slices, slice_keys, scale);
    else
        launch_tq<kPrefillTokens>(vw, grid, stream, q, k, v, out, part, pos, n_tok, n_head, group, head_dim, kv_dim,
                                  q_stride, n_slices, slice_keys, scale);
    if (hipGetLastError() != hipSuccess) return -4;
    if (n_slices > 1) {
        hipLaunchKernelGGL(attn_any_combine, dim3(n_head), dim3(kThreads), 0, stream, part, out, head_dim, n_slices);
        if (hipGetLastError() != hipSuccess) return -4;
    }
    return 0;
}

}  // namespace ingot

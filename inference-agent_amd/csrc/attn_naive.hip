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
// Workgroup = one (query head, token, key slice), 256 threads. Per chunk: thread t scores key
// c0 + t (the dot product over head_dim in f32, q staged in LDS, the f16 K row read 16, 4 or 2
// bytes at a time as the row alignment allows), the workgroup reduces the chunk's max and sum
// through LDS, and thread t then accumulates output dims t, t + 256, ... over the chunk's keys
// (consecutive threads read consecutive V elements, eight keys' loads in flight). Prefill runs
// one slice per (head, token); decode splits the keys into slices of at least 1024 so that a
// long cache spreads over the CUs, each slice writes (o, m, l) to the workspace, and a second
// launch merges them with the log-sum-exp rule of attn_combine (shaders/kernels.metal:501-516).
// Bytes per unit (one key row of one KV head, read once per query head): 4 * head_dim.
#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ float wave_max64(float x) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}
__device__ __forceinline__ float wave_sum64(float x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// q . k over hd elements, k read VW halves at a time (VW divides hd and the row alignment).
template <int VW>
__device__ __forceinline__ float dot_row(const float* qs, const _Float16* kt, uint32_t hd) {
    typedef _Float16 hv __attribute__((ext_vector_type(VW)));
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    uint32_t i = 0;
    for (; i + 4 * VW <= hd; i += 4 * VW) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const hv k = *reinterpret_cast<const hv*>(kt + i + u * VW);
#pragma unroll
            for (int e = 0; e < VW; e++) acc[u] += qs[i + u * VW + e] * float(k[e]);
        }
    }
    for (; i < hd; i += VW) {
        const hv k = *reinterpret_cast<const hv*>(kt + i);
#pragma unroll
        for (int e = 0; e < VW; e++) acc[0] += qs[i + e] * float(k[e]);
    }
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

// VPT: output dims per thread (head_dim <= 256 * VPT); VW: K read width (halves).
// Workgroup b: slice b % n_slices of the (token, head) pair b / n_slices. With one slice the
// output is written directly; with several, the slice's record (o[hd] unnormalized, m, l) goes
// to part[((pair) * n_slices + slice) * (hd + 2)].
template <int VPT, int VW>
__global__ __launch_bounds__(kThreads) void attn_any_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ K, const _Float16* __restrict__ V,
    float* __restrict__ out, float* __restrict__ part, uint32_t pos, uint32_t n_head, uint32_t group,
    uint32_t hd, uint32_t kv_dim, uint32_t q_stride, uint32_t n_slices, uint32_t slice_keys, float scale) {
    __shared__ float qs[kThreads * VPT];
    __shared__ float ps[kThreads];
    __shared__ float red[2][kWaves];

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t pair = blockIdx.x / n_slices, slice = blockIdx.x % n_slices;
    const uint32_t h = pair % n_head, tok = pair / n_head;
    const uint32_t n = pos + tok + 1;  // keys 0..pos+tok are visible
    const uint32_t kb = slice * slice_keys, ke = min(n, kb + slice_keys);
    const float* qh = q + size_t(tok) * q_stride + size_t(h) * hd;
    const _Float16* Kh = K + size_t(h / group) * hd;
    const _Float16* Vh = V + size_t(h / group) * hd;
    for (uint32_t i = tid; i < hd; i += kThreads) qs[i] = qh[i];
    __syncthreads();

    float m_run = kNoMax, l_run = 0.f;
    float o[VPT];
#pragma unroll
    for (int j = 0; j < VPT; j++) o[j] = 0.f;

    for (uint32_t c0 = kb; c0 < ke; c0 += kThreads) {
        const uint32_t t = c0 + tid;
        const float s = t < ke ? dot_row<VW>(qs, Kh + size_t(t) * kv_dim, hd) * scale : kNoMax;
        // chunk max
        float x = wave_max64(s);
        if (lane == 0) red[0][wave] = x;
        __syncthreads();
        float cmax = red[0][0];
#pragma unroll
        for (int w = 1; w < kWaves; w++) cmax = fmaxf(cmax, red[0][w]);
        const float m_new = fmaxf(m_run, cmax);
        const float alpha = expf(m_run - m_new);
        const float p = t < ke ? expf(s - m_new) : 0.f;
        ps[tid] = p;
        x = wave_sum64(p);
        if (lane == 0) red[1][wave] = x;
        __syncthreads();
        float csum = red[1][0];
#pragma unroll
        for (int w = 1; w < kWaves; w++) csum += red[1][w];
        l_run = l_run * alpha + csum;
        m_run = m_new;
        const uint32_t nk = min(uint32_t(kThreads), ke - c0);
#pragma unroll
        for (int j = 0; j < VPT; j++) {
            const uint32_t d = tid + kThreads * j;
            if (d < hd) {
                const _Float16* vt = Vh + size_t(c0) * kv_dim + d;
                float acc[8] = {o[j] * alpha, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                uint32_t k = 0;
                for (; k + 8 <= nk; k += 8) {
                    _Float16 vv[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) vv[u] = vt[size_t(k + u) * kv_dim];
#pragma unroll
                    for (int u = 0; u < 8; u++) acc[u] += ps[k + u] * float(vv[u]);
                }
                for (; k < nk; k++) acc[0] += ps[k] * float(vt[size_t(k) * kv_dim]);
                o[j] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
            }
        }
        __syncthreads();  // ps and red are rewritten by the next chunk
    }
    if (n_slices == 1) {
        const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
        float* oh = out + size_t(tok) * q_stride + size_t(h) * hd;
#pragma unroll
        for (int j = 0; j < VPT; j++) {
            const uint32_t d = tid + kThreads * j;
            if (d < hd) oh[d] = o[j] * inv;
        }
        return;
    }
    float* rec = part + (size_t(pair) * n_slices + slice) * (hd + 2);
#pragma unroll
    for (int j = 0; j < VPT; j++) {
        const uint32_t d = tid + kThreads * j;
        if (d < hd) rec[d] = o[j];
    }
    if (tid == 0) {
        rec[hd] = m_run;
        rec[hd + 1] = l_run;
    }
}

// Merge of the decode slices' records: workgroup = one head, thread = output dims d, d + 256...
__global__ __launch_bounds__(kThreads) void attn_any_combine(const float* __restrict__ part, float* __restrict__ out,
                                                             uint32_t hd, uint32_t n_slices) {
    const uint32_t h = blockIdx.x;
    const float* recs = part + size_t(h) * n_slices * (hd + 2);
    float M = kNoMax;
    for (uint32_t s = 0; s < n_slices; s++) M = fmaxf(M, recs[s * (hd + 2) + hd]);
    float L = 0.f;
    for (uint32_t s = 0; s < n_slices; s++) L += recs[s * (hd + 2) + hd + 1] * expf(recs[s * (hd + 2) + hd] - M);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    for (uint32_t d = threadIdx.x; d < hd; d += kThreads) {
        float acc = 0.f;
        for (uint32_t s = 0; s < n_slices; s++) acc += recs[s * (hd + 2) + d] * expf(recs[s * (hd + 2) + hd] - M);
        out[size_t(h) * hd + d] = acc * inv;
    }
}

template <int VPT>
void launch_vpt(uint32_t vw, dim3 grid, hipStream_t stream, const float* q, const _Float16* k, const _Float16* v,
                float* out, float* part, uint32_t pos, uint32_t n_head, uint32_t group, uint32_t hd,
                uint32_t kv_dim, uint32_t q_stride, uint32_t n_slices, uint32_t slice_keys, float scale) {
    const dim3 block{uint32_t(kThreads)};
    if (vw == 8)
        hipLaunchKernelGGL((attn_any_kernel<VPT, 8>), grid, block, 0, stream, q, k, v, out, part, pos, n_head,
                           group, hd, kv_dim, q_stride, n_slices, slice_keys, scale);
    else if (vw == 2)
        hipLaunchKernelGGL((attn_any_kernel<VPT, 2>), grid, block, 0, stream, q, k, v, out, part, pos, n_head,
                           group, hd, kv_dim, q_stride, n_slices, slice_keys, scale);
    else
        hipLaunchKernelGGL((attn_any_kernel<VPT, 1>), grid, block, 0, stream, q, k, v, out, part, pos, n_head,
                           group, hd, kv_dim, q_stride, n_slices, slice_keys, scale);
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
    if (head_dim == 0 || head_dim > 1024) return -2;
    const uint32_t n_slices = part != nullptr ? attn_any_slices(pos + 1, n_tok) : 1u;  // no records: one slice
    const uint32_t slice_keys = (pos + n_tok + n_slices - 1) / n_slices;
    const uint64_t blocks = uint64_t(n_head) * n_tok * n_slices;
    if (blocks > 0x7fffffffu) return -1;
    const uint32_t group = n_head / n_head_kv, kv_dim = n_head_kv * head_dim;
    // K rows start at element t * kv_dim + kvh * head_dim: 16-byte aligned when head_dim is a
    // multiple of 8 (the cache base and kv_offset are 16-byte aligned), 4-byte when it is even.
    const uint32_t vw = head_dim % 8 == 0 ? 8 : head_dim % 2 == 0 ? 2 : 1;
    const dim3 grid{uint32_t(blocks)};
    if (head_dim <= 256)
        launch_vpt<1>(vw, grid, stream, q, k, v, out, part, pos, n_head, group, head_dim, kv_dim, q_stride, n_slices,
                      slice_keys, scale);
    else if (head_dim <= 512)
        launch_vpt<2>(vw, grid, stream, q, k, v, out, part, pos, n_head, group, head_dim, kv_dim, q_stride, n_slices,
                      slice_keys, scale);
    else
        launch_vpt<4>(vw, grid, stream, q, k, v, out, part, pos, n_head, group, head_dim, kv_dim, q_stride, n_slices,
                      slice_keys, scale);
    if (hipGetLastError() != hipSuccess) return -4;
    if (n_slices > 1) {
        hipLaunchKernelGGL(attn_any_combine, dim3(n_head), dim3(kThreads), 0, stream, part, out, head_dim, n_slices);
        if (hipGetLastError() != hipSuccess) return -4;
    }
    return 0;
}

}  // namespace ingot

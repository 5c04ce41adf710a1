// attn_naive.hip — attention for head sizes the MFMA kernels do not cover (anything but 64,
// 128 and 256, up to 1024): decode and causal prefill in one kernel.
//
// The counterpart of the reference's naive `attention` kernel (shaders/kernels.metal:639-702),
// which src/metal_backend.mm:373-382 runs for every shape outside its flash paths: query i of
// head h at absolute position pos + i attends to cache rows 0..pos+i of KV head h / group, with
// the semantics of src/cpu_backend.cpp:51-69 (scores q.k * scale, softmax, weighted sum of V).
// The reference keeps all pos+i+1 scores in threadgroup memory; here a workgroup walks the keys
// in chunks of 256 with an online softmax (running max and sum, rescaled per chunk), so the
// context length is not bounded by LDS.
//
// Workgroup = one (query head, token), 256 threads. Per chunk: thread t scores key c0 + t (the
// dot product over head_dim in f32 from q staged in LDS and the f16 K row), the workgroup
// reduces the chunk's max and sum through LDS, and thread t then accumulates output dims
// t, t + 256, ... over the chunk's keys (consecutive threads read consecutive V elements).
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

// VPT: output dims per thread (head_dim <= 256 * VPT).
template <int VPT>
__global__ __launch_bounds__(kThreads) void attn_any_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ K, const _Float16* __restrict__ V,
    float* __restrict__ out, uint32_t pos, uint32_t n_head, uint32_t group, uint32_t hd, uint32_t kv_dim,
    uint32_t q_stride, float scale) {
    __shared__ float qs[kThreads * VPT];
    __shared__ float ps[kThreads];
    __shared__ float red[2][kWaves];

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t h = blockIdx.x % n_head, tok = blockIdx.x / n_head;
    const uint32_t n = pos + tok + 1;  // keys 0..pos+tok are visible
    const float* qh = q + size_t(tok) * q_stride + size_t(h) * hd;
    const _Float16* Kh = K + size_t(h / group) * hd;
    const _Float16* Vh = V + size_t(h / group) * hd;
    for (uint32_t i = tid; i < hd; i += kThreads) qs[i] = qh[i];
    __syncthreads();

    float m_run = kNoMax, l_run = 0.f;
    float o[VPT];
#pragma unroll
    for (int j = 0; j < VPT; j++) o[j] = 0.f;

    for (uint32_t c0 = 0; c0 < n; c0 += kThreads) {
        const uint32_t t = c0 + tid;
        float s = kNoMax;
        if (t < n) {
            const _Float16* kt = Kh + size_t(t) * kv_dim;
            float dot = 0.f;
            for (uint32_t i = 0; i < hd; i++) dot += qs[i] * float(kt[i]);
            s = dot * scale;
        }
        // chunk max
        float x = wave_max64(s);
        if (lane == 0) red[0][wave] = x;
        __syncthreads();
        float cmax = red[0][0];
#pragma unroll
        for (int w = 1; w < kWaves; w++) cmax = fmaxf(cmax, red[0][w]);
        const float m_new = fmaxf(m_run, cmax);
        const float alpha = expf(m_run - m_new);
        const float p = t < n ? expf(s - m_new) : 0.f;
        ps[tid] = p;
        x = wave_sum64(p);
        if (lane == 0) red[1][wave] = x;
        __syncthreads();
        float csum = red[1][0];
#pragma unroll
        for (int w = 1; w < kWaves; w++) csum += red[1][w];
        l_run = l_run * alpha + csum;
        m_run = m_new;
        const uint32_t nk = min(uint32_t(kThreads), n - c0);
#pragma unroll
        for (int j = 0; j < VPT; j++) {
            const uint32_t d = tid + kThreads * j;
            if (d < hd) {
                const _Float16* vt = Vh + size_t(c0) * kv_dim + d;
                float acc = o[j] * alpha;
                for (uint32_t k = 0; k < nk; k++) acc += ps[k] * float(vt[size_t(k) * kv_dim]);
                o[j] = acc;
            }
        }
        __syncthreads();  // ps and red are rewritten by the next chunk
    }
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    float* oh = out + size_t(tok) * q_stride + size_t(h) * hd;
#pragma unroll
    for (int j = 0; j < VPT; j++) {
        const uint32_t d = tid + kThreads * j;
        if (d < hd) oh[d] = o[j] * inv;
    }
}

}  // namespace

int launch_attn_any(const float* q, const _Float16* k, const _Float16* v, float* out, uint32_t pos,
                    uint32_t n_tok, uint32_t q_stride, uint32_t n_head, uint32_t n_head_kv, uint32_t head_dim,
                    float scale, hipStream_t stream) {
    const uint64_t blocks = uint64_t(n_head) * n_tok;
    if (blocks > 0x7fffffffu) return -1;
    const uint32_t group = n_head / n_head_kv, kv_dim = n_head_kv * head_dim;
    const dim3 grid{uint32_t(blocks)}, block{uint32_t(kThreads)};
    if (head_dim <= 256)
        hipLaunchKernelGGL(attn_any_kernel<1>, grid, block, 0, stream, q, k, v, out, pos, n_head, group, head_dim,
                           kv_dim, q_stride, scale);
    else if (head_dim <= 512)
        hipLaunchKernelGGL(attn_any_kernel<2>, grid, block, 0, stream, q, k, v, out, pos, n_head, group, head_dim,
                           kv_dim, q_stride, scale);
    else if (head_dim <= 1024)
        hipLaunchKernelGGL(attn_any_kernel<4>, grid, block, 0, stream, q, k, v, out, pos, n_head, group, head_dim,
                           kv_dim, q_stride, scale);
    else
        return -2;
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace ingot

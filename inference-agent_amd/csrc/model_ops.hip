// model_ops.hip — the small per-layer ops of the Llama forward pass around attention and the
// linear layers, for gfx950: RMS norm, SiLU-gate, and the embedding-row lookup.
//
// All three are HBM-bound elementwise/row work; each is one launch.
//   rmsnorm      out = x * (1/sqrt(mean(x^2) + eps)) * w per row (ops::rmsnorm, src/ops.cpp:226-231;
//                Metal rmsnorm, shaders/kernels.metal:230-252, encoded at src/metal_backend.mm:312-322)
//   silu_mul     gate = silu(gate) * up, silu(g) = g / (1 + exp(-g)) (src/ops.h:35,
//                src/cpu_backend.cpp:77; Metal silu_mul, shaders/kernels.metal:706-710)
//   get_rows     out[t] = dequantized row tokens[t] of the embedding table (ops::dequant_row,
//                src/ops.cpp:196-198, used at src/cpu_backend.cpp:33 and src/metal_backend.mm:428)
#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace {

// One workgroup per row; 256 threads, float4 per thread per iteration. out may alias x (each
// thread rewrites only the elements it read).
// One workgroup per row. Thread t sums the squares of the float4s at 4t, 4t + 1024, ... in that
// order, then the wave sums, then the four wave partials in fixed order (the fused projection
// prologue in linear.hip repeats exactly this order). Rows of up to kRowRegs * 1024 elements
// are held in registers with every load of x and w issued up front (a row of 3072: one round
// trip instead of three dependent ones).
constexpr int kRowRegs = 8;
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* x, const float* __restrict__ w,
                                                      float* out, uint32_t n, float eps) {
    __shared__ float part[4];
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + size_t(row) * n;
    float* orow = out + size_t(row) * n;
    float ss = 0.f;
    const bool held = n <= 1024u * kRowRegs;
    float4v xv[kRowRegs], wv[kRowRegs];
    if (held) {
#pragma unroll
        for (int k = 0; k < kRowRegs; k++) {
            const uint32_t i = 4 * tid + 1024 * k;
            if (i < n) {
                xv[k] = *reinterpret_cast<const float4v*>(xr + i);
                wv[k] = *reinterpret_cast<const float4v*>(w + i);
            }
        }
#pragma unroll
        for (int k = 0; k < kRowRegs; k++) {
            const uint32_t i = 4 * tid + 1024 * k;
            if (i < n) ss += xv[k][0] * xv[k][0] + xv[k][1] * xv[k][1] + xv[k][2] * xv[k][2] + xv[k][3] * xv[k][3];
        }
    } else {
        for (uint32_t i = 4 * tid; i < n; i += 1024) {
            const float4v v = *reinterpret_cast<const float4v*>(xr + i);
            ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
        }
    }
    ss = row16_sum(ss);
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    if (tid % 64 == 0) part[tid / 64] = ss;
    __syncthreads();
    const float total = (part[0] + part[1]) + (part[2] + part[3]);
    const float scale = 1.0f / sqrtf(total / float(n) + eps);
    if (held) {
#pragma unroll
        for (int k = 0; k < kRowRegs; k++) {
            const uint32_t i = 4 * tid + 1024 * k;
            if (i < n) *reinterpret_cast<float4v*>(orow + i) = xv[k] * scale * wv[k];
        }
    } else {
        for (uint32_t i = 4 * tid; i < n; i += 1024) {
            const float4v v = *reinterpret_cast<const float4v*>(xr + i);
            const float4v g = *reinterpret_cast<const float4v*>(w + i);
            *reinterpret_cast<float4v*>(orow + i) = v * scale * g;
        }
    }
}

__global__ __launch_bounds__(256) void silu_mul_kernel(float* __restrict__ gate,
                                                       const float* __restrict__ up, uint64_t n4) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n4) return;
    float4v g = reinterpret_cast<float4v*>(gate)[i];
    const float4v u = reinterpret_cast<const float4v*>(up)[i];
    for (int e = 0; e < 4; e++) g[e] = g[e] / (1.0f + expf(-g[e])) * u[e];
    reinterpret_cast<float4v*>(gate)[i] = g;
}

__device__ __forceinline__ float h2f(uint32_t h) { return float(__builtin_bit_cast(_Float16, uint16_t(h))); }
__device__ __forceinline__ uint32_t u16at(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// Element e of a row (the block formats of src/ops.cpp:33-87).
__device__ float deq1(uint32_t type, const uint8_t* row, uint32_t e) {
    switch (type) {
        case 0: return reinterpret_cast<const float*>(row)[e];
        case 1: return h2f(u16at(row + 2 * e));
        case 30: return __uint_as_float(u16at(row + 2 * e) << 16);
        case 8: {
            const uint8_t* b = row + 34 * (e / 32);
            return h2f(u16at(b)) * float(int8_t(b[2 + e % 32]));
        }
        case 2: {
            const uint8_t* b = row + 18 * (e / 32);
            const uint32_t i = e % 32, q = b[2 + i % 16];
            return h2f(u16at(b)) * float(int((i < 16 ? q : q >> 4) & 0xF) - 8);
        }
        case 3: {
            const uint8_t* b = row + 20 * (e / 32);
            const uint32_t i = e % 32, q = b[4 + i % 16];
            return h2f(u16at(b)) * float((i < 16 ? q : q >> 4) & 0xF) + h2f(u16at(b + 2));
        }
        case 14: {
            const uint8_t* b = row + 210 * (e / 256);
            const uint32_t r = e % 256, h = r / 128, g = (r % 128) / 32, l = r % 32;
            const uint32_t ql = b[h * 64 + l + 32 * (g & 1)], qh = b[128 + h * 32 + l];
            const int q = int(((g >= 2 ? ql >> 4 : ql) & 0xF) | (((qh >> (2 * g)) & 3) << 4)) - 32;
            return h2f(u16at(b + 208)) * float(int8_t(b[192 + h * 8 + l / 16 + 2 * g])) * float(q);
        }
        default: return 0.f;
    }
}

// One workgroup per token row. Ids outside [0, n_rows) give a zero row (the caller validates
// ids on the host first, as forward_batch does); they are never used as an address.
__global__ __launch_bounds__(256) void get_rows_kernel(uint32_t type, const uint8_t* __restrict__ w,
                                                       uint64_t row_bytes, uint32_t n, uint32_t n_rows,
                                                       const int32_t* __restrict__ tokens,
                                                       float* __restrict__ out) {
    const uint32_t t = blockIdx.x;
    const int32_t id = tokens[t];
    float* o = out + size_t(t) * n;
    if (id < 0 || uint32_t(id) >= n_rows) {
        for (uint32_t e = threadIdx.x; e < n; e += 256) o[e] = 0.f;
        return;
    }
    const uint8_t* row = w + uint64_t(id) * row_bytes;
    for (uint32_t e = threadIdx.x; e < n; e += 256) o[e] = deq1(type, row, e);
}

}  // namespace

int launch_rmsnorm(const float* x, const float* w, float* out, uint32_t n, uint32_t n_rows, float eps,
                   hipStream_t stream) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(n_rows), dim3(256), 0, stream, x, w, out, n, eps);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_silu_mul(float* gate, const float* up, uint64_t n, hipStream_t stream) {
    const uint64_t n4 = n / 4, blocks = (n4 + 255) / 256;
    if (blocks > 0x7fffffffu) return -1;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(uint32_t(blocks)), dim3(256), 0, stream, gate, up, n4);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_get_rows(uint32_t type, const void* w, uint64_t row_bytes, uint32_t n, uint32_t n_rows,
                    const int32_t* tokens, uint32_t n_tok, float* out, hipStream_t stream) {
    hipLaunchKernelGGL(get_rows_kernel, dim3(n_tok), dim3(256), 0, stream, type,
                       static_cast<const uint8_t*>(w), row_bytes, n, n_rows, tokens, out);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace ingot

// bw_probe.hip — streaming-read and copy probes used to calibrate the attention roofline.
// Measurement infrastructure (the counterpart of the reference's bw_sum/bwtest read probes,
// shaders/kernels.metal:951-957, src/main.cpp:449-455); not part of the attention ABI.
//
//   probe_read: each workgroup sums a contiguous chunk of `bytes` with 16-byte loads and writes
//               one float, so the kernel's HBM traffic is `bytes` read.
//   probe_copy: dst = src, 16-byte loads and stores (known FETCH_SIZE and WRITE_SIZE).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float float4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void probe_read(const float4v* __restrict__ src, size_t n4,
                                                  size_t per_block, float* __restrict__ sink) {
    const size_t b0 = size_t(blockIdx.x) * per_block;
    const size_t b1 = b0 + per_block < n4 ? b0 + per_block : n4;
    float4v acc = {0.f, 0.f, 0.f, 0.f};
    for (size_t i = b0 + threadIdx.x; i < b1; i += 256 * 4) {
        float4v x0 = src[i];
        float4v x1 = i + 256 < b1 ? src[i + 256] : float4v{};
        float4v x2 = i + 512 < b1 ? src[i + 512] : float4v{};
        float4v x3 = i + 768 < b1 ? src[i + 768] : float4v{};
        acc += (x0 + x1) + (x2 + x3);
    }
    float s = acc[0] + acc[1] + acc[2] + acc[3];
    if (s == 12345.678f) sink[blockIdx.x] = s;  // practically never: keeps the loads alive
}

__global__ __launch_bounds__(256) void probe_copy(const float4v* __restrict__ src,
                                                  float4v* __restrict__ dst, size_t n4) {
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n4; i += size_t(gridDim.x) * 256)
        dst[i] = src[i];
}

extern "C" int ingot_probe_read(const void* src, size_t bytes, uint32_t n_blocks, float* sink,
                                void* stream) {
    const size_t n4 = bytes / 16;
    const size_t per = (n4 + n_blocks - 1) / n_blocks;
    hipLaunchKernelGGL(probe_read, dim3(n_blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const float4v*>(src), n4, per, sink);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

extern "C" int ingot_probe_copy(const void* src, void* dst, size_t bytes, uint32_t n_blocks,
                                void* stream) {
    hipLaunchKernelGGL(probe_copy, dim3(n_blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const float4v*>(src), static_cast<float4v*>(dst), bytes / 16);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

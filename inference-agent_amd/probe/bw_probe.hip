// bw_probe.hip — streaming-read and copy probes used to calibrate the attention roofline.
// Measurement infrastructure (the counterpart of the reference's bw_sum/bwtest read probes,
// shaders/kernels.metal:951-957, src/main.cpp:449-455); not part of the attention ABI.
//
//   probe_read: each workgroup sums a contiguous chunk of `bytes` with 16-byte loads and writes
//               one float, so the kernel's HBM traffic is `bytes` read.
//   probe_copy: dst = src, 16-byte loads and stores (known FETCH_SIZE and WRITE_SIZE).
//   probe_mfma: back-to-back f16 MFMAs with no memory traffic (independent accumulator chains
//               per wave: 8 of 32x32x16 or 16 of 16x16x32), the achievable matrix-core rate that the
//               prefill kernels are measured against next to the 2.5 PFLOP/s spec figure.
//   probe_count / probe_handoff: the memory-order facts the decode kernels' split hand-off rests
//               on (decode_merge.h), checked across XCDs: a relaxed device-scope atomic counts
//               exactly whichever XCD each workgroup runs on, and a device-scope store, a wait
//               for its acknowledgement and a counter increment make the store visible to the
//               device-scope loads of the workgroup that counts last, wherever that one runs.
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

typedef _Float16 half8p __attribute__((ext_vector_type(8)));
typedef float float16p __attribute__((ext_vector_type(16)));

template <int SHAPE>  // 0: 32x32x16, 1: 16x16x32
__global__ __launch_bounds__(256) void probe_mfma(float* __restrict__ sink, int iters) {
    const half8p a = half8p{} + _Float16(0.001f * (threadIdx.x % 7));
    const half8p b = half8p{} + _Float16(0.002f * (threadIdx.x % 5));
    float s = 0.f;
    if constexpr (SHAPE == 0) {
        float16p acc[8];
        for (int c = 0; c < 8; c++) acc[c] = float16p{};
        for (int i = 0; i < iters; i++)
#pragma unroll
            for (int c = 0; c < 8; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
        for (int c = 0; c < 8; c++) s += acc[c][0];
    } else {
        float4v acc[16];
        for (int c = 0; c < 16; c++) acc[c] = float4v{};
        for (int i = 0; i < iters; i++)
#pragma unroll
            for (int c = 0; c < 16; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
        for (int c = 0; c < 16; c++) s += acc[c][0];
    }
    if (s == 12345.678f) sink[blockIdx.x] = s;  // practically never: keeps the chains alive
}

// FLOPs of one launch: blocks * 4 waves * iters * (8 * 32*32*16 or 16 * 16*16*32) * 2.
extern "C" int ingot_probe_mfma(int shape, uint32_t n_blocks, int iters, float* sink, void* stream) {
    if (shape == 0)
        hipLaunchKernelGGL(probe_mfma<0>, dim3(n_blocks), dim3(256), 0, static_cast<hipStream_t>(stream), sink, iters);
    else
        hipLaunchKernelGGL(probe_mfma<1>, dim3(n_blocks), dim3(256), 0, static_cast<hipStream_t>(stream), sink, iters);
    return hipGetLastError() == hipSuccess ? 0 : -4;
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

// Hardware id of the XCD (accelerator complex die) the wave runs on (gfx940+ HW_REG_XCC_ID).
__device__ __forceinline__ uint32_t xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15; }

__global__ __launch_bounds__(64) void probe_count(unsigned* __restrict__ ctr, unsigned* __restrict__ ret,
                                                  unsigned* __restrict__ xcc) {
    if (threadIdx.x != 0) return;
    ret[blockIdx.x] = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    xcc[blockIdx.x] = xcc_id();
}

typedef unsigned u32x4p __attribute__((ext_vector_type(4)));
constexpr int kProbeBufferFlags = 0x00020000;  // buffer descriptor word 3 (raw, 32-bit format)
constexpr int kProbeScDevice = 16;             // cache-policy bits: sc1 = device scope

// Workgroup b stores b + 1 into slot b (device scope), waits for the acknowledgement, counts
// itself in; the last one reads every slot with device-scope loads: res = {sum, slots that did
// not hold their value, the last one's XCD}.
__global__ __launch_bounds__(64) void probe_handoff(unsigned* __restrict__ ctr, unsigned* __restrict__ slot,
                                                    unsigned* __restrict__ res, unsigned n) {
    if (threadIdx.x != 0) return;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(slot, 0, int(n * 4), kProbeBufferFlags);
    __builtin_amdgcn_raw_buffer_store_b32(blockIdx.x + 1, rs, int(blockIdx.x * 4), 0, kProbeScDevice);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const unsigned p = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (p != n - 1) return;
    unsigned sum = 0, bad = 0;
    for (unsigned i = 0; i < n; i++) {
        const unsigned v = __builtin_amdgcn_raw_buffer_load_b32(rs, int(i * 4), 0, kProbeScDevice);
        sum += v;
        bad += v != i + 1;
    }
    res[0] = sum;
    res[1] = bad;
    res[2] = xcc_id();
}

extern "C" int ingot_probe_count(unsigned* ctr, unsigned* ret, unsigned* xcc, uint32_t n_blocks, void* stream) {
    hipLaunchKernelGGL(probe_count, dim3(n_blocks), dim3(64), 0, static_cast<hipStream_t>(stream), ctr, ret, xcc);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

extern "C" int ingot_probe_handoff(unsigned* ctr, unsigned* slot, unsigned* res, uint32_t n_blocks, void* stream) {
    hipLaunchKernelGGL(probe_handoff, dim3(n_blocks), dim3(64), 0, static_cast<hipStream_t>(stream), ctr, slot, res,
                       n_blocks);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
